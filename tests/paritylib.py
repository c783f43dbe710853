"""Helpers shared by the parity tests: golden record comparison and model
construction from the random-init writer."""
from __future__ import annotations

import hashlib

import numpy as np

from conftest import bits_equal, describe_diff, golden

BIG_F32 = ("q", "k", "v", "attn", "o", "g", "u", "sw")
INT_STAGES = ("h8", "q8", "o8", "s8", "kc", "vc")
STAGES = ("h", "h8", "hs", "q", "k", "v", "q8", "qs", "kc", "ks", "vc", "vs", "attn", "o8", "os",
          "o", "g", "u", "sw", "s8", "ss", "x")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def golden_stage(g, prefix: str, name: str):
    """Returns ('full', array) or ('sha', (sha, last_row, shape)) or None."""
    if f"{prefix}{name}" in g.files:
        return "full", g[f"{prefix}{name}"]
    if f"{prefix}{name}_sha" in g.files:
        return "sha", (str(g[f"{prefix}{name}_sha"]), g[f"{prefix}{name}_last"],
                       tuple(g[f"{prefix}{name}_shape"]))
    return None


def compare_stage(g, prefix: str, name: str, got: np.ndarray, rows: slice | None = None) -> str | None:
    """None if equal (bit-exact), else a description.  `rows` restricts a
    full-array comparison to some rows (used where a path only writes the
    last row)."""
    spec = golden_stage(g, prefix, name)
    if spec is None:
        return f"{prefix}{name}: no golden"
    kind, val = spec
    got = np.ascontiguousarray(got)
    if kind == "full":
        exp = val if rows is None else val[rows]
        g2 = got if rows is None else got[rows]
        if not bits_equal(g2, exp):
            return f"{prefix}{name}: {describe_diff(g2, exp)}"
        return None
    digest, last, shape = val
    if rows is not None:
        if not bits_equal(got[-1:], last):
            return f"{prefix}{name}[last]: {describe_diff(got[-1:], last)}"
        return None
    if tuple(got.shape) != shape:
        return f"{prefix}{name}: shape {got.shape} != {shape}"
    if sha(got) != digest:
        if not bits_equal(got[-1:], last):
            return f"{prefix}{name}: sha differs; last row {describe_diff(got[-1:], last)}"
        return f"{prefix}{name}: sha differs (last row equal)"
    return None


def load_cfg(name: str):
    return golden(f"{name}.npz")
