"""PQWF converter: a Hugging Face Qwen3 checkpoint directory (config.json +
model.safetensors, BF16/F16/F32 tensors) into the device blob.

Follows tools/convert_pqwf.py:125-220 and tools/pqwf.py:279-360:

- the layout comes from the checkpoint's config (optionally fewer layers or
  vocabulary rows) plus ``seq`` / ``max_seq``;
- every projection, the embedding and the lm_head (the embedding when the
  checkpoint ties them, convert_pqwf.py:186) are quantised per output row
  to int8 with an f32 scale: absmax * f32(1/127), quotient rounded half to
  even, NaN -> 0, clipped to +-127 (pqwf.py:344-360; ``q3_quantize_rows_host``
  computes exactly that);
- norms are stored as f32, RoPE tables as f32(cos / sin) of f64 angles
  ``pos / theta^(i / half)`` (convert_pqwf.py:46-52);
- ids default to ``100 + 10 i`` (convert_pqwf.py:37-43) and CTRL holds
  ``[n_prompt, n_gen, max_seq, 0]``.

Tensors are read a block of rows at a time through ``safetensors`` (no full
copy of the checkpoint in memory); the blob is a numpy array or, with
``out``, a file-backed memmap ready for ``q3ops.model.Model``.
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

import numpy as np

from .layout import Layout, ModelShape, quantize_rows_host

__all__ = ["rope_tables", "parse_ids", "Checkpoint", "convert", "main"]

# HF projection name -> (module, blob view key); pqwf.py's per-layer order
PROJECTIONS = (("q_proj", "self_attn", "wq"), ("k_proj", "self_attn", "wk"),
               ("v_proj", "self_attn", "wv"), ("o_proj", "self_attn", "wo"),
               ("gate_proj", "mlp", "wg"), ("up_proj", "mlp", "wu"),
               ("down_proj", "mlp", "wd"))
NORMS = (("input_layernorm", "n1"), ("self_attn.q_norm", "nq"),
         ("self_attn.k_norm", "nk"), ("post_attention_layernorm", "n2"))


def rope_tables(max_seq: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """[max_seq][head_dim / 2] f32 cos and sin tables (convert_pqwf.py:46-52)."""
    half = head_dim // 2
    inv_freq = 1.0 / (float(theta) ** (np.arange(half, dtype=np.float64) / float(half)))
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def parse_ids(text: str, n: int) -> list[int]:
    """Comma-separated ids, else 100 + 10 i; padded with 0 / cut to n
    (convert_pqwf.py:37-43)."""
    ids = [int(t) for t in text.split(",") if t.strip()] if text else []
    if not ids:
        ids = [100 + 10 * i for i in range(n)]
    return (ids + [0] * n)[:n]


class Checkpoint:
    """Row blocks of a safetensors file as f32 numpy arrays."""

    def __init__(self, path: str | Path):
        from safetensors import safe_open
        self._f = safe_open(str(path), framework="pt")
        self._names = set(self._f.keys())

    def __contains__(self, name: str) -> bool:
        return name in self._names

    def shape(self, name: str) -> tuple:
        return tuple(self._f.get_slice(name).get_shape())

    def rows_f32(self, name: str, r0: int, r1: int) -> np.ndarray:
        import torch
        t = self._f.get_slice(name)[r0:r1]
        return t.to(torch.float32).numpy()

    def vector_f32(self, name: str) -> np.ndarray:
        import torch
        return self._f.get_tensor(name).to(torch.float32).numpy().reshape(-1)


def _quantize_into(ck: Checkpoint, name: str, q: np.ndarray, s: np.ndarray,
                   chunk: int = 2048) -> None:
    rows, cols = q.shape
    have = ck.shape(name)
    if len(have) != 2 or have[1] != cols or have[0] < rows:
        raise ValueError(f"{name}: checkpoint shape {have}, blob needs [{rows}][{cols}]")
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        q[r0:r1], s[r0:r1] = quantize_rows_host(ck.rows_f32(name, r0, r1))


def convert(model_dir: str | Path, *, layers: int = 0, vocab: int = 0, seq: int = 32,
            max_seq: int = 256, n_prompt: int = 32, n_gen: int = 0, ids: str = "",
            out: str | Path | None = None, log=None) -> tuple[Layout, np.ndarray]:
    """Returns (layout, blob bytes); with ``out`` the blob is that file."""
    model_dir = Path(model_dir)
    cfg = json.loads((model_dir / "config.json").read_text())
    shape = ModelShape(hidden=int(cfg["hidden_size"]),
                       layers=int(layers or cfg["num_hidden_layers"]),
                       heads=int(cfg["num_attention_heads"]),
                       kv_heads=int(cfg["num_key_value_heads"]),
                       head_dim=int(cfg["head_dim"]), inter=int(cfg["intermediate_size"]),
                       vocab=int(vocab or cfg["vocab_size"]), seq=seq, max_seq=max_seq)
    if n_prompt + n_gen > max_seq:
        raise ValueError(f"n_prompt + n_gen = {n_prompt + n_gen} > max_seq {max_seq}")
    lay = Layout(shape)
    if out is None:
        blob = np.zeros(lay.size, np.uint8)
    else:
        Path(out).parent.mkdir(parents=True, exist_ok=True)
        blob = np.memmap(out, dtype=np.uint8, mode="w+", shape=(lay.size,))
    ck = Checkpoint(model_dir / "model.safetensors")
    g = lay.global_views(blob)
    n = n_prompt + n_gen
    g["ids"][:n] = parse_ids(ids, n)
    g["ctrl"][:] = [n_prompt, n_gen, max_seq, 0]
    g["nf"][:] = ck.vector_f32("model.norm.weight")
    g["cos"][:], g["sin"][:] = rope_tables(max_seq, shape.head_dim,
                                           float(cfg.get("rope_theta", 1e6)))
    if log:
        log("embedding / lm_head ...")
    _quantize_into(ck, "model.embed_tokens.weight", g["emb8"], g["emb_s"])
    lm = "lm_head.weight" if "lm_head.weight" in ck else "model.embed_tokens.weight"
    _quantize_into(ck, lm, g["lm8"], g["lm_s"])
    for li in range(shape.layers):
        w = lay.weight_views(blob, li)
        pre = f"model.layers.{li}."
        for proj, module, key in PROJECTIONS:
            _quantize_into(ck, f"{pre}{module}.{proj}.weight", w[key], w[key + "_s"])
        for hf, key in NORMS:
            w[key][:] = ck.vector_f32(f"{pre}{hf}.weight")
        if log and (li + 1) % 4 == 0:
            log(f"  {li + 1}/{shape.layers} layers")
    if isinstance(blob, np.memmap):
        blob.flush()
    return lay, blob


def main(argv=None) -> int:
    """Command line of tools/convert_pqwf.py (its numpy reference run aside)."""
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--model-dir", required=True)
    ap.add_argument("--layers", type=int, default=0, help="number of layers (0 = all)")
    ap.add_argument("--vocab", type=int, default=0, help="vocab rows to keep (0 = all)")
    ap.add_argument("--seq", type=int, default=32)
    ap.add_argument("--max-seq", type=int, default=256)
    ap.add_argument("--n-prompt", type=int, default=32)
    ap.add_argument("--n-gen", type=int, default=0)
    ap.add_argument("--ids", default="")
    ap.add_argument("--header", default="build/model_big.h")
    ap.add_argument("--blob", default="build/qwen3_big_data.bin")
    a = ap.parse_args(argv)
    lay, _ = convert(a.model_dir, layers=a.layers, vocab=a.vocab, seq=a.seq, max_seq=a.max_seq,
                     n_prompt=a.n_prompt, n_gen=a.n_gen, ids=a.ids, out=a.blob,
                     log=lambda m: print(m, flush=True))
    Path(a.header).parent.mkdir(parents=True, exist_ok=True)
    Path(a.header).write_text(lay.header_text())
    print(f"blob:   {a.blob} ({lay.size} bytes)\nheader: {a.header}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
