"""Blob layout (tools/pqwf.py:95-273) and the random-init model image.

`Layout` wraps q3_layout_compute; `init_random_blob` wraps
q3_init_random_blob.  Both run on the host only.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import CLayout, InitParams, LAYOUT_DIMS, LAYOUT_OFFSETS, check, lib


@dataclass(frozen=True)
class ModelShape:
    hidden: int = 1024
    layers: int = 28
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    inter: int = 3072
    vocab: int = 151936
    seq: int = 32
    max_seq: int = 256


class Layout:
    """tools/pqwf.py Layout: shape fields plus every blob byte offset."""

    def __init__(self, shape: ModelShape | None = None, **kw):
        shape = shape or ModelShape(**kw)
        self.shape = shape
        self.c = CLayout()
        check(lib().q3_layout_compute(shape.hidden, shape.layers, shape.heads, shape.kv_heads,
                                      shape.head_dim, shape.inter, shape.vocab, shape.seq,
                                      shape.max_seq, C.byref(self.c)), "q3_layout_compute")
        self.offsets = {n: int(getattr(self.c, n)) for n in LAYOUT_OFFSETS}
        for n in LAYOUT_DIMS:
            setattr(self, n, int(getattr(self.c, n)))

    def __getitem__(self, name: str) -> int:
        return self.offsets[name]

    @property
    def size(self) -> int:
        return self.offsets["kSCRATCH_END"]

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim

    def header_text(self) -> str:
        n = lib().q3_layout_header_text(C.byref(self.c), None, 0)
        buf = C.create_string_buffer(n + 1)
        lib().q3_layout_header_text(C.byref(self.c), buf, n + 1)
        return buf.value.decode()

    # -- typed host views on a blob (numpy uint8 array) ---------------------
    def weight_views(self, blob: np.ndarray, layer: int) -> dict[str, np.ndarray]:
        o, H, HD, I = self.offsets, self.hidden, self.head_dim, self.inter
        QW, KW = self.q_width, self.kv_width
        w = layer * o["kLAYERW_STRIDE"]
        n = layer * o["kLAYERN_STRIDE"]

        def i8(off, r, c):
            return blob[off:off + r * c].view(np.int8).reshape(r, c)

        def f32(off, cnt):
            return blob[off:off + 4 * cnt].view(np.float32)

        return dict(
            wq=i8(o["kLQ"] + w, QW, H), wq_s=f32(o["kLQ_SCALE"] + w, QW),
            wk=i8(o["kLK"] + w, KW, H), wk_s=f32(o["kLK_SCALE"] + w, KW),
            wv=i8(o["kLV"] + w, KW, H), wv_s=f32(o["kLV_SCALE"] + w, KW),
            wo=i8(o["kLO"] + w, H, QW), wo_s=f32(o["kLO_SCALE"] + w, H),
            wg=i8(o["kLG"] + w, I, H), wg_s=f32(o["kLG_SCALE"] + w, I),
            wu=i8(o["kLU"] + w, I, H), wu_s=f32(o["kLU_SCALE"] + w, I),
            wd=i8(o["kLD"] + w, H, I), wd_s=f32(o["kLD_SCALE"] + w, H),
            n1=f32(o["kN1"] + n, H), nq=f32(o["kNQ"] + n, HD),
            nk=f32(o["kNK"] + n, HD), n2=f32(o["kN2"] + n, H),
        )

    def global_views(self, blob: np.ndarray) -> dict[str, np.ndarray]:
        o, H, V, MS, HALF = self.offsets, self.hidden, self.vocab, self.max_seq, self.half
        return dict(
            ids=blob[o["kIDS"]:o["kIDS"] + 4 * MS].view(np.int32),
            ctrl=blob[o["kCTRL"]:o["kCTRL"] + 16].view(np.int32),
            emb8=blob[o["kEMB"]:o["kEMB"] + V * H].view(np.int8).reshape(V, H),
            emb_s=blob[o["kEMB"] + V * H:o["kEMB"] + V * H + 4 * V].view(np.float32),
            lm8=blob[o["kLM"]:o["kLM"] + V * H].view(np.int8).reshape(V, H),
            lm_s=blob[o["kLM"] + V * H:o["kLM"] + V * H + 4 * V].view(np.float32),
            nf=blob[o["kNF"]:o["kNF"] + 4 * H].view(np.float32),
            cos=blob[o["kCOS"]:o["kCOS"] + 4 * MS * HALF].view(np.float32).reshape(MS, HALF),
            sin=blob[o["kSIN"]:o["kSIN"] + 4 * MS * HALF].view(np.float32).reshape(MS, HALF),
        )


@dataclass(frozen=True)
class InitConfig:
    """Deterministic random-init model (the offline stand-in for the HF
    checkpoint that tools/convert_pqwf.py quantises)."""
    weight_seed: int = 0x5EED0000
    ids_seed: int = 0x5EED0001
    weight_std: float = 0.02
    gain_std: float = 0.05
    rope_theta: float = 1e6
    n_prompt: int = 40
    n_gen: int = 2
    mode: int = 0


def init_random_blob(layout: Layout, cfg: InitConfig, threads: int = 0,
                     out: np.ndarray | None = None) -> np.ndarray:
    """Host uint8 array of layout.size bytes holding the random-init model."""
    if out is None:
        out = np.empty(layout.size, dtype=np.uint8)
    assert out.dtype == np.uint8 and out.size >= layout.size and out.flags.c_contiguous
    p = InitParams(cfg.weight_seed, cfg.ids_seed, cfg.weight_std, cfg.gain_std, cfg.rope_theta,
                   cfg.n_prompt, cfg.n_gen, cfg.mode)
    check(lib().q3_init_random_blob(C.byref(layout.c), C.byref(p),
                                    out.ctypes.data_as(C.c_void_p), threads),
          "q3_init_random_blob")
    return out


def init_normal(seed: int, stream: int, first: int, n: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(lib().q3_init_normal(seed, stream, first, n, mean, std,
                               out.ctypes.data_as(C.c_void_p)), "q3_init_normal")
    return out


def stream_id(layer: int, which: int) -> int:
    return int(lib().q3_init_stream_id(layer, which))


def quantize_rows_host(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty(rows, dtype=np.float32)
    check(lib().q3_quantize_rows_host(w.ctypes.data_as(C.c_void_p), rows, cols,
                                      q.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p)),
          "q3_quantize_rows_host")
    return q, s


# BASELINE configurations (shape + init) used by tests and the benchmark.
CONFIGS = {
    # config 0: 1 layer, 1024 vocab, 40-token prompt as 32+8, 2 greedy tokens
    "cfg0": (ModelShape(layers=1, vocab=1024, seq=32, max_seq=256),
             InitConfig(n_prompt=40, n_gen=2, mode=0)),
    # config 2: full depth, one 32-token prefill with full logits
    "cfg2": (ModelShape(seq=32, max_seq=256), InitConfig(n_prompt=32, n_gen=0, mode=1)),
    # config 3 (parity): 15-token prompt, 6 greedy tokens, fused argmax
    "cfg3": (ModelShape(seq=32, max_seq=256), InitConfig(n_prompt=15, n_gen=6, mode=0)),
    # config 3 (perf): one 512-token prefill chunk then 64 greedy decode steps
    "cfg3_perf": (ModelShape(seq=512, max_seq=640), InitConfig(n_prompt=512, n_gen=64, mode=0)),
}
