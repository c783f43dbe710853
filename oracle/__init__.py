"""CPU oracle: ctypes front end of oracle/liboracle.so, the C restatement of
the reference's numpy mirror tools/ref_qwen3.py.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker (or as the timed CPU baseline); the product path never calls it.

Every wrapper names the reference function it follows.  Model-level entry
points take the host blob plus its layout offsets (a dict with the
tools/pqwf.py names), so the oracle reads weights exactly like
tools/convert_pqwf.py:76-122 reference_model does.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)


class OrcLayer(C.Structure):
    _fields_ = ([(n, _i8p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")]
                + [(n, _f32p) for n in ("wq_s", "wk_s", "wv_s", "wo_s", "wg_s", "wu_s", "wd_s")]
                + [(n, _f32p) for n in ("n1", "nq", "nk", "n2")])


class OrcModel(C.Structure):
    _fields_ = ([(n, C.c_int) for n in ("hidden", "heads", "kv_heads", "head_dim", "inter",
                                        "vocab", "seq", "max_seq", "n_layers")]
                + [("layers", C.POINTER(OrcLayer)), ("emb8", _i8p), ("emb_s", _f32p),
                   ("lm8", _i8p), ("lm_s", _f32p), ("nf", _f32p), ("cos_t", _f32p),
                   ("sin_t", _f32p)])


class OrcCache(C.Structure):
    _fields_ = [("k8", _i8p), ("k_s", _f32p), ("v8", _i8p), ("v_s", _f32p)]


REC_FIELDS = [("h", np.float32, "H"), ("h8", np.int8, "H"), ("hs", np.float32, "H256"),
              ("q", np.float32, "QW"), ("k", np.float32, "KW"), ("v", np.float32, "KW"),
              ("q8", np.int8, "QW"), ("qs", np.float32, "NH"), ("attn", np.float32, "QW"),
              ("o8", np.int8, "QW"), ("os", np.float32, "NH"), ("o", np.float32, "H"),
              ("g", np.float32, "I"), ("u", np.float32, "I"), ("sw", np.float32, "I"),
              ("s8", np.int8, "I"), ("ss", np.float32, "I256"), ("x", np.float32, "H")]


class OrcRecord(C.Structure):
    _fields_ = ([(name, _i8p if dt == np.int8 else _f32p) for name, dt, _ in REC_FIELDS]
                + [("rows_written", C.c_int32)])


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB_PATH))
        L.orc_exp2f.restype = C.c_float
        L.orc_exp2f.argtypes = [C.c_float]
        L.orc_exp_f32.restype = C.c_float
        L.orc_exp_f32.argtypes = [C.c_float]
        L.orc_tree_sum.restype = C.c_float
        L.orc_tree_max.restype = C.c_float
        L.orc_forward_chunk.restype = C.c_int
        L.orc_generate.restype = C.c_int
        L.orc_argmax_logits.restype = C.c_int
        L.orc_get_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, t=C.c_void_p):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(t)


def set_threads(n: int) -> None:
    lib().orc_set_threads(C.c_int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


# ---- primitives (ref_qwen3.py:27-296) -------------------------------------
def exp_f32(x: np.ndarray) -> np.ndarray:
    """ref_qwen3.py:27-29."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_exp_f32_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def exp2f(x: float) -> float:
    return float(lib().orc_exp2f(C.c_float(x)))


def tree_sum(v: np.ndarray) -> np.float32:
    """ref_qwen3.py:53-54 (one row)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return np.float32(lib().orc_tree_sum(_p(v), C.c_int(v.size)))


def tree_max(v: np.ndarray) -> np.float32:
    """ref_qwen3.py:57-58 (one row)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return np.float32(lib().orc_tree_max(_p(v), C.c_int(v.size)))


def quant_rows_heads(x: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    """ref_qwen3.py:86-97."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // group), np.float32)
    lib().orc_quant_rows_heads(_p(x), rows, cols, group, _p(q), _p(s))
    return q, s


def gemm_nt_group(a8, a_scale, w8, w_scale, group: int) -> np.ndarray:
    """ref_qwen3.py:145-158."""
    a8 = np.ascontiguousarray(a8, np.int8)
    w8 = np.ascontiguousarray(w8, np.int8)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    w_scale = np.ascontiguousarray(w_scale, np.float32)
    rows, k = a8.shape
    n = w8.shape[0]
    out = np.empty((rows, n), np.float32)
    lib().orc_gemm_nt_group(_p(a8), _p(a_scale), rows, k, _p(w8), _p(w_scale), n, group, _p(out))
    return out


def gemm_nt_group_bg(a8, a_scale, w8, w_scale, group: int) -> np.ndarray:
    """ref_qwen3.py:145-158 with per-(row, group) weight scales
    w_scale [n][k // group] (not a reference function)."""
    a8 = np.ascontiguousarray(a8, np.int8)
    w8 = np.ascontiguousarray(w8, np.int8)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    w_scale = np.ascontiguousarray(w_scale, np.float32)
    rows, k = a8.shape
    n = w8.shape[0]
    assert w_scale.shape == (n, k // group), w_scale.shape
    out = np.empty((rows, n), np.float32)
    lib().orc_gemm_nt_group_bg(_p(a8), _p(a_scale), rows, k, _p(w8), _p(w_scale), n, group,
                               _p(out))
    return out


def gemm_nt_group_i32(a8, w8, group: int) -> np.ndarray:
    """Per-group exact int32 partials, [rows][groups][n]."""
    a8 = np.ascontiguousarray(a8, np.int8)
    w8 = np.ascontiguousarray(w8, np.int8)
    rows, k = a8.shape
    n = w8.shape[0]
    out = np.empty((rows, k // group, n), np.int32)
    lib().orc_gemm_nt_group_i32(_p(a8), rows, k, _p(w8), n, group, _p(out))
    return out


def rmsnorm_rows(x: np.ndarray, w: np.ndarray, inv: float) -> np.ndarray:
    """ref_qwen3.py:161-177."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm_rows(_p(x), rows, cols, cols, _p(w), C.c_float(inv), _p(out), cols)
    return out


def rope_head_hd(x, cos_t, sin_t) -> np.ndarray:
    """ref_qwen3.py:180-191."""
    x = np.ascontiguousarray(x, np.float32)
    cos_t = np.ascontiguousarray(cos_t, np.float32)
    sin_t = np.ascontiguousarray(sin_t, np.float32)
    rows, hd = x.shape
    out = np.empty_like(x)
    lib().orc_rope_head_hd(_p(x), rows, hd, hd, _p(cos_t), _p(sin_t), _p(out), hd)
    return out


def swiglu(gate, up) -> np.ndarray:
    """ref_qwen3.py:194-200."""
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.empty_like(gate)
    lib().orc_swiglu(_p(gate), _p(up), C.c_size_t(gate.size), _p(out))
    return out


def attention_heads_gqa_tokscale(q8, q_scale, k8, k_scale, v8, v_scale, heads: int,
                                 kv_heads: int, hd: int, causal: bool,
                                 qk_scale: float) -> np.ndarray:
    """ref_qwen3.py:269-289 (contiguous cache rows [kv_len][kv_heads*hd])."""
    q8 = np.ascontiguousarray(q8, np.int8)
    k8 = np.ascontiguousarray(k8, np.int8)
    v8 = np.ascontiguousarray(v8, np.int8)
    q_scale = np.ascontiguousarray(q_scale, np.float32)
    k_scale = np.ascontiguousarray(k_scale, np.float32)
    v_scale = np.ascontiguousarray(v_scale, np.float32)
    rows = q8.shape[0]
    kv_len = k8.shape[0]
    out = np.empty((rows, heads * hd), np.float32)
    lib().orc_attention_heads_gqa_tokscale(_p(q8), _p(q_scale), rows, _p(k8), _p(k_scale), _p(v8),
                                           _p(v_scale), kv_len, heads, kv_heads, hd,
                                           int(bool(causal)), C.c_float(qk_scale), _p(out))
    return out


def embedding_rmsnorm(emb8, emb_s, ids, w, inv: float) -> tuple[np.ndarray, np.ndarray]:
    """ref_qwen3.py:292-296: returns (h, x)."""
    emb8 = np.ascontiguousarray(emb8, np.int8)
    emb_s = np.ascontiguousarray(emb_s, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    hidden = emb8.shape[1]
    rows = ids.size
    h = np.empty((rows, hidden), np.float32)
    x = np.empty((rows, hidden), np.float32)
    lib().orc_embedding_rmsnorm(_p(emb8), _p(emb_s), hidden, _p(ids), rows, _p(w),
                                C.c_float(inv), _p(h), _p(x))
    return h, x


def argmax_logits(logits: np.ndarray) -> int:
    """ref_qwen3.py:447-464."""
    logits = np.ascontiguousarray(logits, np.float32).reshape(-1)
    return int(lib().orc_argmax_logits(_p(logits), logits.size))


# ---- model (ref_qwen3.py:302-490) -----------------------------------------
class OracleModel:
    """ref_qwen3.Model over a host blob (keeps the blob alive)."""

    def __init__(self, blob: np.ndarray, offsets: dict, dims: dict):
        self.blob = blob
        o = offsets
        H, HD, I, V = dims["hidden"], dims["head_dim"], dims["inter"], dims["vocab"]
        QW, KW = dims["heads"] * HD, dims["kv_heads"] * HD
        self.dims = dict(dims)
        L = dims["layers"]
        base = blob.ctypes.data

        def pi8(off):
            return C.cast(C.c_void_p(base + off), _i8p)

        def pf(off):
            return C.cast(C.c_void_p(base + off), _f32p)

        self._layers = (OrcLayer * L)()
        for li in range(L):
            w = li * o["kLAYERW_STRIDE"]
            n = li * o["kLAYERN_STRIDE"]
            ly = self._layers[li]
            for nm, key in (("wq", "kLQ"), ("wk", "kLK"), ("wv", "kLV"), ("wo", "kLO"),
                            ("wg", "kLG"), ("wu", "kLU"), ("wd", "kLD")):
                setattr(ly, nm, pi8(o[key] + w))
                setattr(ly, nm + "_s", pf(o[key + "_SCALE"] + w))
            ly.n1, ly.nq, ly.nk, ly.n2 = (pf(o["kN1"] + n), pf(o["kNQ"] + n), pf(o["kNK"] + n),
                                          pf(o["kN2"] + n))
        self.c = OrcModel(H, dims["heads"], dims["kv_heads"], HD, I, V, dims["seq"],
                          dims["max_seq"], L, self._layers, pi8(o["kEMB"]),
                          pf(o["kEMB"] + V * H), pi8(o["kLM"]), pf(o["kLM"] + V * H),
                          pf(o["kNF"]), pf(o["kCOS"]), pf(o["kSIN"]))
        MS = dims["max_seq"]
        self.k8 = np.zeros((L, MS, KW), np.int8)
        self.v8 = np.zeros((L, MS, KW), np.int8)
        self.k_s = np.zeros((L, MS, dims["kv_heads"]), np.float32)
        self.v_s = np.zeros((L, MS, dims["kv_heads"]), np.float32)
        self._caches = (OrcCache * L)()
        for li in range(L):
            self._caches[li] = OrcCache(self.k8[li].ctypes.data_as(_i8p),
                                        self.k_s[li].ctypes.data_as(_f32p),
                                        self.v8[li].ctypes.data_as(_i8p),
                                        self.v_s[li].ctypes.data_as(_f32p))
        self._widths = dict(H=H, H256=H // 256, QW=QW, KW=KW, NH=dims["heads"], I=I,
                            I256=I // 256)

    def new_record(self, rows: int) -> tuple[OrcRecord, dict]:
        bufs = {name: np.zeros((rows, self._widths[w]), dt) for name, dt, w in REC_FIELDS}
        rec = OrcRecord(*[bufs[name].ctypes.data_as(_i8p if dt == np.int8 else _f32p)
                          for name, dt, _ in REC_FIELDS], 0)
        return rec, bufs

    def reset_cache(self) -> None:
        for a in (self.k8, self.v8, self.k_s, self.v_s):
            a[...] = 0

    def forward_chunk(self, ids: np.ndarray, pos: int, rows: int, want_logits: bool,
                      record: bool = False):
        """ref_qwen3.py:366-444 (the caches persist across calls)."""
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.zeros(self.dims["vocab"], np.float32)
        rec, bufs = self.new_record(rows) if record else (None, None)
        rc = lib().orc_forward_chunk(C.byref(self.c), _p(ids), self._caches, pos, rows,
                                     int(want_logits), C.byref(rec) if rec else None, _p(logits))
        if rc != 0:
            raise RuntimeError(f"orc_forward_chunk failed ({rc})")
        return (logits if want_logits else None), bufs

    def generate(self, ids: np.ndarray, n_prompt: int, n_gen: int, record: bool = True):
        """ref_qwen3.py:467-490: returns (last_logits, generated, record, ids)."""
        total = n_prompt + n_gen
        ids = np.ascontiguousarray(np.asarray(ids, np.int32)[:total].copy())
        if ids.size < total:
            ids = np.concatenate([ids, np.zeros(total - ids.size, np.int32)])
        logits = np.zeros(self.dims["vocab"], np.float32)
        gen = np.zeros(max(n_gen, 1), np.int32)
        rec, bufs = self.new_record(self.dims["seq"]) if record else (None, None)
        rc = lib().orc_generate(C.byref(self.c), _p(ids), n_prompt, n_gen, self._caches,
                                C.byref(rec) if rec else None, _p(logits), _p(gen))
        if rc < 0:
            raise RuntimeError(f"orc_generate failed ({rc})")
        if bufs is not None:
            bufs = {k: v[:rec.rows_written] for k, v in bufs.items()}
        return logits, gen[:n_gen], bufs, ids
