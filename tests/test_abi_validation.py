"""Host-side argument validation of the C ABI, without a GPU.

Every case here must be rejected before anything is launched: an undersized
output or scale view has to come back as Q3_ERR_VIEW (a kernel would
otherwise write past it on the device), a degenerate layout as
Q3_ERR_UNSUPPORTED, and the row limit of the argmax ops through the
reference's silent-unsupported switch.  The data pointers are host
addresses that are never dereferenced.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from q3ops import _lib
from q3ops.layout import Layout, ModelShape

OK, ERR_VIEW, ERR_UNSUPPORTED = 0, -3, -4
DT_I8, DT_I32, DT_F32 = _lib.DT_I8, _lib.DT_I32, _lib.DT_F32
_ARENA = np.zeros(1 << 16, np.uint8)  # a 16-byte aligned, never-read address
_ADDR = (_ARENA.ctypes.data + 255) & ~255


def V(rows, cols, dt, row_bytes=None, col_bytes=None):
    es = 1 if dt == DT_I8 else 4
    rb = cols * es if row_bytes is None else row_bytes
    cb = es if col_bytes is None else col_bytes
    return C.byref(_lib.View(_ADDR, rb, cb, rows, cols, dt))


def gemm_operands(M, K, N, group=256):
    return (V(M, K, DT_I8), V(M, K // group, DT_F32), V(N, K, DT_I8), V(N, 1, DT_F32))


def paged(row_bytes=1024, scale_row_bytes=32):
    return _lib.PagedKV(_ADDR, _ADDR, _ADDR, _ADDR, _ADDR, 32, 32 * row_bytes, row_bytes,
                        32 * scale_row_bytes, scale_row_bytes)


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def test_head_quant_epilogue_scale_shape(lib):
    M, K, N = 8, 1024, 1024
    a, as_, b, bs = gemm_operands(M, K, N)
    q8 = V(M, N, DT_I8)
    for qs in (V(M - 1, N // 128, DT_F32),        # too few rows
               V(M, N // 128 - 1, DT_F32),        # too few heads
               V(M, N // 128, DT_F32, col_bytes=0),
               V(M, N // 128, DT_F32, row_bytes=16, col_bytes=8)):  # rows overlap
        assert lib.q3_gemm_nt_group_store(a, as_, b, bs, None, 256, None, q8, qs, None, None,
                                          None, C.c_float(0), None) == ERR_VIEW


def test_attention_scale_shapes(lib):
    rows, heads, kvh = 4, 16, 8
    kv = paged()
    q8, o8 = V(rows, heads * 128, DT_I8), V(rows, heads * 128, DT_I8)
    good = V(rows, heads, DT_F32)
    for qsc, osc in ((V(rows - 1, heads, DT_F32), good), (V(rows, heads - 1, DT_F32), good),
                     (good, V(rows - 1, heads, DT_F32)), (good, V(rows, heads - 2, DT_F32))):
        assert lib.q3_attention_heads_gqa_tokscale_paged(q8, qsc, C.byref(kv), 64, o8, osc, heads,
                                                         kvh, 128, 1, C.c_float(0.088),
                                                         None) == ERR_VIEW


def test_kv_paged_scale_row_bytes(lib):
    M, K, N = 8, 1024, 1024
    a, as_, b, bs = gemm_operands(M, K, N)
    kv = paged(scale_row_bytes=16)  # 4 heads' scales for an 8-head projection
    assert lib.q3_gemm_nt_group_kv_paged(a, as_, b, bs, 256, C.byref(kv), 0, 1, None, None,
                                         None, C.c_float(0), None) == ERR_VIEW


def test_norm_rope_quant_scale_shape(lib):
    x, q8 = V(6, 1024, DT_F32), V(6, 1024, DT_I8)
    w = V(128, 1, DT_F32)
    for sc in (V(6, 7, DT_F32), V(5, 8, DT_F32)):
        assert lib.q3_norm_rope_quant_heads(x, w, None, None, q8, sc, 8, C.c_float(1 / 128), 0,
                                            None) == ERR_VIEW


def test_gate_up_scale_shape(lib):
    M, K, N = 8, 1024, 3072
    a, as_, wg, wgs = gemm_operands(M, K, N)
    s8 = V(M, N, DT_I8)
    for ss in (V(M, N // 256 - 1, DT_F32), V(M, N // 256, DT_F32, col_bytes=0)):
        assert lib.q3_gemm_gate_up_swiglu_quant(a, as_, wg, wgs, wg, wgs, s8, ss, 256,
                                                None) == ERR_VIEW


@pytest.mark.parametrize("fn", ["q3_gemm_nt_group_argmax", "q3_gemm_nt_group_argmax_noalloc"])
def test_argmax_row_limit_is_unsupported(lib, fn):
    """More than 256 rows: Q3_ERR_UNSUPPORTED, or a silent no-op with the
    reference's behaviour switched on (kernels/lm_argmax.h:82)."""
    M, K, N = 300, 1024, 1024
    a, as_, b, bs = gemm_operands(M, K, N)
    best, bidx = V(M, 1, DT_F32), V(M, 1, DT_I32)
    f = getattr(lib, fn)
    assert f(a, as_, b, bs, best, bidx, 256, None) == ERR_UNSUPPORTED
    prev = lib.q3_set_silent_unsupported(1)
    try:
        assert f(a, as_, b, bs, best, bidx, 256, None) == OK
    finally:
        lib.q3_set_silent_unsupported(prev)


def test_model_open_rejects_zero_kv_heads(lib):
    lay = Layout(ModelShape(layers=1, vocab=1024))
    c = _lib.CLayout.from_buffer_copy(lay.c)
    c.kv_heads = 0
    h = C.c_void_p()
    assert lib.q3_model_open(C.c_void_p(_ADDR), C.byref(c), None, C.byref(h)) == ERR_UNSUPPORTED
    assert not h.value


def test_argmax_noalloc_key_limit(lib):
    """More keys than the fixed 2^19-slot array (256 rows x 2374 column
    blocks of 128): rejected before launch, like the allocating entry point,
    whose per-stream workspace has the same size."""
    M, K, N = 256, 1024, 2374 * 128
    a, as_, b, bs = gemm_operands(M, K, N)
    best, bidx = V(M, 1, DT_F32), V(M, 1, DT_I32)
    for fn in (lib.q3_gemm_nt_group_argmax_noalloc, lib.q3_gemm_nt_group_argmax):
        assert fn(a, as_, b, bs, best, bidx, 256, None) == ERR_UNSUPPORTED


def test_group_bscale_only_for_stores(lib):
    """b_scale [N][K/g] (per row and K-group) is taken by the plain and
    residual stores only: the head epilogues, the paged K/V GEMM, gate/up and
    argmax report Q3_ERR_UNSUPPORTED before anything is launched."""
    M, K, N = 8, 1024, 1024
    a, as_, b, _ = gemm_operands(M, K, N)
    bsg = V(N, K // 256, DT_F32)
    q8, qs = V(M, N, DT_I8), V(M, N // 128, DT_F32)
    assert lib.q3_gemm_nt_group_store(a, as_, b, bsg, None, 256, None, q8, qs, None, None, None,
                                      C.c_float(0), None) == ERR_UNSUPPORTED
    kv = paged()
    assert lib.q3_gemm_nt_group_kv_paged(a, as_, b, bsg, 256, C.byref(kv), 0, 1, None, None, None,
                                         C.c_float(0), None) == ERR_UNSUPPORTED
    s8, ss = V(M, N, DT_I8), V(M, N // 256, DT_F32)
    assert lib.q3_gemm_gate_up_swiglu_quant(a, as_, b, bsg, b, bsg, s8, ss, 256,
                                            None) == ERR_UNSUPPORTED
    best, bidx = V(M, 1, DT_F32), V(M, 1, DT_I32)
    assert lib.q3_gemm_nt_group_argmax(a, as_, b, bsg, best, bidx, 256, None) == ERR_UNSUPPORTED
    # a [N][K/g] view with too few rows is an inconsistent view, not per-group
    assert lib.q3_gemm_nt_group_store(a, as_, b, V(N - 1, K // 256, DT_F32), V(M, N, DT_F32), 256,
                                      None, None, None, None, None, None, C.c_float(0),
                                      None) == ERR_VIEW


def test_zero_rows_return_ok_without_launching(lib):
    """An operator with 0 rows returns Q3_OK before any device call (this
    runs with no GPU), and 0-row views may carry NULL data, which is what an
    empty torch tensor hands over: the reference's row loops
    (group_gemm.h:91, swiglu_quant.h:164, lm_argmax.h:72, rmsnorm.h:34,
    quant.h:89, norm_rope_quant.h:88, attention_gqa.h:549) do nothing."""
    def E(cols, dt):
        es = 1 if dt == DT_I8 else 4
        return C.byref(_lib.View(None, cols * es, es, 0, cols, dt))

    K, N = 1024, 2048
    a, as_ = E(K, DT_I8), E(K // 256, DT_F32)
    b, bs = V(N, K, DT_I8), V(N, 1, DT_F32)
    assert lib.q3_gemm_nt_group_store(a, as_, b, bs, E(N, DT_F32), 256, None, None, None, None,
                                      None, None, C.c_float(0), None) == OK
    assert lib.q3_gemm_nt_group_store(a, as_, b, bs, E(N, DT_F32), 256, E(N, DT_F32), None, None,
                                      None, None, None, C.c_float(0), None) == OK
    kv = paged()
    assert lib.q3_gemm_nt_group_kv_paged(a, as_, V(1024, K, DT_I8), V(1024, 1, DT_F32), 256,
                                         C.byref(kv), 5, 1, None, None, None, C.c_float(0),
                                         None) == OK
    assert lib.q3_gemm_gate_up_swiglu_quant(a, as_, V(3072, K, DT_I8), V(3072, 1, DT_F32),
                                            V(3072, K, DT_I8), V(3072, 1, DT_F32),
                                            E(3072, DT_I8), E(12, DT_F32), 256, None) == OK
    for fn in (lib.q3_gemm_nt_group_argmax, lib.q3_gemm_nt_group_argmax_noalloc):
        assert fn(a, as_, b, bs, E(1, DT_F32), E(1, DT_I32), 256, None) == OK
    H = 1024
    w = V(H, 1, DT_F32)
    assert lib.q3_rmsnorm_rows(E(H, DT_F32), w, E(H, DT_F32), C.c_float(1 / H), None) == OK
    assert lib.q3_quant_rows_heads(E(H, DT_F32), E(H, DT_I8), E(8, DT_F32), 128, None) == OK
    assert lib.q3_embedding_rmsnorm_rows(V(64, H, DT_I8), V(64, 1, DT_F32), E(1, DT_I32),
                                         E(H, DT_F32), w, E(H, DT_F32), C.c_float(1 / H),
                                         None) == OK
    assert lib.q3_norm_rope_quant_heads(E(H, DT_F32), V(128, 1, DT_F32), E(64, DT_F32),
                                        E(64, DT_F32), E(H, DT_I8), E(8, DT_F32), 8,
                                        C.c_float(1 / 128), 1, None) == OK
    for causal in (1, 0):
        assert lib.q3_attention_heads_gqa_tokscale_paged(
            E(16 * 128, DT_I8), E(16, DT_F32), C.byref(kv), 40, E(16 * 128, DT_I8),
            E(16, DT_F32), 16, 8, 128, causal, C.c_float(0.088), None) == OK
    # a NULL data pointer on a view that has rows is still rejected
    assert lib.q3_rmsnorm_rows(C.byref(_lib.View(None, 4 * H, 4, 2, H, DT_F32)), w,
                               V(2, H, DT_F32), C.c_float(1 / H), None) == -1
