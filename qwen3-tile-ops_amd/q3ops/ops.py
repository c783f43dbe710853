"""Python mirror of the reference operator surface (kernels/*.h) over the C
ABI.  Arguments are torch tensors on the GPU (or None where the reference
passes nullptr); names, argument order and meaning follow the reference
signatures cited on each function.  Shapes follow the reference's
MatrixView conventions: 2-D row-major tensors, and [n][1] column vectors for
per-row scales and norm gains (a 1-D tensor is taken as [n][1]).

Every call enqueues work on torch's current stream and raises Q3Error on a
non-zero status.  There is no fallback path: the HIP library must be built.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import DT_F32, DT_I8, DT_I32, LM_ARGMAX, PagedKV, View, check, lib

_DT = {torch.int8: DT_I8, torch.float32: DT_F32, torch.int32: DT_I32}


def view(t: torch.Tensor | None):
    """MatrixView of a tensor (kernels/matrix.h:27-34); None -> NULL."""
    if t is None:
        return None
    if t.dtype not in _DT:
        raise TypeError(f"unsupported dtype {t.dtype}")
    if not t.is_cuda:
        raise ValueError("operator views must point at device memory")
    es = t.element_size()
    if t.dim() == 1:
        if t.stride(0) != 1:
            raise ValueError("1-D views must be contiguous")
        return C.byref(View(t.data_ptr(), es, es, t.shape[0], 1, _DT[t.dtype]))
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("views must be 2-D with dense columns")
    row_bytes = t.stride(0) * es if t.shape[0] > 1 else t.shape[1] * es
    return C.byref(View(t.data_ptr(), row_bytes, es, t.shape[0], t.shape[1], _DT[t.dtype]))


def _stream(stream=None) -> C.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def paged_kv(k: torch.Tensor, v: torch.Tensor, ks: torch.Tensor, vs: torch.Tensor,
             table: torch.Tensor, page_tokens: int = 32) -> PagedKV:
    """kernels/kv_pages.h:13-24.  k/v: [pages, page_tokens, kv_dim] int8,
    ks/vs: [pages, page_tokens, kv_heads] f32, table: int16/uint16-compatible
    logical->physical map on the device.

    The returned struct holds only device addresses, so it also keeps the
    five tensors alive (a freed table would be reallocated under the
    kernel's feet).  Every table entry is checked against the page count,
    because the C ABI, like the reference PagedKV, carries no page count."""
    for t in (k, v, ks, vs):
        assert t.is_cuda and t.is_contiguous()
    assert k.dtype == torch.int8 and v.dtype == torch.int8
    assert ks.dtype == torch.float32 and vs.dtype == torch.float32
    assert table.dtype in (torch.int16, torch.uint16) and table.is_cuda and table.is_contiguous()
    n_pages = k.shape[0]
    assert v.shape[0] == n_pages and ks.shape[0] == n_pages and vs.shape[0] == n_pages
    tab = table.cpu().numpy().view("uint16")
    if tab.size and int(tab.max()) >= n_pages:
        raise ValueError(f"page table entry {int(tab.max())} >= {n_pages} pages")
    kv_dim = k.shape[-1]
    kv_heads = ks.shape[-1]
    kv = PagedKV(k.data_ptr(), v.data_ptr(), ks.data_ptr(), vs.data_ptr(), table.data_ptr(),
                 page_tokens, page_tokens * kv_dim, kv_dim, page_tokens * kv_heads * 4,
                 kv_heads * 4)
    kv._keep = (k, v, ks, vs, table)
    kv.n_pages = n_pages
    kv.n_logical = table.numel()
    return kv


def _check_tokens(kv: PagedKV, end_token: int) -> None:
    n_logical = getattr(kv, "n_logical", None)
    if n_logical is not None and end_token > n_logical * kv.page_tokens:
        raise ValueError(f"token {end_token - 1} is beyond the page table "
                         f"({n_logical} pages of {kv.page_tokens})")


def embedding_rmsnorm_rows(table, scale, ids, tmp, w, out, inv, stream=None):
    """kernels/embedding.h:99-168."""
    check(lib().q3_embedding_rmsnorm_rows(view(table), view(scale), view(ids), view(tmp),
                                          view(w), view(out), C.c_float(inv), _stream(stream)),
          "embedding_rmsnorm_rows")


def rmsnorm_rows(x, w, out, inv, stream=None):
    """kernels/rmsnorm.h:34-81."""
    check(lib().q3_rmsnorm_rows(view(x), view(w), view(out), C.c_float(inv), _stream(stream)),
          "rmsnorm_rows")


def quant_rows_heads(x, qi8, scale, group_cols, stream=None):
    """kernels/quant.h:89-138."""
    check(lib().q3_quant_rows_heads(view(x), view(qi8), view(scale), group_cols,
                                    _stream(stream)), "quant_rows_heads")


def gemm_nt_group_store(a, a_scale, b, b_scale, out, group_k=128, add=None, q8=None, qs=None,
                        nw=None, cos=None, sin=None, inv_hd=0.0, stream=None):
    """kernels/group_gemm.h:27-222."""
    check(lib().q3_gemm_nt_group_store(view(a), view(a_scale), view(b), view(b_scale),
                                       view(out), group_k, view(add), view(q8), view(qs),
                                       view(nw), view(cos), view(sin), C.c_float(inv_hd),
                                       _stream(stream)), "gemm_nt_group_store")


def gemm_nt_group_kv_paged(a, a_scale, b, b_scale, group_k, kv: PagedKV, pos0, is_v, nw=None,
                           cos=None, sin=None, inv_hd=0.0, stream=None):
    """K/V epilogues of gemm_nt_group_store writing page slots
    (main_big.cpp:185-209)."""
    _check_tokens(kv, pos0 + a.shape[0])
    check(lib().q3_gemm_nt_group_kv_paged(view(a), view(a_scale), view(b), view(b_scale),
                                          group_k, C.byref(kv), pos0, int(is_v), view(nw),
                                          view(cos), view(sin), C.c_float(inv_hd),
                                          _stream(stream)), "gemm_nt_group_kv_paged")


def norm_rope_quant_heads(x, w, cos, sin, q8, scale, heads, inv_hd, do_rope=True, stream=None):
    """kernels/norm_rope_quant.h:88-111."""
    check(lib().q3_norm_rope_quant_heads(view(x), view(w), view(cos), view(sin), view(q8),
                                         view(scale), heads, C.c_float(inv_hd), int(do_rope),
                                         _stream(stream)), "norm_rope_quant_heads")


def attention_heads_gqa_tokscale_paged(q8, q_scale, kv: PagedKV, kv_len, o8, os, heads,
                                       kv_heads, head_dim, causal, qk_scale, stream=None):
    """kernels/attention_gqa.h:549-572."""
    _check_tokens(kv, kv_len)
    check(lib().q3_attention_heads_gqa_tokscale_paged(view(q8), view(q_scale), C.byref(kv),
                                                      kv_len, view(o8), view(os), heads,
                                                      kv_heads, head_dim, int(causal),
                                                      C.c_float(qk_scale), _stream(stream)),
          "attention_heads_gqa_tokscale_paged")


def gemm_gate_up_swiglu_quant(a, a_scale, wg, wgs, wu, wus, s8, ss, group_k=256, stream=None):
    """kernels/swiglu_quant.h:164-255."""
    check(lib().q3_gemm_gate_up_swiglu_quant(view(a), view(a_scale), view(wg), view(wgs),
                                             view(wu), view(wus), view(s8), view(ss), group_k,
                                             _stream(stream)), "gemm_gate_up_swiglu_quant")


def gemm_nt_group_argmax(a, a_scale, b, b_scale, best, bidx, group_k=128, stream=None):
    """kernels/lm_argmax.h:72-182 (best/bidx are read and updated)."""
    check(lib().q3_gemm_nt_group_argmax(view(a), view(a_scale), view(b), view(b_scale),
                                        view(best), view(bidx), group_k, _stream(stream)),
          "gemm_nt_group_argmax")


def gemm_nt_group_argmax_noalloc(a, a_scale, b, b_scale, best, bidx, group_k=128, stream=None):
    """gemm_nt_group_argmax with the library's fixed device key array instead
    of an allocated workspace (no reference counterpart; for callers that
    cannot allocate).  Calls that overlap on one GPU race."""
    check(lib().q3_gemm_nt_group_argmax_noalloc(view(a), view(a_scale), view(b), view(b_scale),
                                                view(best), view(bidx), group_k,
                                                _stream(stream)),
          "gemm_nt_group_argmax_noalloc")


def argmax_logits(logits, out_id, stream=None):
    """main_big.cpp:300-322 (out_id: int32 device tensor, element 0)."""
    check(lib().q3_argmax_logits(view(logits), C.c_void_p(out_id.data_ptr()), _stream(stream)),
          "argmax_logits")


__all__ = ["view", "paged_kv", "embedding_rmsnorm_rows", "rmsnorm_rows", "quant_rows_heads",
           "gemm_nt_group_store", "gemm_nt_group_kv_paged", "norm_rope_quant_heads",
           "attention_heads_gqa_tokscale_paged", "gemm_gate_up_swiglu_quant",
           "gemm_nt_group_argmax", "gemm_nt_group_argmax_noalloc", "argmax_logits", "LM_ARGMAX"]
