"""ctypes binding of libq3ops.so (the C ABI declared in include/q3ops.h).

The library is loaded from this directory.  A missing library is an error:
there is no fallback implementation of any operator.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libq3ops.so"

# dtype codes (kernels/config.h:86-90)
DT_I8, DT_U8, DT_I32, DT_U32, DT_F32 = 0, 1, 2, 3, 4

Q3_OK = 0
STATUS = {
    0: "ok", -1: "invalid argument", -2: "dtype mismatch",
    -3: "inconsistent view shape or stride", -4: "unsupported shape",
    -5: "HIP runtime error", -6: "unsupported CTRL mode",
    -7: "position, page or id out of range",
}
LM_NONE, LM_LOGITS, LM_ARGMAX = 0, 1, 2


class Q3Error(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS.get(status, status)} ({status})")
        self.status = status


class View(C.Structure):
    """q3_view == kernels/matrix.h MatrixView (data is a device address)."""
    _fields_ = [("data", C.c_void_p), ("row_bytes", C.c_int32), ("col_bytes", C.c_int32),
                ("rows", C.c_uint32), ("cols", C.c_uint32), ("dtype", C.c_uint8)]


class PagedKV(C.Structure):
    """q3_paged_kv == kernels/kv_pages.h PagedKV."""
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("ks", C.c_void_p), ("vs", C.c_void_p),
                ("table", C.c_void_p), ("page_tokens", C.c_uint32), ("page_bytes", C.c_uint32),
                ("row_bytes", C.c_uint32), ("scale_page_bytes", C.c_uint32),
                ("scale_row_bytes", C.c_uint32)]


LAYOUT_DIMS = ["hidden", "layers", "heads", "kv_heads", "head_dim", "inter", "vocab", "seq",
               "max_seq", "half"]
LAYOUT_OFFSETS = [
    "kIDS", "kCTRL", "kX", "kEMB", "kLM", "kNF", "kCOS", "kSIN",
    "kLAYERW_BASE", "kLAYERW_STRIDE",
    "kLQ", "kLQ_SCALE", "kLK", "kLK_SCALE", "kLV", "kLV_SCALE", "kLO", "kLO_SCALE",
    "kLG", "kLG_SCALE", "kLU", "kLU_SCALE", "kLD", "kLD_SCALE",
    "kLAYERN_BASE", "kLAYERN_STRIDE", "kN1", "kNQ", "kNK", "kN2",
    "kLOGITS", "kBLOCK_END",
    "kH", "kH8", "kHS", "kQ", "kK", "kV", "kQ8", "kK8", "kV8", "kQS", "kKS", "kVS",
    "kATTN", "kO", "kO8", "kOS", "kG", "kU", "kSW", "kS8", "kSS", "kARGF", "kARGI",
    "kKV_BASE", "kKV_STRIDE", "kKV_VOFF", "kKV_SOFF", "kSCRATCH_END",
]


class CLayout(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in LAYOUT_DIMS] + [(n, C.c_int64) for n in LAYOUT_OFFSETS]


class InitParams(C.Structure):
    _fields_ = [("weight_seed", C.c_uint64), ("ids_seed", C.c_uint64),
                ("weight_std", C.c_double), ("gain_std", C.c_double),
                ("rope_theta", C.c_double), ("n_prompt", C.c_int32),
                ("n_gen", C.c_int32), ("mode", C.c_int32)]


# Every symbol include/q3ops.h declares, with its argument types.
_VP, _I, _U, _F = C.c_void_p, C.c_int, C.c_uint32, C.c_float
_PV = C.POINTER(View)
_PK = C.POINTER(PagedKV)
SIGNATURES = {
    "q3_set_silent_unsupported": (_I, [_I]),
    "q3_status_str": (C.c_char_p, [_I]),
    "q3_embedding_rmsnorm_rows": (_I, [_PV, _PV, _PV, _PV, _PV, _PV, _F, _VP]),
    "q3_rmsnorm_rows": (_I, [_PV, _PV, _PV, _F, _VP]),
    "q3_quant_rows_heads": (_I, [_PV, _PV, _PV, _U, _VP]),
    "q3_gemm_nt_group_store": (_I, [_PV, _PV, _PV, _PV, _PV, _U, _PV, _PV, _PV, _PV, _PV, _PV,
                                    _F, _VP]),
    "q3_gemm_nt_group_kv_paged": (_I, [_PV, _PV, _PV, _PV, _U, _PK, _U, _I, _PV, _PV, _PV, _F,
                                       _VP]),
    "q3_norm_rope_quant_heads": (_I, [_PV, _PV, _PV, _PV, _PV, _PV, _I, _F, _I, _VP]),
    "q3_attention_heads_gqa_tokscale_paged": (_I, [_PV, _PV, _PK, _U, _PV, _PV, _I, _I, _I, _I,
                                                   _F, _VP]),
    "q3_gemm_gate_up_swiglu_quant": (_I, [_PV, _PV, _PV, _PV, _PV, _PV, _PV, _PV, _U, _VP]),
    "q3_gemm_nt_group_argmax": (_I, [_PV, _PV, _PV, _PV, _PV, _PV, _U, _VP]),
    "q3_gemm_nt_group_argmax_noalloc": (_I, [_PV, _PV, _PV, _PV, _PV, _PV, _U, _VP]),
    "q3_argmax_logits": (_I, [_PV, _VP, _VP]),
    "q3_layout_compute": (_I, [_U] * 9 + [C.POINTER(CLayout)]),
    "q3_layout_header_text": (_I, [C.POINTER(CLayout), C.c_char_p, C.c_size_t]),
    "q3_init_random_blob": (_I, [C.POINTER(CLayout), C.POINTER(InitParams), _VP, _I]),
    "q3_init_normal": (_I, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_size_t, C.c_double,
                            C.c_double, _VP]),
    "q3_init_stream_id": (C.c_uint64, [_I, _I]),
    "q3_quantize_rows_host": (_I, [_VP, C.c_size_t, C.c_size_t, _VP, _VP]),
    "q3_model_open": (_I, [_VP, C.POINTER(CLayout), _VP, C.POINTER(_VP)]),
    "q3_model_set_page_table": (_I, [_VP, _VP, _U]),
    "q3_forward_chunk": (_I, [_VP, _U, _U, _I, _I]),
    "q3_generate": (_I, [_VP]),
    "q3_model_close": (_I, [_VP]),
    "q3_decode_batch": (_I, [_VP, _U, _VP, _VP, _VP, _U, _VP]),
    "q3_model_info": (_I, [_VP, C.POINTER(CLayout), C.POINTER(_VP), C.POINTER(_VP)]),
    "q3_model_fused_status": (_I, [_VP, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "q3_model_repack": (_I, [_VP]),
    "q3_sched_create": (_I, [_U, _U, C.POINTER(_VP)]),
    "q3_sched_destroy": (_I, [_VP]),
    "q3_sched_add": (_I, [_VP, _U, _U, _VP]),
    "q3_sched_get": (_I, [_VP, C.c_int32, _VP]),
    "q3_sched_set": (_I, [_VP, C.c_int32, _VP]),
    "q3_sched_pages": (_I, [_VP, C.c_int32, _VP, _U, _VP]),
    "q3_sched_free_pages": (_I, [_VP, _VP, _U, _VP]),
    "q3_sched_alloc_page": (_I, [_VP, C.c_int32, _VP]),
    "q3_sched_ensure": (_I, [_VP, C.c_int32, _U, _VP]),
    "q3_sched_release": (_I, [_VP, C.c_int32]),
    "q3_sched_finish": (_I, [_VP, C.c_int32]),
    "q3_sched_build": (_I, [_VP, _U, _VP, _U, _VP, _VP]),
    "q3_sched_commit": (_I, [_VP, _VP, _U, _VP]),
    "q3_sched_finish_exhausted": (_I, [_VP, _VP]),
    "q3_sched_run": (_I, [_VP, _VP, _VP, _U, _VP, _VP, _VP, _VP, C.c_uint64]),
    "q3_model_set_kernel_timing": (_I, [_VP, _U]),
    "q3_model_kernel_time": (_I, [_VP, _I, C.POINTER(C.c_double), C.POINTER(C.c_uint32)]),
}

_lib = None


def lib() -> C.CDLL:
    """Loads libq3ops.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python qwen3-tile-ops_amd/build.py` "
                "(there is no CPU fallback for the HIP operators)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != Q3_OK:
        raise Q3Error(status, what)
