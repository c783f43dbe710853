"""Blob layout and C ABI checks that need no GPU: offsets equal the
reference's tools/pqwf.py Layout (golden layout.json), the writer's
quantisation, every exported symbol, and the host-side error paths."""
from __future__ import annotations

import ctypes as C
import re

import numpy as np
import pytest

from conftest import REPO, golden
from q3ops import _lib
from q3ops.layout import CONFIGS, InitConfig, Layout, ModelShape, init_random_blob, quantize_rows_host


def test_layout_matches_reference():
    ref = golden("layout.json")
    for case in ref["cases"]:
        lay = Layout(ModelShape(**case["params"]))
        for k, v in lay.offsets.items():
            assert v == case["offsets"][k], (case["params"], k)
    assert Layout().header_text() == ref["default_header"]


def test_default_layout_offsets():
    """The default (Qwen3-0.6B, max_seq 256) layout's scratch end and KV
    strides with per-(token, KV head) scales, tools/pqwf.py:124-135 (the
    reference's checked-in config/model_big.h predates those scales: one
    scale per token, a KV stride of 526336)."""
    lay = Layout()
    assert lay["kSCRATCH_END"] == 791_880_192
    assert lay["kKV_STRIDE"] == 540_672
    assert lay["kKV_VOFF"] == 270_336


def test_header_symbols_exported():
    text = (REPO / "include" / "q3ops.h").read_text()
    names = set(re.findall(r"^\w[\w\s\*]*?\b(q3_\w+)\(", text, flags=re.M))
    assert len(names) >= 20
    lib = _lib.lib()
    for n in sorted(names):
        assert hasattr(lib, n), n
    assert names <= set(_lib.SIGNATURES), names - set(_lib.SIGNATURES)


def test_library_is_gfx950_only_and_independent_of_oracle():
    data = (REPO / "qwen3-tile-ops_amd" / "q3ops" / "libq3ops.so").read_bytes()
    assert b"gfx950" in data
    assert b"liboracle" not in data and b"orc_" not in data


def test_quantize_rows_host_semantics():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (64, 1024)).astype(np.float32)
    q, s = quantize_rows_host(w)
    assert np.abs(q.astype(int)).max() == 127
    assert np.all(s == (np.abs(w).max(1) * np.float32(1 / np.float32(127))).astype(np.float32))
    q0, s0 = quantize_rows_host(np.zeros((2, 16), np.float32))
    assert not q0.any() and not s0.any()


def test_writer_deterministic_and_ctrl():
    shape, init = CONFIGS["cfg0"]
    lay = Layout(shape)
    a = init_random_blob(lay, init, threads=1)
    b = init_random_blob(lay, init, threads=7)
    assert np.array_equal(a, b)
    gv = lay.global_views(a)
    assert list(gv["ctrl"]) == [40, 2, 256, 0]
    assert np.all((gv["ids"][:40] >= 0) & (gv["ids"][:40] < 1024))
    # ids_seed 0 reproduces convert_pqwf.parse_ids' default ids 100 + 10 i
    c = init_random_blob(lay, InitConfig(ids_seed=0, n_prompt=5, n_gen=1))
    assert list(lay.global_views(c)["ids"][:6]) == [100, 110, 120, 130, 140, 150]


def _view(ptr=0, rb=4, cb=4, rows=1, cols=1, dt=_lib.DT_F32):
    return C.byref(_lib.View(ptr, rb, cb, rows, cols, dt))


def test_error_paths_on_host():
    """Argument validation runs before any launch, so these need no GPU."""
    L = _lib.lib()
    assert L.q3_rmsnorm_rows(None, None, None, C.c_float(1.0), None) == -1
    # dtype mismatch: an i8 view where f32 is expected
    assert L.q3_rmsnorm_rows(_view(16, 1024, 1, 1, 1024, _lib.DT_I8), _view(16), _view(16),
                             C.c_float(1.0), None) == -2
    # GEMM with N not a multiple of 128 is rejected (group_gemm.h:47-49) ...
    a = _view(16, 256, 1, 1, 256, _lib.DT_I8)
    b = _view(16, 256, 1, 100, 256, _lib.DT_I8)
    s = _view(16, 4, 4, 100, 1, _lib.DT_F32)
    o = _view(16, 400, 4, 1, 100, _lib.DT_F32)
    rc = L.q3_gemm_nt_group_store(a, s, b, s, o, 256, None, None, None, None, None, None,
                                  C.c_float(0), None)
    assert rc == -4
    # ... and is a silent no-op in the reference-compatible mode
    prev = L.q3_set_silent_unsupported(1)
    try:
        rc = L.q3_gemm_nt_group_store(a, s, b, s, o, 256, None, None, None, None, None, None,
                                      C.c_float(0), None)
        assert rc == 0
    finally:
        L.q3_set_silent_unsupported(prev)
    # attention only supports head_dim 128
    kv = _lib.PagedKV(16, 16, 16, 16, 16, 32, 32 * 256, 256, 32 * 8, 8)
    q = _view(16, 256, 1, 1, 256, _lib.DT_I8)
    qs = _view(16, 8, 4, 1, 2, _lib.DT_F32)
    assert L.q3_attention_heads_gqa_tokscale_paged(q, qs, C.byref(kv), 1, q, qs, 2, 1, 64, 1,
                                                   C.c_float(0.1), None) == -4
    assert L.q3_status_str(-6) == b"unsupported CTRL mode"


def test_model_open_rejects_unsupported_layout():
    lay = Layout(ModelShape(head_dim=64, layers=1, vocab=1024))
    h = C.c_void_p()
    assert _lib.lib().q3_model_open(C.c_void_p(16), C.byref(lay.c), None, C.byref(h)) == -4
