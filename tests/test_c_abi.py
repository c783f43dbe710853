"""The boundary from compiled callers, the way the reference's only caller of
the ops (src/main_big.cpp:332-369) would use it:

- a C99 program (tests/c_abi/abi_check.c), compiled here with -std=c99
  -pedantic -Werror against include/q3ops.h and linked with libq3ops.so,
  computes blob layouts and hits the host error paths (CPU);
- a C++ driver (tests/c_abi/generate_cfg0.cpp, built by
  qwen3-tile-ops_amd/build.py) runs the model-level replacement of that
  caller (layout, blob, q3_model_open, q3_generate) on config 0, and its ids
  and logits are compared with the reference's goldens (GPU).
"""
from __future__ import annotations

import shutil
import subprocess

import numpy as np
import pytest

from conftest import REPO, bits_equal, describe_diff, golden
from q3ops.layout import CONFIGS, Layout

C_DIR = REPO / "tests" / "c_abi"
LIBDIR = REPO / "qwen3-tile-ops_amd" / "q3ops"


def _parse(out: str) -> dict[str, list[str]]:
    res = {}
    for line in out.splitlines():
        k, *v = line.split()
        res[k] = v
    return res


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c99_caller_layout_and_error_paths(tmp_path):
    exe = tmp_path / "abi_check"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    f"-I{REPO / 'include'}", str(C_DIR / "abi_check.c"), f"-L{LIBDIR}", "-lq3ops",
                    f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)], check=True)
    r = _parse(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    # layouts: equal to the Python mirror, which test_layout_abi pins to the
    # reference's tools/pqwf.py offsets (golden layout.json)
    lay = Layout()
    assert int(r["layout_rc"][0]) == 0
    for k in ("kSCRATCH_END", "kKV_STRIDE", "kKV_VOFF", "kLOGITS"):
        assert int(r[k][0]) == lay[k], k
    assert int(r["cfg0_kSCRATCH_END"][0]) == Layout(CONFIGS["cfg0"][0])["kSCRATCH_END"]
    assert int(r["header_len"][0]) == len(lay.header_text())
    assert r["header_nul"] == ["1"]
    # host error paths: Q3_ERR_ARG, nothing launched
    err_arg = int(r["Q3_OK"][2])
    assert int(r["Q3_OK"][0]) == 0 and err_arg == -1
    for k in ("layout_null", "open_null", "open_null_layout", "generate_null", "close_null"):
        assert int(r[k][0]) == err_arg, k
    # pqwf.py quantize_rows, closed form: scale = 1 * RN(1/127); 0.5 / scale =
    # 63.5 -> 64 (half to even), -1 -> -127, 0.25 -> 31.75 -> 32; a zero row
    # has scale 0 and codes 0
    assert int(r["quant_rc"][0]) == 0
    assert [int(v) for v in r["quant_row0"]] == [64, -127, 32, 0]
    assert r["quant_row1_zero"] == ["1"]


@pytest.mark.gpu
def test_cpp_driver_generates_cfg0(cuda, tmp_path):
    exe = C_DIR / "bin" / "generate_cfg0"
    assert exe.exists(), "build first: python qwen3-tile-ops_amd/build.py"
    out = tmp_path / "cfg0.bin"
    p = subprocess.run([str(exe), str(out)], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    data = out.read_bytes()
    g = golden("cfg0.npz")
    ids = np.frombuffer(data[:8], np.int32)
    logits = np.frombuffer(data[8:], np.float32)
    assert np.array_equal(ids, g["generated"]), (ids, g["generated"])
    assert bits_equal(logits, g["logits"]), describe_diff(logits, g["logits"])
