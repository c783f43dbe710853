"""Builds libq3ops.so (HIP kernels for gfx950 + host orchestration).

    python qwen3-tile-ops_amd/build.py          # compile everything
    python qwen3-tile-ops_amd/build.py -j 8

HIP sources (csrc/*.hip) are compiled by hipcc for gfx950 only; host-only
sources (csrc/*.cpp) by g++.  The shared library is written next to the
Python binding (q3ops/libq3ops.so) so it travels with the source tree.

Numerics flags: -ffp-contract=off (no FMA contraction: every f32 expression
is one IEEE operation, as in the numpy mirror); no fast-math; f32 denormals
are kept (no -fgpu-flush-denormals-to-zero); correctly rounded f32 division
and sqrt stay on (clang's HIP default).  Packed-f32 instructions are turned
off for device code (-target-feature -packed-fp32-ops).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "q3ops" / "libq3ops.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-parameter",
    f"-I{REPO / 'include'}", f"-I{CSRC}",
]
CXX_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Wall", "-Wno-unused-parameter", f"-I{REPO / 'include'}", f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(jobs: int = 0, verbose: bool = False) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    hipcc = str(ROCM / "bin" / "hipcc")
    objs: list[Path] = []
    cmds: list[list[str]] = []
    for src in sorted(CSRC.glob("*.hip")):
        obj = BUILD / (src.stem + ".hip.o")
        cmds.append([hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
        objs.append(obj)
    for src in sorted(CSRC.glob("*.cpp")):
        obj = BUILD / (src.stem + ".cpp.o")
        cmds.append(["g++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)])
        objs.append(obj)
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_run, c) for c in cmds]
        for f in futs:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-pthread"])
    os.replace(tmp, OUT)
    build_c_driver()
    if verbose:
        print(f"built {OUT}")
    return OUT


C_DRIVER_SRC = REPO / "tests" / "c_abi" / "generate_cfg0.cpp"
C_DRIVER = REPO / "tests" / "c_abi" / "bin" / "generate_cfg0"


def build_c_driver() -> Path | None:
    """A C++ caller of the model-level ABI (tests/c_abi/generate_cfg0.cpp),
    linked against libq3ops.so and the HIP runtime; the GPU test runs it."""
    if not C_DRIVER_SRC.exists():
        return None
    C_DRIVER.parent.mkdir(parents=True, exist_ok=True)
    rel = os.path.relpath(OUT.parent, C_DRIVER.parent)
    _run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
          f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}", str(C_DRIVER_SRC),
          f"-L{OUT.parent}", "-lq3ops", f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,$ORIGIN/{rel}:{ROCM / 'lib'}", "-o", str(C_DRIVER)])
    return C_DRIVER


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=0)
    args = ap.parse_args()
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
