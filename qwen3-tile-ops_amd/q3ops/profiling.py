"""Summaries of rocprofv3 CSV output for the measurement record
(profiles/).  Every summary there is produced by this module from the CSV
files of one of the rocprofv3 commands named in the summary.

    python -m q3ops.profiling stats <kernel_stats.csv> --cmd "<command>" [--top N] [--title T]
        [--no-classes]
        -> markdown table of the per-kernel statistics (stdout)

    python -m q3ops.profiling pmc --fetch <counter_collection.csv>
        --write <counter_collection.csv> --calib-bytes N --cmd "<command>"
        -> JSON: per kernel class, FETCH_SIZE / WRITE_SIZE per dispatch
           (KiB, as read) and HBM-side bytes per dispatch after calibration

    python -m q3ops.profiling counters <counter_collection.csv> [...]
        --cmd "<command>" [--cus 256]
        -> JSON: per kernel class, the mean of every collected counter per
           dispatch, plus the derived MFMA and VALU figures (below)

Calibration: the profiled command ends with device-to-device copies of
N bytes (bench.py --calib-copy); each reads and writes exactly N bytes, so
factor = N / (counter KiB * 1024) for the copy dispatches of that size, and
every kernel's counter is scaled by it.  FETCH_SIZE and WRITE_SIZE count
L2 <-> fabric traffic, i.e. bytes that left the L2 (last-level-cache hits
included).

Derived figures (when their counters were collected), rocprofv3's own
MfmaUtil and VALUBusy expressions with one change: under --pmc every
dispatch is serialised and GRBM_GUI_ACTIVE also counts the profiler's own
window around it (several times the kernel), so the kernel's cycles are
taken from a separate --kernel-trace run of the same command (--stats, its
average duration x --clock-ghz):
  int8 ops per dispatch = SQ_INSTS_VALU_MFMA_MOPS_I8 * 512
  MFMA util   = SQ_VALU_MFMA_BUSY_CYCLES / (kernel cycles * CUs * 4 SIMDs)
  VALU busy   = SQ_ACTIVE_INST_VALU / (kernel cycles * CUs)
  co-issue    = SQ_VALU_MFMA_COEXEC_CYCLES / (kernel cycles * CUs * 4 SIMDs)
  achieved    = int8 ops per dispatch / kernel duration
  L2 hit rate = TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import sys

# kernel symbol -> kernel class.  Decode classes are those of
# q3_model_set_kernel_timing; gemv_wr_kernel<prologue, KB, NMAT, R, ...>,
# gemv_kernel<GPW, KSTEPS, NT, NMAT, prologue,
# partials, ...> and gemm_tile_kernel<BM, BN, WGM, NMAT, STAGES, KS, epilogue,
# group, ...> and gemm_stream_kernel<BM, NWN, KP, NT, NMAT, D, KB, epilogue,
# group, ...> are matched on their template arguments (epilogue numbers:
# 1 residual add, 2 V head quant, 3 Q/K norm+RoPE+quant, 6 SwiGLU+quant,
# 7 the three-segment Q|K|V launch).
CLASS_OF = [
    (r"attn_decode_kernel<1, ", "attn_decode"),
    (r"qkv_attn_kernel<", "attn_decode"),        # Q|K|V projection + attention, one launch
    (r"down_qkv_attn_kernel", "attn_decode"),    # the same with the previous layer's down projection
    (r"attn_decode_kernel<2, ", "attn_decode_batch"),
    (r"gemv_wr_kernel<[13], 1, 1, 2,", "gemv_qkv"),
    (r"gemv_wr_kernel<1, 1, 2, 3,", "gemv_gate_up"),
    (r"gemv_wr_kernel<2, 3, 1, 1,", "gemv_down"),
    (r"gemv_kernel<1, 4, 1, 1, [13], 0", "gemv_qkv"),
    (r"gemv_kernel<4, 2, 1, 1,", "gemv_o"),
    (r"gemv_kernel<1, 4, 1, 2, 1, 1", "gemv_gate_up"),
    (r"gemv_kernel<3, 4, 1, 1, 2, 2", "gemv_down"),
    (r"gemv_kernel<1, 4, 1, 1, 0, 0, \w+, [24],", "batch_qkv"),
    (r"gemv_kernel<1, 4, 1, 2, 0, 0, \w+, [24],", "batch_gate_up"),
    (r"gemv_kernel<3, 4, 1, 1, 0, 0,", "batch_down"),
    (r"gemv_row_kernel<1, 4", "lm_head"),
    (r"gemv_stream_kernel<", "lm_head_rows"),
    (r"gemm_tile_kernel<\d+, \d+, \d+, 2, \d+, \d+, 6,", "prefill_gate_up"),
    (r"gemm_tile_kernel<\d+, \d+, \d+, 1, \d+, \d+, 7,", "prefill_qkv"),
    (r"gemm_tile_kernel<\d+, \d+, \d+, 1, \d+, \d+, 1, 128", "prefill_o"),
    (r"gemm_tile_kernel<\d+, \d+, \d+, 1, \d+, \d+, 1, 256", "prefill_down"),
    (r"gemm_stream_kernel<(\d+, ){7}6,", "prefill_gate_up"),
    (r"gemm_stream_kernel<(\d+, ){7}7,", "prefill_qkv"),
    (r"gemm_stream_kernel<(\d+, ){7}1, 128", "prefill_o"),
    (r"gemm_stream_kernel<(\d+, ){7}1, 256", "prefill_down"),
    (r"pack_b_kernel", "pack_weights"),
    (r"attn_prefill_kernel", "prefill_attention"),
    (r"attention_kernel", "prefill_attention"),
    (r"rows1024_kernel", "norm_quant_rows"),
    (r"quant_groups_kernel", "quant_rows"),
    (r"qkv_heads_kernel", "qkv_heads"),
    (r"gemm_tile_kernel<(\d+, ){6}4,", "lm_head_batch"),
    (r"argmax_finish_kernel", "argmax_finish"),
]


def short_name(name: str, width: int = 90) -> str:
    """Kernel symbol without return type, anonymous namespace and argument
    list, cut to `width` characters (library kernels have very long template
    names)."""
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            n = n[:i]
            break
    return n if len(n) <= width else n[:width - 3] + "..."


def class_of(name: str) -> str | None:
    for pat, cls in CLASS_OF:
        if re.search(pat, name):
            return cls
    return None


def stats_md(path: str, cmd: str, top: int, title: str | None = None, classes: bool = True) -> str:
    """classes=False leaves the class column empty (a workload of op-level
    calls, whose kernels the model-path classes would misname)."""
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ([f"# {title}", ""] if title else []) + [f"Command: `{cmd}`", "", f"Source: rocprofv3 `--kernel-trace --stats` ({path.split('/')[-1]})", "",
           "| kernel | class | calls | avg us | min us | max us | % time |", "|---|---|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        cls = (class_of(r["Name"]) or "") if classes else ""
        out.append(f"| `{short_name(r['Name'])}` | {cls} | {r['Calls']} | "
                   f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    return "\n".join(out) + "\n"


def _per_kernel(path: str, counter: str) -> dict[str, list[float]]:
    agg: dict[str, list[float]] = {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        agg.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return agg


def _calibration(agg: dict[str, list[float]], calib_bytes: int) -> float:
    kib = calib_bytes / 1024.0
    vals = [v for v in agg.get("__amd_rocclr_copyBuffer", []) if v > 0.25 * kib]
    if not vals:
        raise SystemExit("no calibration copy dispatches found")
    return kib / statistics.median(vals)


def pmc_json(fetch: str, write: str, calib_bytes: int, cmd: str) -> dict:
    f = _per_kernel(fetch, "FETCH_SIZE")
    w = _per_kernel(write, "WRITE_SIZE")
    cf, cw = _calibration(f, calib_bytes), _calibration(w, calib_bytes)
    kernels = {}
    for name in sorted(set(f) | set(w)):
        cls = class_of(name)
        if cls is None:
            continue
        # a class with several variants (e.g. the layer-0 embedding prologue
        # of the Q|K|V GEMV) is represented by its most frequent one
        if cls in kernels and kernels[cls]["dispatches"] >= len(f.get(name, [])):
            continue
        fk = statistics.mean(f.get(name, [0.0]))
        wk = statistics.mean(w.get(name, [0.0]))
        kernels[cls] = {
            "kernel": short_name(name),
            "dispatches": len(f.get(name, [])),
            "fetch_kib_raw": fk, "write_kib_raw": wk,
            "fetch_bytes": fk * 1024 * cf, "write_bytes": wk * 1024 * cw,
            "bytes_per_dispatch": fk * 1024 * cf + wk * 1024 * cw,
        }
    return {"command": cmd, "calibration": {"copy_bytes": calib_bytes, "fetch_factor": cf,
                                            "write_factor": cw},
            "kernels": kernels}


def _trace_durations(stats: str | None) -> dict[str, float]:
    """kernel symbol -> average duration in ns from a kernel_stats.csv."""
    if not stats:
        return {}
    return {r["Name"]: float(r["AverageNs"]) for r in csv.DictReader(open(stats))}


def counters_json(paths: list[str], cmd: str, cus: int, stats: str | None = None,
                  clock_ghz: float = 2.4, peak_tops: float = 5000.0) -> dict:
    """Per kernel class (and per kernel symbol within it): the mean of every
    counter over its dispatches, merged over several PMC passes, and the
    derived figures of the module docstring."""
    per: dict[str, dict[str, list[float]]] = {}
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            per.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    durs = _trace_durations(stats)
    kernels = {}
    for name, cnt in sorted(per.items()):
        cls = class_of(name)
        if cls is None:
            continue
        mean = {c: statistics.mean(v) for c, v in cnt.items()}
        d = {"kernel": short_name(name), "dispatches": max(len(v) for v in cnt.values()),
             "counters": mean}
        ops = mean.get("SQ_INSTS_VALU_MFMA_MOPS_I8")
        if ops is not None:
            d["int8_ops_per_dispatch"] = ops * 512
        ns = durs.get(name)
        if ns:
            cyc = ns * clock_ghz
            d["trace_avg_us"] = ns / 1e3
            if ops is not None:
                d["achieved_tops"] = ops * 512 / ns / 1e3
                d["frac_of_int8_peak"] = d["achieved_tops"] / peak_tops
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                d["mfma_util"] = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * cus * 4)
            if "SQ_ACTIVE_INST_VALU" in mean:
                d["valu_busy"] = mean["SQ_ACTIVE_INST_VALU"] / (cyc * cus)
            if "SQ_VALU_MFMA_COEXEC_CYCLES" in mean:
                d["mfma_valu_coissue"] = mean["SQ_VALU_MFMA_COEXEC_CYCLES"] / (cyc * cus * 4)
        if "TCC_HIT_sum" in mean and "TCC_MISS_sum" in mean:
            tot = mean["TCC_HIT_sum"] + mean["TCC_MISS_sum"]
            d["l2_hit_rate"] = mean["TCC_HIT_sum"] / tot if tot else None
        key = cls if cls not in kernels else f"{cls}:{short_name(name)}"
        kernels[key] = d
    return {"command": cmd, "cus": cus, "clock_ghz": clock_ghz, "kernels": kernels}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m q3ops.profiling")
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--cmd", required=True)
    s.add_argument("--top", type=int, default=20)
    s.add_argument("--title", help="heading of the markdown summary")
    s.add_argument("--no-classes", action="store_true", help="leave the class column empty")
    p = sub.add_parser("pmc")
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--calib-bytes", type=int, required=True)
    p.add_argument("--cmd", required=True)
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    c.add_argument("--cmd", required=True)
    c.add_argument("--cus", type=int, default=256)
    c.add_argument("--stats", help="kernel_stats.csv of a --kernel-trace run of the same command")
    c.add_argument("--clock-ghz", type=float, default=2.4)
    a = ap.parse_args(argv)
    if a.cmd_name == "stats":
        sys.stdout.write(stats_md(a.csv, a.cmd, a.top, a.title, not a.no_classes))
    elif a.cmd_name == "counters":
        json.dump(counters_json(a.csv, a.cmd, a.cus, a.stats, a.clock_ghz), sys.stdout, indent=1)
        sys.stdout.write("\n")
    else:
        json.dump(pmc_json(a.fetch, a.write, a.calib_bytes, a.cmd), sys.stdout, indent=1)
        sys.stdout.write("\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
