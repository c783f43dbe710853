#!/usr/bin/env python3
"""Benchmark of the Qwen3 W8A8 forward path on one MI355X.

    python bench.py [--gpus 1] [--steps 5] [--warmup 2] [--no-cpu]

Workload (perf leg): the 28-layer Qwen3-0.6B shape with
random-init int8 weights (per-row scales), one 512-token prefill chunk and
64 greedy decode steps at batch 1 with the fused lm_head+argmax (CTRL mode
0), i.e. one q3_generate over CTRL = [512, 64, 640, 0].  One step = that
whole generation; inputs (weights, prompt ids) are resident in HBM before
the timed region.  value = (512 + 64) tokens / step time.

Also reported:
  - prefill and decode rates separately (prefill timed alone through
    q3_forward_chunk with the same arguments generate uses);
  - roofline: the dominant kernel, timed live with HIP events on the stream
    it is launched on, against its algorithmic bytes or ops;
  - cpu_baseline: the CPU oracle (oracle/, a C port of tools/ref_qwen3.py)
    running the same generation on the host cores (rank 0 only).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "qwen3-tile-ops_amd"))
sys.path.insert(0, str(REPO))

METRIC = "tok/s prefill(512)+decode(b=1,64), Qwen3-0.6B W8A8, 1 MI355X; %HBM/MFMA peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
N_PROMPT, N_GEN = 512, 64


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_events(fn, reps: int, stream) -> float:
    """Average milliseconds of fn() over reps, HIP events on `stream`."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


def time_graph(launch, count: int, stream, replays: int = 3) -> float:
    """Average milliseconds per launch of `count` back-to-back launches
    (launch(i), i = 0..count-1) captured into one HIP graph on `stream` and
    replayed: the launches reach the GPU without host submission gaps, which
    at a few microseconds per kernel would otherwise dominate (each ctypes
    call through the C ABI costs the host about 10 us).  One eager pass
    first sets up everything a first call does (function attributes,
    workspaces); HIP events on `stream` time the replays."""
    import torch
    for i in range(min(count, 2)):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(count):
            launch(i)
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            g.replay()
        end.record(stream)
    end.synchronize()
    ms = start.elapsed_time(end) / (replays * count)
    del g
    return ms


def kernel_rooflines(stream) -> dict:
    """Times single-kernel shapes of the path through the C ABI, on the
    stream they are launched on, and derives achieved bandwidth / ops."""
    import numpy as np
    import torch
    from q3ops import ops

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    res = {}

    def t8(*shape):
        return torch.from_numpy(rng.integers(-127, 128, shape).astype(np.int8)).to(dev)

    def tf(*shape):
        return torch.from_numpy(rng.uniform(1e-3, 1e-1, shape).astype(np.float32)).to(dev)

    # rotate over copies so the 256 MB MALL cannot serve repeated reads
    def copies(nbytes):
        return max(1, min(8, int(2.0e9 // max(nbytes, 1))))

    # lm_head fused argmax GEMV: M=1, N=151936, K=1024 (decode, HBM bound)
    V, H = 151936, 1024
    nb = V * H
    ws = [(t8(V, H), tf(V)) for _ in range(copies(nb))]
    a, as_ = t8(1, H), tf(1, H // 256)
    best = torch.empty(1, dtype=torch.float32, device=dev)
    bidx = torch.empty(1, dtype=torch.int32, device=dev)

    def lm(i):
        w, s = ws[i % len(ws)]
        ops.gemm_nt_group_argmax(a, as_, w, s, best, bidx, 256, stream=stream)

    ms = time_graph(lm, 24, stream)
    byts = V * H + 4 * V + H + 4 * (H // 256) + 8
    res["lm_argmax_gemv"] = {"ms": ms, "bytes": byts, "GBs": byts / ms / 1e6, "bound": "hbm"}
    del ws

    # decode gate/up GEMV (M=1, N=3072 x2, K=1024): HBM bound
    I = 3072
    ws = [(t8(I, H), tf(I), t8(I, H), tf(I)) for _ in range(copies(2 * I * H))]
    s8 = torch.empty((1, I), dtype=torch.int8, device=dev)
    ss = torch.empty((1, I // 256), dtype=torch.float32, device=dev)

    def gu1(i):
        wg, wgs, wu, wus = ws[i % len(ws)]
        ops.gemm_gate_up_swiglu_quant(a, as_, wg, wgs, wu, wus, s8, ss, 256, stream=stream)

    ms = time_graph(gu1, 64, stream)
    byts = 2 * I * H + 8 * I + H + 16 + I + 4 * (I // 256)
    res["gate_up_gemv_m1"] = {"ms": ms, "bytes": byts, "GBs": byts / ms / 1e6, "bound": "hbm"}
    del ws

    # prefill gate/up GEMM (M=512): the largest prefill GEMM
    M = 512
    a5, as5 = t8(M, H), tf(M, H // 256)
    wg, wgs, wu, wus = t8(I, H), tf(I), t8(I, H), tf(I)
    s85 = torch.empty((M, I), dtype=torch.int8, device=dev)
    ss5 = torch.empty((M, I // 256), dtype=torch.float32, device=dev)
    ms = time_graph(lambda i: ops.gemm_gate_up_swiglu_quant(a5, as5, wg, wgs, wu, wus, s85, ss5, 256,
                                                            stream=stream), 32, stream)
    flops = 2 * M * (2 * I) * H
    res["gate_up_gemm_m512"] = {"ms": ms, "ops": flops, "TOPs": flops / ms / 1e9, "bound": "mfma"}
    return res


# the per-group int8 GEMM with f32 output and residual add
# over M x (K, N, group) (Q, K+V, gate+up, down, O).
CFG1_SHAPES = [(1024, 2048, 256, "Q"), (1024, 1024, 256, "K+V"), (1024, 6144, 256, "gate+up"),
               (3072, 1024, 256, "down"), (2048, 1024, 128, "O")]
CFG1_M = [1, 32, 512, 2048]
CFG1_ROTATE_BYTES = 1 << 30  # every launch reads operands the 256 MB MALL does not hold


def cfg1_bytes(M: int, K: int, N: int, group: int, per_group: bool) -> int:
    """Algorithmic HBM bytes of one launch: weights and their scales, the A
    operand and its per-group scales, the residual read and the result
    written (f32)."""
    ng = K // group
    return N * K + 4 * N * (ng if per_group else 1) + M * K + 4 * M * ng + 8 * M * N


def run_cfg1(stream, reps_min: int = 64) -> dict:
    """Times q3_gemm_nt_group_store with the residual epilogue on every
    config-1 shape, with per-row and with per-(row, group) B scales.  Each
    (shape, M) rotates over enough operand sets (weights, scales, A, x) that
    the launches stream >= 1 GiB of distinct data, so the last-level cache
    cannot serve repeated reads; HIP events on the launch stream give the
    average launch time (the launches replayed from one HIP graph, so that
    host submission does not pace them).  Reported against the attainable bound
    min(int8 peak, arithmetic intensity x HBM peak)."""
    import torch
    from q3ops import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED0001)
    rows = []
    for K, N, group, name in CFG1_SHAPES:
        ng = K // group
        for M in CFG1_M:
            per_set = cfg1_bytes(M, K, N, group, True)
            R = max(2, min(1024, -(-CFG1_ROTATE_BYTES // per_set)))
            with torch.cuda.stream(stream):
                B = torch.randint(-127, 128, (R, N, K), dtype=torch.int8, device=dev, generator=gen)
                A = torch.randint(-127, 128, (R, M, K), dtype=torch.int8, device=dev, generator=gen)
                AS = torch.rand((R, M, ng), device=dev, generator=gen) * 0.099 + 1e-3
                BS = torch.rand((R, N, 1), device=dev, generator=gen) * 0.099 + 1e-3
                BSG = torch.rand((R, N, ng), device=dev, generator=gen) * 0.099 + 1e-3
                X = torch.randn((R, M, N), device=dev, generator=gen)
            stream.synchronize()
            for per_group in (False, True):
                scales = BSG if per_group else BS

                def launch(j):
                    i = j % R
                    ops.gemm_nt_group_store(A[i], AS[i], B[i], scales[i], None, group, add=X[i],
                                            stream=stream)

                ms = time_graph(launch, max(reps_min, R), stream)
                byts = cfg1_bytes(M, K, N, group, per_group)
                ops_n = 2 * M * N * K
                tops = ops_n / ms / 1e9
                gbs = byts / ms / 1e6
                bound_tops = min(INT8_PEAK_TOPS, ops_n / byts * HBM_PEAK_GBS / 1e3)
                rows.append({"shape": name, "M": M, "K": K, "N": N, "group": group,
                             "b_scale": "row+group" if per_group else "row", "us": ms * 1e3,
                             "TOPs": tops, "GBs": gbs, "bytes": byts,
                             "bound": "hbm" if bound_tops < INT8_PEAK_TOPS else "mfma",
                             "frac_of_attainable": tops / bound_tops,
                             "frac_of_int8_peak": tops / INT8_PEAK_TOPS,
                             "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "rotated_sets": R})
            del A, AS, B, BS, BSG, X
            torch.cuda.empty_cache()
    return {"workload": ("config 1: q3_gemm_nt_group_store with residual add, int8 U[-127,127] "
                         "operands, scales U(1e-3,1e-1), x N(0,1); operand sets rotated over "
                         ">= 1 GiB"), "shapes": rows}


# Algorithmic HBM bytes of one launch of each decode kernel class (model
# shape of the workload): every operand read once, every result written once.
# ofused: the O projection runs inside the attention kernel (per-head f32
# partials, NH x H, written there and read by the gate/up and down GEMVs).
def decode_class_bytes(name: str, kv_len: int, ofused: bool = True, qkv_fused: bool = False,
                       merged: float = 0.0) -> int:
    """Algorithmic HBM bytes of one launch of a decode kernel class at
    kv_len keys.  qkv_fused: the attention launch also runs the Q|K|V
    projection; merged: the fraction of attention launches that also run
    the previous layer's down projection."""
    H, QW, KW, KVH, NH, I, V = 1024, 2048, 1024, 8, 16, 3072, 151936
    part = NH * H * 4 if ofused else 0
    if name == "attn_decode":
        kv_rows = kv_len * (2 * KW + 2 * KVH * 4)       # K, V rows + per-head scales
        ins = (QW + 2 * KW) * 4 + 2 * 128 * 4 + 2 * 64 * 4  # f32 q|k|v rows, q/k gains, cos/sin
        outs = (QW + NH * 4) * 2 + 2 * (KW + KVH * 4)  # q8/qs + o8/os, new K/V rows + scales
        o = (H * QW + 4 * H) + part if ofused else 0   # Wo and its scales, the partials
        qkv = decode_class_bytes("gemv_qkv", kv_len) - 4 * (QW + 2 * KW) if qkv_fused else 0  # (rows counted in ins)
        down = merged * decode_class_bytes("gemv_down", kv_len, ofused)
        return int(kv_rows + ins + outs + o + qkv + down)
    if name == "gemv_qkv":     # RMSNorm prologue (x, gain) + Q|K|V weights, f32 outputs
        N = QW + 2 * KW
        return N * H + 4 * N + 2 * 4 * H + 4 * N + (H + 4 * H + 16)
    if name == "gemv_o":       # o8/os + Wo + residual read/write
        return H * QW + 4 * H + QW + 4 * NH + 2 * 4 * H
    if name == "gemv_gate_up":  # prologue (x, gain, O partials) + Wg, Wu + f32 SwiGLU row
        return 2 * I * H + 8 * I + 2 * 4 * H + 4 * I + (H + 4 * H + 16) + part
    if name == "gemv_down":    # f32 SwiGLU row + Wd + residual read/write (+ s8/ss stage, O partials)
        return 4 * I + H * I + 4 * H + 2 * 4 * H + I + 4 * (I // 256) + part
    if name == "lm_head":      # prologue + lm weights and scales (+ keys)
        return V * H + 4 * V + 2 * 4 * H + 8 * 1024
    raise KeyError(name)


def path_roofline(prefill_ms: float, decode_ms: float) -> dict:
    """The whole prefill and decode against their bounds (model shape of the
    workload).  Prefill: int8 MACs of the 28 layers' GEMMs per token
    (Q 2048x1024, K and V 1024x1024, O 1024x2048, gate/up 2x3072x1024,
    down 1024x3072: 15,728,640 x 28), the causal attention (16 heads x
    (QK + PV) x 128 x 512*513/2 per layer) and one lm_head row, x2 ops per
    MAC, at the dense int8 MFMA peak.  Decode: weights and row scales of the
    28 layers, the lm_head and its scales, and K, V rows plus per-head scales
    (2112 B per layer and position) of every cached position, averaged over
    the generated tokens, at the HBM peak."""
    H, L, V, NH, HD = 1024, 28, 151936, 16, 128
    layer_macs = 2048 * H + 2 * 1024 * H + H * 2048 + 2 * 3072 * H + H * 3072
    attn_macs = L * NH * 2 * HD * (N_PROMPT * (N_PROMPT + 1) // 2)
    prefill_ops = 2 * (N_PROMPT * L * layer_macs + attn_macs + V * H)
    prefill_bound_ms = prefill_ops / (INT8_PEAK_TOPS * 1e9)
    layer_scale_bytes = 4 * (2048 + 1024 + 1024 + 1024 + 2 * 3072 + 1024)
    weights = L * (layer_macs + layer_scale_bytes) + V * H + 4 * V
    kv = [L * 2112 * (N_PROMPT + i + 1) for i in range(N_GEN)]
    decode_bytes = weights + sum(kv) / len(kv)
    decode_bound_ms = decode_bytes / (HBM_PEAK_GBS * 1e6)
    return {
        "prefill": {"bound": "mfma", "ops": prefill_ops, "bound_ms": prefill_bound_ms,
                    "frac": prefill_bound_ms / prefill_ms},
        "decode": {"bound": "hbm", "bytes_per_token": decode_bytes, "bound_ms_per_token": decode_bound_ms,
                   "frac": decode_bound_ms / decode_ms},
    }


def attn_prefetch_bytes(kv_len: int, last_layer: bool, ofused: bool = True) -> int:
    """Bytes the attention kernel's prefetch workgroups read per launch
    (q3_model.hip): this layer's gate, up, down weights (and O unless the
    attention computes the O projection itself), the next layer's Q, K, V
    (and O when fused) weights (not after the last layer), and the K/V pages
    and scales of the next attention."""
    H, QW, KW, KVH, I = 1024, 2048, 1024, 8, 3072
    b = 2 * I * H + H * I + (0 if ofused else H * QW)
    if not last_layer:
        b += (QW + 2 * KW) * H + (H * QW if ofused else 0)
    pages = (kv_len + (1 if last_layer else 0) + 31) // 32
    return b + pages * (2 * 32 * KW + 2 * 32 * KVH * 4)


CFG4_SEQS, CFG4_CTX, CFG4_STEPS = 64, 2048, 32
CFG4_PAGES_PER_SEQ = (CFG4_CTX + CFG4_STEPS + 31) // 32   # 65: contexts + the 32 new rows
KV_BYTES_PER_TOKEN = 2 * 1024 + 2 * 8 * 4               # K and V rows + per-head scales


def cfg4_attn_bytes(kv_lens) -> int:
    """Batched attention launch: every row's K/V pages and scales, its q8/qs
    row in and o8/os row out."""
    QW, NH = 2048, 16
    return sum(int(k) * KV_BYTES_PER_TOKEN for k in kv_lens) + len(kv_lens) * 2 * (QW + 4 * NH)


def cfg4_fill_kv(m, lay, seed: int) -> None:
    """Every K/V row of the pool: N(0,1) values quantised per 128-wide head
    (scale = max|x| * (1/127), round half to even), written straight into the
    device blob (torch is only the generator here)."""
    import torch
    o = lay.offsets
    MS, KW, NKV, HD = lay.max_seq, lay.kv_width, lay.kv_heads, lay.head_dim
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    inv127 = torch.tensor(1.0 / 127.0, dtype=torch.float32, device="cuda")
    chunk = 8192
    for li in range(lay.layers):
        base = o["kKV_BASE"] + li * o["kKV_STRIDE"]
        for off in (0, o["kKV_VOFF"]):
            q_dst = m.blob[base + off:base + off + MS * KW].view(torch.int8).view(MS, KW)
            so = base + off + o["kKV_SOFF"]
            s_dst = m.blob[so:so + 4 * MS * NKV].view(torch.float32).view(MS, NKV)
            for t0 in range(0, MS, chunk):
                t1 = min(MS, t0 + chunk)
                x = torch.randn(t1 - t0, NKV, HD, device="cuda", generator=gen)
                sc = x.abs().amax(-1) * inv127
                q = torch.round(x / sc[..., None]).clamp_(-127, 127).to(torch.int8)
                q_dst[t0:t1] = q.view(t1 - t0, KW)
                s_dst[t0:t1] = sc
    torch.cuda.synchronize()


def cfg4_cpu_check(blob, lay, m, tables, ids0, gpu_ids, sample: int, steps: int,
                   threads: int) -> dict:
    """Oracle on a bounded sample of the batch: `sample` sequences, `steps`
    greedy steps each from their 2048-token contexts (read back from the
    device pool through their tables).  Timed (the forwards only) as the CPU
    baseline and compared with the GPU's ids for the same rows and steps."""
    import numpy as np
    import oracle
    o = lay.offsets
    MS, KW, NKV = lay.max_seq, lay.kv_width, lay.kv_heads
    dims = dict(lay.shape.__dict__)
    dims["max_seq"] = (CFG4_CTX + steps + 31) // 32 * 32
    oracle.set_threads(threads)
    om = oracle.OracleModel(blob, o, dims)
    import torch
    got, dt = [], 0.0
    for r in range(sample):
        om.reset_cache()
        pages = torch.from_numpy(tables[r, :CFG4_CTX // 32].astype(np.int64)).cuda()
        for li in range(lay.layers):
            base = o["kKV_BASE"] + li * o["kKV_STRIDE"]
            for dst_q, dst_s, off in ((om.k8, om.k_s, 0), (om.v8, om.v_s, o["kKV_VOFF"])):
                pool_q = m.blob[base + off:base + off + MS * KW].view(torch.int8).view(MS // 32, 32, KW)
                so = base + off + o["kKV_SOFF"]
                pool_s = m.blob[so:so + 4 * MS * NKV].view(torch.float32).view(MS // 32, 32, NKV)
                dst_q[li, :CFG4_CTX] = pool_q[pages].reshape(CFG4_CTX, KW).cpu().numpy()
                dst_s[li, :CFG4_CTX] = pool_s[pages].reshape(CFG4_CTX, NKV).cpu().numpy()
        tok = int(ids0[r])
        seq = []
        for st in range(steps):
            t0 = time.perf_counter()
            logits, _ = om.forward_chunk(np.array([tok], np.int32), CFG4_CTX + st, 1, True)
            dt += time.perf_counter() - t0
            tok = oracle.argmax_logits(logits)
            seq.append(tok)
        got.append(seq)
    exp = [[int(gpu_ids[st][r]) for st in range(steps)] for r in range(sample)]
    mism = [r for r in range(sample) if got[r] != exp[r]]
    return {"value": steps * sample / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"{sample} of the {CFG4_SEQS} sequences x {steps} greedy steps from their "
                       f"{CFG4_CTX}-token contexts, one row at a time: oracle/ C port of "
                       f"tools/ref_qwen3.py, {dt:.1f} s, {threads} OpenMP threads"),
            "matches_gpu_ids": not mism, "mismatched_rows": mism}


def run_cfg4(args) -> dict:
    """Batched paged decode: 64 independent sequences, each with a random
    2048-token context in its own 64 pages (plus one page for the new rows),
    32 greedy steps of all 64 rows through q3_decode_batch.  One bench step =
    those 32 decode steps from the same contexts and first ids (each step
    rewrites the rows at positions 2048..2079)."""
    import numpy as np
    import torch
    from q3ops.layout import InitConfig, Layout, ModelShape, init_random_blob
    from q3ops.model import Model

    n_pages = CFG4_SEQS * CFG4_PAGES_PER_SEQ
    shape = ModelShape(seq=CFG4_SEQS, max_seq=n_pages * 32)
    lay = Layout(shape)
    log(f"cfg4: writing random-init blob ({lay.size / 1e9:.2f} GB) ...")
    blob = init_random_blob(lay, InitConfig(n_prompt=1, n_gen=0, mode=0))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        m = Model(lay, blob, stream=stream)
    log("cfg4: filling the K/V pools ...")
    cfg4_fill_kv(m, lay, seed=0x5EED0004)
    rng = np.random.default_rng(0x5EED0004)
    tables = rng.permutation(n_pages).astype(np.uint16).reshape(CFG4_SEQS, CFG4_PAGES_PER_SEQ)
    ids0 = rng.integers(0, lay.vocab, size=CFG4_SEQS).astype(np.int32)
    ids_a = torch.empty(CFG4_SEQS, dtype=torch.int32, device="cuda")
    ids_b = torch.empty_like(ids_a)
    ids_init = torch.from_numpy(ids0).cuda()
    hist = [torch.empty_like(ids_a) for _ in range(CFG4_STEPS)]
    pos = [np.full(CFG4_SEQS, CFG4_CTX + s, np.int32) for s in range(CFG4_STEPS)]

    def one_step():
        with torch.cuda.stream(stream):
            ids_a.copy_(ids_init)
        cur, nxt = ids_a, ids_b
        for s in range(CFG4_STEPS):
            m.decode_batch(cur, pos[s], tables, nxt)
            with torch.cuda.stream(stream):
                hist[s].copy_(nxt)
            cur, nxt = nxt, cur

    torch.cuda.synchronize()
    log("cfg4: warmup ...")
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    log(f"cfg4: timing {args.steps} steps ...")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    gpu_ids = [h.cpu().numpy() for h in hist[:4]]
    tokens = CFG4_SEQS * CFG4_STEPS
    weight_bytes = 441_778_176 + 156_190_208
    kv_step = sum(CFG4_CTX + 1 + s for s in range(CFG4_STEPS)) / CFG4_STEPS
    step_bytes = weight_bytes + shape.layers * CFG4_SEQS * kv_step * KV_BYTES_PER_TOKEN
    out = {
        "metric": "tok/s batched paged decode (64 seq x 2048 ctx, 32 steps), Qwen3-0.6B W8A8, 1 MI355X",
        "value": tokens / dt, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": dt * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": ("synthetic (random-init weights N(0,0.02) int8 per-row; K/V N(0,1) int8 per head; "
                 "random page tables; uniform first ids)"),
        "config": {"workload": "cfg4: 28-layer Qwen3-0.6B shape, 64 independent sequences x "
                               "2048-token contexts, 32 batched greedy decode steps (M=64)",
                   "sequences": CFG4_SEQS, "context": CFG4_CTX, "decode_steps": CFG4_STEPS,
                   "pages": n_pages, "max_seq": shape.max_seq},
        "ms_per_decode_step": dt * 1e3 / CFG4_STEPS,
        "hbm_bound_ms_per_decode_step": step_bytes / (HBM_PEAK_GBS * 1e6),
        "step_frac_of_hbm_bound": (step_bytes / (HBM_PEAK_GBS * 1e6)) / (dt * 1e3 / CFG4_STEPS),
        "first_ids": [int(v) for v in gpu_ids[0][:8]],
    }
    if not args.no_roofline:
        log("cfg4: attention timing pass ...")
        m.set_kernel_timing(True)
        one_step()
        kt = m.kernel_times()
        m.set_kernel_timing(False)
        tot_ms, n = kt["attn_decode"]
        byts = sum(cfg4_attn_bytes([CFG4_CTX + 1 + s] * CFG4_SEQS)
                   for s in range(CFG4_STEPS)) / CFG4_STEPS
        avg = tot_ms / max(n, 1)
        gbs = byts / avg / 1e6
        out["roofline"] = {"kernel": "attn_decode (batched)", "bound": "hbm", "achieved": gbs,
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                           "traffic": None, "avg_us": avg * 1e3, "bytes_per_launch": int(byts),
                           "launches": n, "share_of_step": tot_ms / (dt * 1e3)}
    if not args.no_cpu:
        threads = args.cpu_threads or host_cores()[0]
        log(f"cfg4: cpu check ({threads} threads) ...")
        out["cpu_check"] = cfg4_cpu_check(blob, lay, m, tables, ids0, gpu_ids, CFG4_SEQS, 4,
                                          threads)
    m.close()
    return out


def load_pmc_traffic() -> dict:
    """Per-kernel HBM bytes per dispatch from the committed rocprofv3 PMC
    summary (profiles/pmc_traffic.json), if present."""
    p = REPO / "profiles" / "pmc_traffic.json"
    if not p.exists():
        return {}
    try:
        return json.loads(p.read_text()).get("kernels", {})
    except (OSError, ValueError):
        return {}


def host_cores() -> tuple[int, int]:
    """(threads used, nproc): nproc is the CPUs this process may run on; a
    GPU box shares its host, and one GPU's share is 16 CPUs, so at most 16
    OpenMP threads are used there whatever nproc reports."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return min(16, nproc), nproc


def shuffled_table_run(m, lay, steps: int, stream, ref_ids) -> dict:
    """The cfg3 workload with the pages in a random order instead of the
    default reversed table (main_big.cpp:168-171), then the default
    restored: step, prefill and decode times, and whether the ids match."""
    import numpy as np
    import torch
    from q3ops import LM_ARGMAX

    n = lay.max_seq // 32
    tab = np.random.default_rng(11).permutation(n).astype(np.uint16)
    m.set_page_table(tab)
    m.generate()  # warm: the decode graph is captured anew for the new table
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.generate()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    ids = m.ids()[N_PROMPT:N_PROMPT + N_GEN]
    prefill = time_events(lambda: m.forward_chunk(0, N_PROMPT, LM_ARGMAX, True), steps, stream)
    m.set_page_table((n - 1 - np.arange(n)).astype(np.uint16))
    m.generate()
    torch.cuda.synchronize()
    return {"table": f"random permutation of the {n} pages (seed 11)", "steps": steps,
            "ms_per_step": dt * 1e3, "prefill_ms": prefill,
            "decode_ms_per_token": (dt * 1e3 - prefill) / N_GEN,
            "same_ids": bool(np.array_equal(np.asarray(ids), np.asarray(ref_ids)))}


def cpu_baseline(threads: int, nproc: int, runs: int = 5) -> dict:
    """The CPU oracle (oracle/, the C port of tools/ref_qwen3.py) on the same
    workload: the median of `runs` timed generations on `threads` OpenMP
    threads after one untimed warm run, and a 1-thread line on the same
    workload (512-token prefill + 64 greedy steps, one run of ~25 s; the
    threaded runs warmed the caches)."""
    import numpy as np
    import oracle
    from q3ops.layout import CONFIGS, Layout, init_random_blob

    shape, init = CONFIGS["cfg3_perf"]
    lay = Layout(shape)
    blob = init_random_blob(lay, init)
    om = oracle.OracleModel(blob, lay.offsets, dict(shape.__dict__))
    ids = lay.global_views(blob)["ids"]

    def timed(n_prompt, n_gen, reps, warm=True):
        out, ts = None, []
        for _ in range(reps + (1 if warm else 0)):  # a first run warms caches and pages
            om.reset_cache()
            t0 = time.perf_counter()
            _, gen, _, _ = om.generate(ids, n_prompt, n_gen, record=False)
            ts.append(time.perf_counter() - t0)
            out = gen
        ts = ts[1:] if warm else ts
        return sorted(ts)[len(ts) // 2], ts, out

    oracle.set_threads(threads)
    med, ts, gen = timed(N_PROMPT, N_GEN, runs)
    oracle.set_threads(1)
    med1, ts1, gen1 = timed(N_PROMPT, N_GEN, 1, warm=False)
    oracle.set_threads(threads)
    assert np.array_equal(np.asarray(gen1), np.asarray(gen)), "1-thread oracle run differs"
    return {"value": (N_PROMPT + N_GEN) / med, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"the full workload (512-token prefill + 64 greedy decode steps), median of "
                       f"{runs} runs ({med:.2f} s) after a warm run: oracle/ C port of "
                       f"tools/ref_qwen3.py on {threads} OpenMP threads (nproc {nproc}; one GPU's "
                       f"share of the box is 16 CPUs)"),
            "nproc": nproc, "runs_s": [round(t, 3) for t in ts],
            "one_thread": {"value": (N_PROMPT + N_GEN) / med1, "unit": "tok/s", "cores": 1,
                           "sample": (f"the same workload (512-token prefill + 64 greedy decode "
                                      f"steps), one run ({med1:.2f} s) on 1 thread after the "
                                      f"threaded runs; same generated ids"),
                           "runs_s": [round(t, 3) for t in ts1]},
            "generated": [int(v) for v in np.asarray(gen)]}


ENGINE_REQS, ENGINE_PROMPT, ENGINE_GEN = 32, 256, 64


def run_engine(args) -> dict:
    """The continuous-batching engine (q3ops.engine, tools/engine.py) on the
    28-layer shape: ENGINE_REQS requests of ENGINE_PROMPT uniform prompt ids,
    ENGINE_GEN greedy ids each, batches of at most 32 rows (prefill chunks of
    32 first, then one row per decoding request), one shared page pool.  One
    bench step = admitting every request and running the engine until all
    have finished; the host scheduler and page bookkeeping are inside the
    timed region."""
    import numpy as np
    import torch
    from q3ops.engine import SamplingParams, make_gpu_engine
    from q3ops.layout import InitConfig, Layout, ModelShape, init_random_blob
    from q3ops.model import Model

    per_req = -(-(ENGINE_PROMPT + ENGINE_GEN) // 32)
    shape = ModelShape(seq=32, max_seq=ENGINE_REQS * per_req * 32)
    lay = Layout(shape)
    log(f"engine: writing random-init blob ({lay.size / 1e9:.2f} GB) ...")
    blob = init_random_blob(lay, InitConfig(n_prompt=1, n_gen=0, mode=0))
    m = Model(lay, blob)
    rng = np.random.default_rng(0x5EED0005)
    prompts = [[int(t) for t in rng.integers(0, lay.vocab, size=ENGINE_PROMPT)]
               for _ in range(ENGINE_REQS)]

    def one_step():
        eng = make_gpu_engine(m)
        for p in prompts:
            eng.add_request(p, SamplingParams(max_new=ENGINE_GEN))
        eng.run(max_steps=100000)
        return eng

    torch.cuda.synchronize()
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    log(f"engine: timing {args.steps} steps ...")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng = one_step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    outs = eng.outputs()
    assert all(len(v) == ENGINE_GEN for v in outs.values())
    assert eng.pool.free_pages == eng.pool.num_pages
    fed = ENGINE_REQS * (ENGINE_PROMPT + ENGINE_GEN - 1)
    gen = ENGINE_REQS * ENGINE_GEN
    return {
        "metric": "tok/s continuous-batching engine (32 req x 256 prompt + 64 greedy), "
                  "Qwen3-0.6B W8A8, 1 MI355X",
        "value": fed / dt, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": dt * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (random-init weights N(0,0.02) int8 per-row; uniform prompt ids)",
        "config": {"workload": "engine: q3ops.engine over q3_forward_chunk (32-row prefill "
                               "chunks) and q3_decode_batch (greedy rows), 28-layer shape",
                   "requests": ENGINE_REQS, "prompt": ENGINE_PROMPT, "generated": ENGINE_GEN,
                   "max_rows": 32, "pages": eng.pool.num_pages},
        "generated_tok_s": gen / dt, "engine_batches": eng.steps,
        "launches": dict(eng.guest_step.launches),
        "first_ids": outs[0][:8],
    }


def run_prefill(args) -> dict:
    """Config 3's prefill alone: the 512-token chunk through
    q3_forward_chunk with the fused lm_head+argmax of its last row, as
    q3_generate runs it; `steps` chunks timed with HIP events on the model's
    stream (the workload profiled for the prefill kernels' counters)."""
    import torch
    from q3ops import LM_ARGMAX
    from q3ops.layout import CONFIGS, Layout, init_random_blob
    from q3ops.model import Model

    shape, init = CONFIGS["cfg3_perf"]
    lay = Layout(shape)
    blob = init_random_blob(lay, init)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        m = Model(lay, blob, stream=stream)
    for _ in range(args.warmup):
        m.forward_chunk(0, N_PROMPT, LM_ARGMAX, True)
    torch.cuda.synchronize()
    ms = time_events(lambda: m.forward_chunk(0, N_PROMPT, LM_ARGMAX, True), args.steps, stream)
    best, idx = m.argmax()
    m.close()
    pr = path_roofline(ms, 1.0)["prefill"]
    return {"metric": "tok/s prefill (one 512-token chunk), Qwen3-0.6B W8A8, 1 MI355X",
            "value": N_PROMPT / (ms / 1e3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8",
            "data": "synthetic (random-init weights N(0,0.02) int8 per-row, uniform prompt ids)",
            "config": {"workload": "cfg3 prefill: 28-layer Qwen3-0.6B shape, one 512-token chunk "
                                   "with the fused lm_head+argmax of the last row"},
            "path_roofline": pr, "argmax": [float(best), idx]}


def calib_copies(mib: int) -> int:
    """Three device-to-device copies of `mib` MiB: the known-size kernel the
    PMC byte counters are scaled by.  Returns the bytes of one copy."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return n


def run_decode(args) -> dict:
    """Config 3's b = 1 decode launches alone, eagerly (no decode graph):
    the 512-token prefill, then `warmup` + `steps` single-token
    q3_forward_chunk calls at positions 512, 513, ... with the fused
    lm_head+argmax, each synchronised and reported on stderr; the steps
    timed with HIP events.  The workload profiled for the decode kernels'
    counters (every launch of a step is its own dispatch)."""
    import torch
    from q3ops import LM_ARGMAX
    from q3ops.layout import CONFIGS, Layout, init_random_blob
    from q3ops.model import Model

    shape, init = CONFIGS["cfg3_perf"]
    lay = Layout(shape)
    blob = init_random_blob(lay, init)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        m = Model(lay, blob, stream=stream)
    m.forward_chunk(0, N_PROMPT, LM_ARGMAX, True)
    m.synchronize()
    log("prefill done")
    pos = N_PROMPT
    for i in range(args.warmup):
        m.forward_chunk(pos, 1, LM_ARGMAX, True)
        m.synchronize()
        log(f"warmup token {i} done")
        pos += 1
    total = 0.0
    for i in range(args.steps):
        total += time_events(lambda: m.forward_chunk(pos, 1, LM_ARGMAX, True), 1, stream)
        log(f"token {i} done")
        pos += 1
    fused, gave_up = m.fused_status()
    m.close()
    ms = total / max(1, args.steps)
    return {"metric": "ms per b=1 decode token (eager), Qwen3-0.6B W8A8, 1 MI355X",
            "value": ms, "unit": "ms/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8", "data": "synthetic (random-init weights N(0,0.02) int8 per-row)",
            "config": {"workload": f"cfg3 decode: 28-layer Qwen3-0.6B shape, tokens at {N_PROMPT}.. "
                                   "after a 512-token prefill, one q3_forward_chunk each"},
            "fused_status": [fused, gave_up]}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-cfg1", action="store_true", help="skip the config 1 GEMM sweep leg")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the config 4 batched-decode leg")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="finish with 3 device-to-device copies of MIB MiB (PMC calibration)")
    ap.add_argument("--workload", choices=("cfg3", "cfg4", "engine", "prefill", "decode", "cfg1"), default="cfg3",
                    help="cfg3: 512-token prefill + 64 b=1 decode steps (the headline line); "
                         "cfg4: 64-sequence batched paged decode; engine: continuous batching; "
                         "prefill: the 512-token chunk alone; decode: eager b=1 decode tokens; "
                         "cfg1: the config 1 GEMM sweep alone")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        return 2
    if args.workload == "cfg1":  # the config 1 GEMM sweep alone (for profiling its kernels)
        import torch
        assert torch.cuda.is_available(), "bench.py needs a ROCm device"
        torch.cuda.set_device(0)
        print(json.dumps(run_cfg1(torch.cuda.Stream())), flush=True)
        return 0
    if args.workload in ("cfg4", "engine", "prefill", "decode"):
        import torch
        assert torch.cuda.is_available(), "bench.py needs a ROCm device"
        torch.cuda.set_device(0)
        run = {"cfg4": run_cfg4, "engine": run_engine, "prefill": run_prefill,
               "decode": run_decode}[args.workload]
        res = run(args)
        if "cpu_check" in res:  # the standalone cfg4 line reports it as its CPU baseline
            res["cpu_baseline"] = res.pop("cpu_check")
        if args.calib_copy > 0:
            res["calib_copy_bytes"] = calib_copies(args.calib_copy)
        print(json.dumps(res), flush=True)
        return 0

    import numpy as np
    import torch
    from q3ops import LM_ARGMAX
    from q3ops.layout import CONFIGS, Layout, init_random_blob
    from q3ops.model import Model

    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    torch.cuda.set_device(0)
    shape, init = CONFIGS["cfg3_perf"]
    lay = Layout(shape)
    log(f"writing random-init blob ({lay.size / 1e9:.2f} GB) ...")
    blob = init_random_blob(lay, init)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        m = Model(lay, blob, stream=stream)
    m.set_ctrl(N_PROMPT, N_GEN, 0)
    torch.cuda.synchronize()
    log("warmup ...")
    for _ in range(args.warmup):
        m.generate()
    torch.cuda.synchronize()

    log(f"timing {args.steps} steps ...")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.generate()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    gen_ids = m.ids()[N_PROMPT:N_PROMPT + N_GEN]

    # prefill alone (the first chunk of generate), HIP events on the model stream
    prefill_ms = time_events(lambda: m.forward_chunk(0, N_PROMPT, LM_ARGMAX, True),
                             max(3, args.steps), stream)
    step_ms = dt * 1e3
    decode_ms = max(step_ms - prefill_ms, 1e-9) / N_GEN
    out = {
        "metric": METRIC,
        "value": (N_PROMPT + N_GEN) / dt,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init weights N(0,0.02) int8 per-row, uniform prompt ids)",
        "config": {"workload": "cfg3 perf: 28-layer Qwen3-0.6B shape, one 512-token prefill "
                               "chunk + 64 greedy decode steps (b=1), fused lm_head+argmax",
                   "prefill_tokens": N_PROMPT, "decode_tokens": N_GEN, "chunk": shape.seq,
                   "max_seq": shape.max_seq},
        "prefill_ms": prefill_ms,
        "prefill_tok_s": N_PROMPT / (prefill_ms / 1e3),
        "decode_ms_per_token": decode_ms,
        "decode_tok_s": 1e3 / decode_ms,
        "path_roofline": path_roofline(prefill_ms, decode_ms),
        "generated": [int(v) for v in gen_ids],
    }
    # the same workload over a fragmented page table (every logical page at a
    # random physical one): the decode prefetch walks the sequence's pages
    out["shuffled_table"] = shuffled_table_run(m, lay, max(3, args.steps), stream, gen_ids)
    # in-situ kernel timing: one more (untimed) generation with every decode
    # launch bracketed by HIP events on the model's stream
    if not args.no_roofline:
        log("decode kernel timing pass ...")
        m.set_kernel_timing(True)
        m.generate()
        kt = m.kernel_times()
        m.set_kernel_timing(False)
        layers = shape.layers
        # decode step i (0-based) attends over kv_len = N_PROMPT + 1 + i keys
        n_steps = max(1, kt["attn_decode"][1] // layers)
        kv_lens = [N_PROMPT + 1 + i for i in range(n_steps)]
        ofused = kt.get("gemv_o", (0.0, 0))[1] == 0  # no O GEMV launches: fused
        qkv_fused = kt.get("gemv_qkv", (0.0, 0))[1] == 0  # no Q|K|V GEMV launches: in the attention's
        # the attention launches that also ran the previous layer's down projection
        merged = max(0.0, 1.0 - kt.get("gemv_down", (0.0, 0))[1] / max(1, kt["attn_decode"][1]))
        classes = {}
        for name, (tot_ms, n) in kt.items():
            if n == 0:
                continue
            if name == "lm_head":
                byts = decode_class_bytes(name, 0)
            else:
                byts = sum(decode_class_bytes(name, kv, ofused, qkv_fused, merged)
                           for kv in kv_lens) / len(kv_lens)
            avg = tot_ms / n
            classes[name] = {"launches": n, "avg_us": avg * 1e3, "total_ms": tot_ms,
                             "bytes_per_launch": int(byts), "GBs": byts / avg / 1e6}
        dec_total = sum(c["total_ms"] for c in classes.values())
        for c in classes.values():
            c["share_of_timed"] = c["total_ms"] / dec_total if dec_total else 0.0
        out["decode_kernels"] = classes
        dom_name = max(classes, key=lambda k: classes[k]["total_ms"])
        dom = classes[dom_name]
        pmc = load_pmc_traffic().get(dom_name)
        pf = None
        if dom_name == "attn_decode":
            pf = sum(attn_prefetch_bytes(kv, l == layers - 1, ofused)
                     for kv in kv_lens for l in range(layers)) / (len(kv_lens) * layers)
        out["roofline"] = {"kernel": dom_name, "bound": "hbm", "achieved": dom["GBs"],
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["GBs"] / HBM_PEAK_GBS,
                           "traffic": (pmc or {}).get("bytes_per_dispatch"),
                           "avg_us": dom["avg_us"], "bytes_per_launch": dom["bytes_per_launch"],
                           "launches": dom["launches"], "layers": layers}
        if pf is not None:
            # traffic counts the prefetch workgroups' reads too (next kernels' weights and KV)
            out["roofline"]["traffic_prefetch"] = int(pf)
    m.close()
    del m
    torch.cuda.synchronize()

    if not args.no_roofline:
        log("kernel rooflines ...")
        out["kernels"] = kernel_rooflines(stream)
    if not args.no_cfg1:
        log("config 1 GEMM sweep ...")
        out["cfg1"] = run_cfg1(stream)
    if not args.no_cfg4:
        log("config 4 batched decode ...")
        c4 = run_cfg4(args)
        out["cfg4"] = {k: c4[k] for k in ("value", "unit", "ms_per_step", "ms_per_decode_step",
                                          "hbm_bound_ms_per_decode_step", "step_frac_of_hbm_bound",
                                          "config", "first_ids") if k in c4}
        for k in ("roofline", "cpu_check"):
            if k in c4:
                out["cfg4"][k] = c4[k]
    if not args.no_cpu:
        threads, nproc = host_cores()
        threads = args.cpu_threads or threads
        log(f"cpu baseline ({threads} threads) ...")
        cb = cpu_baseline(threads, nproc)
        cb_gen = cb.pop("generated")
        cb["matches_gpu_ids"] = cb_gen == [int(v) for v in gen_ids]
        cb["ids_compared"] = len(cb_gen)
        out["cpu_baseline"] = cb
    if args.calib_copy > 0:
        out["calib_copy_bytes"] = calib_copies(args.calib_copy)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
