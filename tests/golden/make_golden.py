#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from the reference's numpy
mirror (tools/ref_qwen3.py, tools/pqwf.py, tools/convert_pqwf.py).

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py [--reference /root/reference] [--skip-full]

numpy's float32 exp2 depends on its SIMD dispatch; NPY_DISABLE_CPU_FEATURES
is set below, before numpy is imported, so that np.exp2 reduces to glibc
exp2f.  The script verifies that on a large sample and records the result,
the numpy and glibc versions in meta.json.

Fixtures (data only: inputs and expected outputs):
  layout.json        pqwf.Layout offsets for several shapes + header text
  exp.npz            exp_f32 inputs/outputs
  ops.npz            gemm_nt_group / quant_rows_heads / swiglu / attention on
                     the closed-form inputs of the reference's guest tests
  cfg0.npz           config 0 (1 layer, vocab 1024, 40+2 tokens), per stage
  cfg2.npz           config 2 (28 layers, 32-token prefill, full logits)
  cfg3.npz           config 3 parity (15-token prompt, 6 greedy tokens)
"""
from __future__ import annotations

import os

os.environ["NPY_DISABLE_CPU_FEATURES"] = (
    "AVX512_SKX AVX512_CLX AVX512_CNL AVX512_ICL AVX512_SPR AVX512F AVX512CD")
os.environ.setdefault("OMP_NUM_THREADS", "8")

import argparse  # noqa: E402
import ctypes  # noqa: E402
import hashlib  # noqa: E402
import json  # noqa: E402
import platform  # noqa: E402
import sys  # noqa: E402
import tempfile  # noqa: E402
import time  # noqa: E402
from pathlib import Path  # noqa: E402

import numpy as np  # noqa: E402

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO / "qwen3-tile-ops_amd"))

from q3ops.layout import (CONFIGS, InitConfig, Layout, ModelShape,  # noqa: E402
                          init_normal, init_random_blob, stream_id)

F = np.float32


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load_reference(root: Path):
    sys.path.insert(0, str(root / "tools"))
    import ref_qwen3 as ref  # noqa: E402
    import pqwf  # noqa: E402
    import convert_pqwf  # noqa: E402
    return ref, pqwf, convert_pqwf


# --------------------------------------------------------------------------
def exp2_pin_check(n: int = 20_000_000) -> dict:
    """np.exp2 (float32, pinned dispatch) against glibc exp2f."""
    libm = ctypes.CDLL("libm.so.6")
    libm.exp2f.restype = ctypes.c_float
    libm.exp2f.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(7)
    x = rng.uniform(-160.0, 130.0, size=n).astype(F)
    got = np.exp2(x)
    # glibc over the same inputs through a tiny C loop is too slow via ctypes
    # for 2e7 values; use numpy's vectorised call on a subsample plus ctypes.
    idx = rng.choice(n, size=200_000, replace=False)
    ref = np.array([libm.exp2f(float(v)) for v in x[idx]], dtype=F)
    bad = int(np.count_nonzero(got[idx].view(np.uint32) != ref.view(np.uint32)))
    return {"sample": int(idx.size), "mismatches": bad}


def make_exp(ref) -> dict:
    rng = np.random.default_rng(11)
    xs = [rng.uniform(-110.0, 0.0, 10000), rng.uniform(-5.0, 5.0, 4000),
          rng.uniform(-200.0, 100.0, 2000),
          np.array([0.0, -0.0, -np.inf, np.inf, -1e-30, 1e-30, -87.3, 88.7, -103.9, -104.0])]
    x = np.concatenate(xs).astype(F)
    return {"x": x, "y": ref.exp_f32(x)}


def make_ops(ref) -> dict:
    """Reference outputs on the closed-form inputs of tests/guest/*.cpp."""
    out = {}
    # tests/guest/group_gemm.cpp:17-20, 50-58: 32x256, N=128, scales 1.0
    R, K, N = 32, 256, 128
    i = np.arange(R)[:, None]
    j = np.arange(N)[:, None]
    k = np.arange(K)[None, :]
    a = ((i * 7 + k * 3 + 1) % 7 - 3).astype(np.int8)
    b = ((j * 5 + k * 2 + 2) % 5 - 2).astype(np.int8)
    out["gg_a"], out["gg_b"] = a, b
    out["gg_out128"] = ref.gemm_nt_group(a, np.ones((R, 2), F), b, np.ones(N, F), group=128)
    out["gg_out256"] = ref.gemm_nt_group(a, np.ones((R, 1), F), b, np.ones(N, F), group=256)
    # group_gemm.cpp:119-131: x = +/-(1..7) pattern, 32x256, groups of 128
    bits = np.array([0x3F800000, 0x40000000, 0x40400000, 0x40800000, 0x40A00000,
                     0x40C00000, 0x40E00000], np.uint32)
    idx = np.arange(R * K)
    xb = bits[idx % 7] | np.where(idx & 1, np.uint32(0x80000000), np.uint32(0))
    x = xb.astype(np.uint32).view(F).reshape(R, K)
    out["qh_x"] = x
    out["qh_q"], out["qh_s"] = ref.quant_rows_heads(x, 128)
    # tests/guest/gate_up.cpp:30-65: 32x512 A, 256x512 gate/up, sb scales
    R, K, N = 32, 512, 256
    i = np.arange(R)[:, None]
    j = np.arange(N)[:, None]
    k = np.arange(K)[None, :]
    sb = np.array([0x3F800000, 0x3F000000, 0x3E800000, 0x40000000, 0x3F400000],
                  np.uint32).view(F)
    a = ((i * 7 + k * 3 + 1) % 7 - 3).astype(np.int8)
    wg = ((j * 5 + k * 2 + 2) % 5 - 2).astype(np.int8)
    wu = ((j * 3 + k * 7 + 4) % 7 - 3).astype(np.int8)
    gi = np.arange(2)[None, :]
    a_s = sb[(np.arange(R)[:, None] + gi) % 5].astype(F)
    wgs = sb[np.arange(N) % 5].astype(F)
    wus = sb[(np.arange(N) * 3) % 5].astype(F)
    g = ref.gemm_nt_group(a, a_s, wg, wgs, group=256)
    u = ref.gemm_nt_group(a, a_s, wu, wus, group=256)
    sw = ref.swiglu(g, u)
    s8, ss = ref.quant_rows_heads(sw, 256)
    out.update(gu_a=a, gu_as=a_s, gu_wg=wg, gu_wu=wu, gu_wgs=wgs, gu_wus=wus, gu_g=g, gu_u=u,
               gu_sw=sw, gu_s8=s8, gu_ss=ss)
    # tests/guest/paged_attn.cpp + paged_attn_multi.cpp (hd128, 4 heads / 2 kv)
    sb4 = np.array([0x3F800000, 0x3F000000, 0x3E800000, 0x3F400000], np.uint32).view(F)
    H, KVH, HD = 4, 2, 128
    QD, KD = H * HD, KVH * HD
    qk = F(0.08838834764831845)
    cases = [  # (name, q_rows, kv_len, q-pattern, k-pattern, v-pattern, scale patterns)
        ("pa", 4, 80, (7, 3, 1, 7, 3), (5, 2, 2, 5, 2), (3, 7, 4, 7, 3),
         lambda i, h: (i + h) % 4, lambda t, h: (t + h) % 4, lambda t, h: (t * 3 + h) % 4),
        ("pm1", 8, 48, (5, 2, 2, 5, 2), (3, 5, 1, 7, 3), (7, 3, 2, 5, 2),
         lambda i, h: (i * 2 + h) % 4, lambda t, h: (t * 2 + h) % 4,
         lambda t, h: (t * 5 + h) % 4),
    ]
    for name, QR, KVL, qp, kp, vp, qsi, ksi, vsi in cases:
        ii = np.arange(QR)[:, None]
        d = np.arange(QD)[None, :]
        q8 = ((ii * qp[0] + d * qp[1] + qp[2]) % qp[3] - qp[4]).astype(np.int8)
        t = np.arange(KVL)[:, None]
        dk = np.arange(KD)[None, :]
        k8 = ((t * kp[0] + dk * kp[1] + kp[2]) % kp[3] - kp[4]).astype(np.int8)
        v8 = ((t * vp[0] + dk * vp[1] + vp[2]) % vp[3] - vp[4]).astype(np.int8)
        qs = sb4[qsi(np.arange(QR)[:, None], np.arange(H)[None, :])].astype(F)
        ks = sb4[ksi(np.arange(KVL)[:, None], np.arange(KVH)[None, :])].astype(F)
        vs = sb4[vsi(np.arange(KVL)[:, None], np.arange(KVH)[None, :])].astype(F)
        attn = ref.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, H, KVH, HD, True, qk)
        o8, os_ = ref.quant_rows_heads(attn, HD)
        out.update({f"{name}_q8": q8, f"{name}_qs": qs, f"{name}_k8": k8, f"{name}_ks": ks,
                    f"{name}_v8": v8, f"{name}_vs": vs, f"{name}_attn": attn,
                    f"{name}_o8": o8, f"{name}_os": os_})
    # the pa case's first 4 rows of the multi test (paged_attn_multi.cpp:68-70)
    # reuse the pa inputs, so they are covered above.
    return out


def make_layout(pqwf) -> dict:
    shapes = [dict(), dict(layers=1, vocab=1024), dict(seq=512, max_seq=640),
              dict(layers=2, vocab=2048, seq=64, max_seq=4096), dict(layers=28, seq=1, max_seq=4224)]
    res = {"cases": []}
    for kw in shapes:
        lay = pqwf.Layout(**kw).compute()
        mine = Layout(ModelShape(**kw))
        assert mine.offsets == {k: lay.offsets[k] for k in mine.offsets}, kw
        res["cases"].append({"params": kw, "offsets": lay.offsets})
    res["default_header"] = pqwf.Layout().compute().header_text()
    assert Layout().header_text() == res["default_header"]
    return res


def reference_model_from_blob(convert_pqwf, pqwf, blob_path: Path, shape: ModelShape,
                              blob: np.ndarray, mine: Layout):
    lay = pqwf.Layout(hidden=shape.hidden, layers=shape.layers, heads=shape.heads,
                      kv_heads=shape.kv_heads, head_dim=shape.head_dim, inter=shape.inter,
                      vocab=shape.vocab, seq=shape.seq, max_seq=shape.max_seq).compute()
    assert lay.offsets["kSCRATCH_END"] == mine.size
    cos_ref, sin_ref = convert_pqwf.rope_tables(shape.max_seq, shape.head_dim, 1e6)
    gv = mine.global_views(blob)
    rope_ok = (np.array_equal(cos_ref.view(np.uint32), gv["cos"].view(np.uint32))
               and np.array_equal(sin_ref.view(np.uint32), gv["sin"].view(np.uint32)))
    model = convert_pqwf.reference_model(blob_path, lay, gv["cos"].copy(), gv["sin"].copy())
    return model, lay, rope_ok


def writer_pin(pqwf, blob: np.ndarray, mine: Layout, cfg: InitConfig, layer: int = 0) -> dict:
    """Blob weights == pqwf.quantize_rows(the writer's f32 draws)."""
    res = {}
    wv = mine.weight_views(blob, layer)
    H, I, QW, KW = mine.hidden, mine.inter, mine.q_width, mine.kv_width
    shapes = {"wq": (3, QW, H), "wk": (4, KW, H), "wv": (5, KW, H), "wo": (6, H, QW),
              "wg": (7, I, H), "wu": (8, I, H), "wd": (9, H, I)}
    for name, (which, rows, cols) in shapes.items():
        w = init_normal(cfg.weight_seed, stream_id(layer, which), 0, rows * cols, 0.0,
                        cfg.weight_std).reshape(rows, cols)
        q, s = pqwf.quantize_rows(w)
        res[name] = bool(np.array_equal(q, wv[name]) and
                         np.array_equal(s.view(np.uint32), wv[name + "_s"].view(np.uint32)))
    gv = mine.global_views(blob)
    rows = min(mine.vocab, 4096)
    w = init_normal(cfg.weight_seed, stream_id(-1, 0), 0, rows * H, 0.0,
                    cfg.weight_std).reshape(rows, H)
    q, s = pqwf.quantize_rows(w)
    res["emb_first_rows"] = bool(np.array_equal(q, gv["emb8"][:rows]) and np.array_equal(
        s.view(np.uint32), gv["emb_s"][:rows].view(np.uint32)))
    return res


class Snapshots(dict):
    """A record dict that keeps a copy of every forward's last-layer stages."""

    def __init__(self):
        super().__init__()
        self.snaps = []

    def update(self, *args, **kw):  # called once per layer by forward_chunk
        super().update(*args, **kw)
        self.latest = {k: (np.array(v, copy=True) if isinstance(v, np.ndarray) else v)
                       for k, v in dict(*args, **kw).items()}

    def __setitem__(self, key, value):  # record["logits"] = ... ends a forward
        super().__setitem__(key, value)
        if key == "logits":
            snap = dict(self.latest)
            snap["logits"] = np.array(value, copy=True)
            self.snaps.append(snap)


BIG_F32 = ("q", "k", "v", "attn", "o", "g", "u", "sw")


def pack_record(prefix: str, rec: dict, out: dict, full: bool) -> None:
    for k, v in rec.items():
        if k == "layer":
            continue
        v = np.asarray(v)
        if not full and k in BIG_F32:
            out[f"{prefix}{k}_sha"] = np.array(sha(v))
            out[f"{prefix}{k}_last"] = v[-1:].copy()
            out[f"{prefix}{k}_shape"] = np.array(v.shape)
        else:
            out[f"{prefix}{k}"] = v


def run_config(name: str, ref, pqwf, convert_pqwf, tmp: Path) -> tuple[dict, dict]:
    shape, cfg = CONFIGS[name]
    mine = Layout(shape)
    blob = init_random_blob(mine, cfg)
    path = tmp / f"{name}.bin"
    blob.tofile(path)
    model, lay, rope_ok = reference_model_from_blob(convert_pqwf, pqwf, path, shape, blob, mine)
    meta = {"shape": shape.__dict__, "init": cfg.__dict__, "rope_tables_equal_reference": rope_ok,
            "writer_pin_layer0": writer_pin(pqwf, blob, mine, cfg),
            "weights_sha256": sha(blob[mine["kEMB"]:mine["kLOGITS"]])}
    gv = mine.global_views(blob)
    total = cfg.n_prompt + cfg.n_gen
    ids = [int(v) for v in gv["ids"][:total]]
    out = {"ids_in": np.array(ids, np.int32)}
    t0 = time.time()
    # chunk 0 of the prefill on its own (generate records only the forwards
    # that produce logits)
    rows0 = min(shape.seq, cfg.n_prompt)
    if rows0 < cfg.n_prompt:
        caches = ref.new_caches(model)
        rec0 = {}
        ref.forward_chunk(model, np.asarray(ids[:rows0], np.int64), caches, 0, rows0, False, rec0)
        pack_record("c0_", rec0, out, False)
    snaps = Snapshots()
    logits, generated = ref.generate(model, ids, cfg.n_prompt, cfg.n_gen, snaps)
    meta["ref_seconds"] = round(time.time() - t0, 2)
    out["generated"] = np.asarray(generated, np.int32)
    out["logits"] = np.asarray(logits, F).reshape(-1)
    out["n_forwards_with_logits"] = np.array(len(snaps.snaps))
    for fi, snap in enumerate(snaps.snaps):
        pack_record(f"f{fi}_", snap, out, snap["h"].shape[0] == 1)
    path.unlink()
    return out, meta


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--skip-full", action="store_true", help="only layout/exp/ops/cfg0")
    ap.add_argument("--tmp", default=None,
                    help="folder for the scratch blobs (default: a fresh temporary folder)")
    args = ap.parse_args()
    ref, pqwf, convert_pqwf = load_reference(Path(args.reference))
    tmp = Path(args.tmp) if args.tmp else Path(tempfile.mkdtemp(prefix="q3_golden_"))
    tmp.mkdir(parents=True, exist_ok=True)

    libc_ver = platform.libc_ver()
    meta = {"numpy": np.__version__, "libc": list(libc_ver),
            "NPY_DISABLE_CPU_FEATURES": os.environ["NPY_DISABLE_CPU_FEATURES"],
            "python": platform.python_version()}
    meta["exp2_pin_check"] = exp2_pin_check()
    print("exp2 pin:", meta["exp2_pin_check"], flush=True)
    assert meta["exp2_pin_check"]["mismatches"] == 0

    (HERE / "layout.json").write_text(json.dumps(make_layout(pqwf), indent=1))
    np.savez_compressed(HERE / "exp.npz", **make_exp(ref))
    np.savez_compressed(HERE / "ops.npz", **make_ops(ref))
    print("layout/exp/ops written", flush=True)

    names = ["cfg0"] if args.skip_full else ["cfg0", "cfg2", "cfg3"]
    for name in names:
        out, m = run_config(name, ref, pqwf, convert_pqwf, tmp)
        np.savez_compressed(HERE / f"{name}.npz", **out)
        meta[name] = m
        print(name, m, flush=True)
    old = {}
    mp = HERE / "meta.json"
    if mp.exists():
        old = json.loads(mp.read_text())
    old.update(meta)
    mp.write_text(json.dumps(old, indent=1))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
