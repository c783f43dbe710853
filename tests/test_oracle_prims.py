"""The CPU oracle's primitives pinned against the reference's own outputs
(golden vectors written by tests/golden/make_golden.py from
tools/ref_qwen3.py) and against what the mathematics fixes."""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

import oracle
from conftest import REPO, bits_equal, describe_diff, golden


@pytest.fixture(scope="module", autouse=True)
def built():
    oracle.build()


def test_exp2_exhaustive_vs_libm():
    """orc_exp2f == glibc exp2f on every float in [-151, 129] (plus a sweep
    outside), i.e. the function numpy's pinned exp2 reduces to."""
    out = subprocess.run([str(REPO / "oracle" / "exp2_check")], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches=0" in out.stdout


def test_exp_f32_golden():
    g = golden("exp.npz")
    y = oracle.exp_f32(g["x"])
    assert bits_equal(y, g["y"]), describe_diff(y, g["y"])


def test_exp_special_values():
    x = np.array([0.0, -0.0, -np.inf, np.inf, 1.0, -1.0], np.float32)
    y = oracle.exp_f32(x)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == 0.0 and np.isinf(y[3])
    # exp(1) and exp(-1) to within 1 ulp of the true values
    assert abs(float(y[4]) - np.e) <= np.spacing(np.float32(np.e))
    assert abs(float(y[5]) - 1 / np.e) <= np.spacing(np.float32(1 / np.e))


def test_tree_reductions():
    # integers below 2^24 sum exactly, whatever the tree shape
    rng = np.random.default_rng(0)
    for n in range(1, 33):
        v = rng.integers(-1000, 1000, n).astype(np.float32)
        assert oracle.tree_sum(v) == np.float32(v.astype(np.int64).sum())
        assert oracle.tree_max(v) == v.max()
    # the pairing is adjacent pairs with the odd tail carried: with
    # [1, 2^-24, 2^-24] the tree gives (1 + 2^-24) + 2^-24 = 1 (RNE twice)
    v = np.array([1.0, 2.0 ** -24, 2.0 ** -24], np.float32)
    assert oracle.tree_sum(v) == np.float32(1.0)
    # while [2^-24, 2^-24, 1] pairs the two small values first
    v = np.array([2.0 ** -24, 2.0 ** -24, 1.0], np.float32)
    assert oracle.tree_sum(v) == np.float32(1.0 + 2.0 ** -23)


def test_group_gemm_golden_and_integer_pin():
    g = golden("ops.npz")
    a, b = g["gg_a"], g["gg_b"]
    for group, key, ns in ((128, "gg_out128", 2), (256, "gg_out256", 1)):
        out = oracle.gemm_nt_group(a, np.ones((32, ns), np.float32), b, np.ones(128, np.float32),
                                   group)
        assert bits_equal(out, g[key]), describe_diff(out, g[key])
        # scales 1.0: the grouped GEMM is a textbook integer matmul
        exact = a.astype(np.int64) @ b.astype(np.int64).T
        assert np.array_equal(out.astype(np.int64), exact)


def test_group_gemm_partials_brute_force():
    rng = np.random.default_rng(1)
    a = rng.integers(-127, 128, (5, 512)).astype(np.int8)
    w = rng.integers(-127, 128, (128, 512)).astype(np.int8)
    p = oracle.gemm_nt_group_i32(a, w, 256)
    for g in range(2):
        ref = a[:, g * 256:(g + 1) * 256].astype(np.int64) @ w[:, g * 256:(g + 1) * 256].astype(
            np.int64).T
        assert np.array_equal(p[:, g, :], ref)


def test_group_gemm_dequant_order():
    """Plant-a-mistake check: multiplying by a_scale before w_scale, or
    summing the groups in another order, changes bits on random data, and
    the oracle matches only the reference order."""
    rng = np.random.default_rng(2)
    a = rng.integers(-127, 128, (8, 1024)).astype(np.int8)
    w = rng.integers(-127, 128, (128, 1024)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, (8, 4)).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-1, 128).astype(np.float32)
    out = oracle.gemm_nt_group(a, as_, w, ws, 256)
    p = oracle.gemm_nt_group_i32(a, w, 256).astype(np.float32)
    F = np.float32
    good = np.zeros((8, 128), F)
    swapped = np.zeros((8, 128), F)
    for g in range(4):
        good = (good + ((p[:, g, :] * ws[None, :]).astype(F) * as_[:, g:g + 1]).astype(F)).astype(F)
        swapped = (swapped + ((p[:, g, :] * as_[:, g:g + 1]).astype(F) * ws[None, :]).astype(F)).astype(F)
    reversed_ = np.zeros((8, 128), F)
    for g in reversed(range(4)):
        reversed_ = (reversed_ + ((p[:, g, :] * ws[None, :]).astype(F) * as_[:, g:g + 1]).astype(F)).astype(F)
    assert bits_equal(out, good)
    assert not bits_equal(out, swapped)
    assert not bits_equal(out, reversed_)


def test_group_gemm_per_group_bscale_pins():
    """BASELINE config 1's per-(row, group) weight scales (not a reference
    function), pinned by what the arithmetic fixes: equal scales across a
    row's groups give the reference's per-row GEMM bit for bit; unit scales
    give the integer matmul; random scales agree with the f64 sum of the
    exact products within the rounding bound of its four roundings per term;
    and the plausible mistakes (one group's scale for every group, the
    [g][n] index, the scale product in the other order) fail."""
    rng = np.random.default_rng(12)
    F = np.float32
    M, K, N, G = 9, 1024, 256, 256
    ng = K // G
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, (M, ng)).astype(F)
    ws = rng.uniform(1e-3, 1e-1, N).astype(F)
    same = np.repeat(ws[:, None], ng, axis=1)
    assert bits_equal(oracle.gemm_nt_group_bg(a, as_, w, same, G), oracle.gemm_nt_group(a, as_, w, ws, G))
    one = oracle.gemm_nt_group_bg(a, np.ones((M, ng), F), w, np.ones((N, ng), F), G)
    assert np.array_equal(one.astype(np.int64), a.astype(np.int64) @ w.astype(np.int64).T)
    wsg = rng.uniform(1e-3, 1e-1, (N, ng)).astype(F)
    out = oracle.gemm_nt_group_bg(a, as_, w, wsg, G)
    p = oracle.gemm_nt_group_i32(a, w, G).astype(np.float64)      # [M][g][N], exact
    terms = p * wsg.T[None, :, :].astype(np.float64) * as_[:, :, None].astype(np.float64)
    exact = terms.sum(axis=1)
    bound = 4 * 2.0 ** -24 * np.abs(terms).sum(axis=1) * ng + 1e-30
    assert np.all(np.abs(out - exact) <= bound)
    p32 = p.astype(F)
    def acc(scale_of, order_ab=True):
        r = np.zeros((M, N), F)
        for g in range(ng):
            x = (p32[:, g, :] * scale_of(g)).astype(F) if order_ab else (p32[:, g, :] * as_[:, g:g + 1]).astype(F)
            x = (x * as_[:, g:g + 1]).astype(F) if order_ab else (x * scale_of(g)).astype(F)
            r = (r + x).astype(F)
        return r
    assert bits_equal(out, acc(lambda g: wsg[None, :, g]))
    assert not bits_equal(out, acc(lambda g: wsg[None, :, 0]))
    assert not bits_equal(out, acc(lambda g: wsg.reshape(ng, N)[g][None, :]))
    assert not bits_equal(out, acc(lambda g: wsg[None, :, g], order_ab=False))


def test_quant_golden_and_invariants():
    g = golden("ops.npz")
    q, s = oracle.quant_rows_heads(g["qh_x"], 128)
    assert bits_equal(q, g["qh_q"]) and bits_equal(s, g["qh_s"])
    rng = np.random.default_rng(3)
    x = rng.normal(size=(16, 512)).astype(np.float32)
    q, s = oracle.quant_rows_heads(x, 256)
    assert np.abs(q.astype(int)).max() <= 127
    # the absmax element of each group quantises to +-127
    for r in range(16):
        for gi in range(2):
            seg = x[r, gi * 256:(gi + 1) * 256]
            j = np.argmax(np.abs(seg))
            assert abs(int(q[r, gi * 256 + j])) == 127
            assert s[r, gi] == np.float32(np.abs(seg).max() * np.float32(1 / np.float32(127)))
    # reconstruction error within half a quantisation step (+ rounding slack)
    rec = q.reshape(16, 2, 256).astype(np.float64) * s[:, :, None]
    err = np.abs(rec - x.reshape(16, 2, 256))
    assert np.all(err <= s[:, :, None] * 0.5001 + 1e-12)
    # all-zero group: scale 0, 0/0 -> NaN -> 0
    q, s = oracle.quant_rows_heads(np.zeros((1, 128), np.float32), 128)
    assert s[0, 0] == 0 and not q.any()


def test_gate_up_swiglu_golden():
    g = golden("ops.npz")
    gg = oracle.gemm_nt_group(g["gu_a"], g["gu_as"], g["gu_wg"], g["gu_wgs"], 256)
    uu = oracle.gemm_nt_group(g["gu_a"], g["gu_as"], g["gu_wu"], g["gu_wus"], 256)
    assert bits_equal(gg, g["gu_g"]) and bits_equal(uu, g["gu_u"])
    sw = oracle.swiglu(gg, uu)
    assert bits_equal(sw, g["gu_sw"]), describe_diff(sw, g["gu_sw"])
    s8, ss = oracle.quant_rows_heads(sw, 256)
    assert bits_equal(s8, g["gu_s8"]) and bits_equal(ss, g["gu_ss"])


def test_swiglu_math():
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    u = np.ones_like(x)
    y = oracle.swiglu(x, u).astype(np.float64)
    ref = x / (1 + np.exp(-x.astype(np.float64)))
    # exp(-x) goes through RN(-x * log2e), an argument error of |x| * 2^-24
    # nats-equivalent, so the bound grows with |x|: 2e-7 * (1 + |x|) relative
    assert np.all(np.abs(y - ref) <= 2e-7 * (1 + np.abs(x)) * np.abs(ref) + 1e-30)


@pytest.mark.parametrize("case", ["pa", "pm1"])
def test_attention_golden(case):
    g = golden("ops.npz")
    out = oracle.attention_heads_gqa_tokscale(
        g[f"{case}_q8"], g[f"{case}_qs"], g[f"{case}_k8"], g[f"{case}_ks"], g[f"{case}_v8"],
        g[f"{case}_vs"], 4, 2, 128, True, np.float32(0.08838834764831845))
    assert bits_equal(out, g[f"{case}_attn"]), describe_diff(out, g[f"{case}_attn"])
    o8, os_ = oracle.quant_rows_heads(out, 128)
    assert bits_equal(o8, g[f"{case}_o8"]) and bits_equal(os_, g[f"{case}_os"])


def test_attention_single_block_is_exact_softmax():
    """One key block, P quantisation aside: a 1-row causal attention over
    <= 32 keys equals softmax(S) . V within the int8 P-quantisation error."""
    rng = np.random.default_rng(4)
    hd, kv = 128, 20
    q8 = rng.integers(-127, 128, (1, hd)).astype(np.int8)
    k8 = rng.integers(-127, 128, (kv, hd)).astype(np.int8)
    v8 = rng.integers(-127, 128, (kv, hd)).astype(np.int8)
    qs = np.array([[0.01]], np.float32)
    ks = rng.uniform(0.001, 0.01, (kv, 1)).astype(np.float32)
    vs = rng.uniform(0.001, 0.01, (kv, 1)).astype(np.float32)
    out = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, 1, 1, hd, True,
                                              np.float32(1 / np.sqrt(128)))
    s = (q8.astype(np.float64) @ k8.T.astype(np.float64)) * ks[:, 0] * 0.01 / np.sqrt(128)
    p = np.exp(s - s.max())
    p /= p.sum()
    ref = (p * vs[:, 0]) @ v8.astype(np.float64)
    scale = np.abs(ref).max()
    assert np.max(np.abs(out[0] - ref)) <= 0.01 * scale


def test_rmsnorm_math():
    rng = np.random.default_rng(5)
    x = rng.normal(size=(4, 1024)).astype(np.float32)
    w = (1 + 0.05 * rng.normal(size=1024)).astype(np.float32)
    y = oracle.rmsnorm_rows(x, w, np.float32(1 / 1024))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.allclose(y, ref, rtol=3e-6, atol=0)


def test_rope_is_rotation():
    rng = np.random.default_rng(6)
    x = rng.normal(size=(3, 128)).astype(np.float32)
    ang = rng.uniform(0, 6.28, size=(3, 64))
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = oracle.rope_head_hd(x, c, s).astype(np.float64)
    xl, xh = x[:, :64].astype(np.float64), x[:, 64:].astype(np.float64)
    ref = np.concatenate([xl * c - xh * s, xl * s + xh * c], 1)
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)
    # norms are preserved (rotation)
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


def test_argmax_logits_first_index():
    v = np.zeros(100, np.float32)
    v[[7, 40, 99]] = 3.0
    assert oracle.argmax_logits(v) == 7
    v = np.full(64, -5.0, np.float32)
    assert oracle.argmax_logits(v) == 0
    rng = np.random.default_rng(8)
    v = rng.normal(size=151936).astype(np.float32)
    assert oracle.argmax_logits(v) == int(np.argmax(v))
