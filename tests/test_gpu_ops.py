"""GPU parity of every operator, called through the C ABI, against the CPU
oracle (and the reference goldens where they exist).  Integer stages and
f32 stages are both required to be bit-exact."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from conftest import bits_equal, describe_diff, golden

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3ops import ops  # noqa: E402

F = np.float32
QK = F(0.08838834764831845)


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def rand_gemm(rng, M, K, N, group):
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    b = rng.integers(-127, 128, (N, K)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, (M, K // group)).astype(F)
    bs = rng.uniform(1e-3, 1e-1, N).astype(F)
    return a, as_, b, bs


SHAPES = [(1024, 2048, 256), (1024, 1024, 256), (1024, 6144, 256), (3072, 1024, 256),
          (2048, 1024, 128)]


@pytest.mark.parametrize("M", [1, 5, 32, 64, 512])
@pytest.mark.parametrize("K,N,group", SHAPES)
def test_gemm_store(cuda, M, K, N, group):
    note(f"gemm store M={M} K={K} N={N} g={group}")
    rng = np.random.default_rng(M * 7 + K + N)
    a, as_, b, bs = rand_gemm(rng, M, K, N, group)
    out = torch.zeros((M, N), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), out, group)
    ref = oracle.gemm_nt_group(a, as_, b, bs, group)
    got = host(out)
    assert bits_equal(got, ref), describe_diff(got, ref)


@pytest.mark.parametrize("K,N,group", SHAPES)
def test_gemm_2048_rows(cuda, K, N, group):
    """BASELINE config 1's largest M on each of its five (K, N) shapes."""
    note(f"gemm store M=2048 K={K} N={N} g={group}")
    rng = np.random.default_rng(99 + K + N)
    a, as_, b, bs = rand_gemm(rng, 2048, K, N, group)
    out = torch.zeros((2048, N), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), out, group)
    ref = oracle.gemm_nt_group(a, as_, b, bs, group)
    got = host(out)
    assert bits_equal(got, ref), describe_diff(got, ref)


@pytest.mark.parametrize("M", [100, 512])
@pytest.mark.parametrize("K,N,group", [(1024, 2048, 256), (3072, 1024, 256), (2048, 1024, 128)])
def test_gemm_tile_variant(cuda, monkeypatch, M, K, N, group):
    """Q3_PREFILL_GEMM=tile (read at every launch): the LDS-staged tile
    kernel in place of the stream kernel for row-major weights, with the
    plain store, the residual add and the per-head quant epilogues, and the
    gate/up SwiGLU + quant at M = 512, against the oracle."""
    note(f"gemm tile variant M={M} K={K} N={N} g={group}")
    monkeypatch.setenv("Q3_PREFILL_GEMM", "tile")
    rng = np.random.default_rng(3 * M + K + N)
    a, as_, b, bs = rand_gemm(rng, M, K, N, group)
    ref = oracle.gemm_nt_group(a, as_, b, bs, group)
    out = torch.zeros((M, N), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), out, group)
    assert bits_equal(host(out), ref), describe_diff(host(out), ref)
    x = rng.normal(size=(M, N)).astype(F)
    xt = dev(x)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, group, add=xt)
    assert bits_equal(host(xt), (ref + x).astype(F))
    q8 = torch.zeros((M, N), dtype=torch.int8, device=cuda)
    qs = torch.zeros((M, N // 128), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, group, q8=q8, qs=qs)
    rq, rs = oracle.quant_rows_heads(ref, 128)
    assert bits_equal(host(q8), rq) and bits_equal(host(qs), rs)
    if K == 1024 and M == 512:
        _, _, wu, wus = rand_gemm(rng, M, 1024, 3072, 256)
        _, _, wg, wgs = rand_gemm(rng, M, 1024, 3072, 256)
        s8 = torch.zeros((M, 3072), dtype=torch.int8, device=cuda)
        ss = torch.zeros((M, 12), dtype=torch.float32, device=cuda)
        ops.gemm_gate_up_swiglu_quant(dev(a), dev(as_), dev(wg), dev(wgs), dev(wu), dev(wus), s8, ss, 256)
        rs8, rss = oracle.quant_rows_heads(oracle.swiglu(oracle.gemm_nt_group(a, as_, wg, wgs, 256),
                                                         oracle.gemm_nt_group(a, as_, wu, wus, 256)), 256)
        assert bits_equal(host(s8), rs8) and bits_equal(host(ss), rss)


def test_gemm_golden_guest_fixture(cuda):
    g = golden("ops.npz")
    for group, key, ns in ((128, "gg_out128", 2), (256, "gg_out256", 1)):
        out = torch.zeros((32, 128), dtype=torch.float32, device=cuda)
        ops.gemm_nt_group_store(dev(g["gg_a"]), dev(np.ones((32, ns), F)), dev(g["gg_b"]),
                                dev(np.ones(128, F)), out, group)
        got = host(out)
        assert bits_equal(got, g[key]), describe_diff(got, g[key])


@pytest.mark.parametrize("M", [1, 7, 40, 64, 300])
def test_gemm_residual_add(cuda, M):
    rng = np.random.default_rng(M)
    a, as_, b, bs = rand_gemm(rng, M, 2048, 1024, 128)
    x = rng.normal(size=(M, 1024)).astype(F)
    xt = dev(x)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, 128, add=xt)
    ref = (x + oracle.gemm_nt_group(a, as_, b, bs, 128)).astype(F)
    got = host(xt)
    assert bits_equal(got, ref), describe_diff(got, ref)


@pytest.mark.parametrize("M", [1, 32, 512, 2048])
@pytest.mark.parametrize("K,N,group", SHAPES)
def test_gemm_residual_config1_grid(cuda, M, K, N, group):
    """f32 output with residual add (group_gemm.h:194-214)
    over its whole M x (K, N) grid: x = D + x."""
    note(f"gemm residual M={M} K={K} N={N} g={group}")
    rng = np.random.default_rng(7 * M + K + 3 * N)
    a, as_, b, bs = rand_gemm(rng, M, K, N, group)
    x = rng.normal(size=(M, N)).astype(F)
    xt = dev(x)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, group, add=xt)
    ref = (oracle.gemm_nt_group(a, as_, b, bs, group) + x).astype(F)
    got = host(xt)
    assert bits_equal(got, ref), describe_diff(got, ref)


@pytest.mark.parametrize("M", [1, 32, 512, 2048])
@pytest.mark.parametrize("K,N,group", SHAPES)
def test_gemm_group_bscale_residual_config1(cuda, M, K, N, group):
    """BASELINE config 1 with its per-(row, group) B scales b_scale [N][K/g]:
    x = D + x over the whole grid, against the oracle's restatement."""
    note(f"gemm per-group B scales + residual M={M} K={K} N={N} g={group}")
    rng = np.random.default_rng(11 * M + K + 5 * N)
    a, as_, b, _ = rand_gemm(rng, M, K, N, group)
    bsg = rng.uniform(1e-3, 1e-1, (N, K // group)).astype(F)
    x = rng.normal(size=(M, N)).astype(F)
    xt = dev(x)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bsg), None, group, add=xt)
    ref = (oracle.gemm_nt_group_bg(a, as_, b, bsg, group) + x).astype(F)
    got = host(xt)
    assert bits_equal(got, ref), describe_diff(got, ref)


@pytest.mark.parametrize("M", [1, 5, 16, 17, 64, 300])
def test_gemm_group_bscale_store(cuda, M):
    """Per-(row, group) B scales with the plain store, on every GEMM path
    (M <= 64: the GEMV kernel, with row tiles above 16; above: the
    prefill-shaped kernels), at both group sizes."""
    for K, N, group in ((1024, 2048, 256), (2048, 1024, 128)):
        rng = np.random.default_rng(M + K)
        a, as_, b, _ = rand_gemm(rng, M, K, N, group)
        bsg = rng.uniform(1e-3, 1e-1, (N, K // group)).astype(F)
        out = torch.zeros((M, N), dtype=torch.float32, device=cuda)
        ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bsg), out, group)
        ref = oracle.gemm_nt_group_bg(a, as_, b, bsg, group)
        got = host(out)
        assert bits_equal(got, ref), (K, N, describe_diff(got, ref))


@pytest.mark.parametrize("M", [1, 9, 40, 130])
def test_gemm_head_quant(cuda, M):
    """V epilogue: per-head int8 quant (group_gemm.h:173-193)."""
    rng = np.random.default_rng(10 + M)
    a, as_, b, bs = rand_gemm(rng, M, 1024, 1024, 256)
    q8 = torch.zeros((M, 1024), dtype=torch.int8, device=cuda)
    qs = torch.zeros((M, 8), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, 256, q8=q8, qs=qs)
    rq, rs = oracle.quant_rows_heads(oracle.gemm_nt_group(a, as_, b, bs, 256), 128)
    assert bits_equal(host(q8), rq), describe_diff(host(q8), rq)
    assert bits_equal(host(qs), rs)


def nrq_ref(x, nw, cos, sin, heads):
    out = x.copy()
    for h in range(heads):
        hx = oracle.rmsnorm_rows(x[:, h * 128:(h + 1) * 128], nw, F(1 / 128))
        out[:, h * 128:(h + 1) * 128] = oracle.rope_head_hd(hx, cos, sin)
    return oracle.quant_rows_heads(out, 128)


@pytest.mark.parametrize("M", [1, 13, 32, 77, 512])
def test_gemm_norm_rope_quant(cuda, M):
    """Q/K epilogue: head RMSNorm + RoPE + quant (norm_rope_quant.h:17-86)."""
    rng = np.random.default_rng(20 + M)
    a, as_, b, bs = rand_gemm(rng, M, 1024, 2048, 256)
    nw = (1 + 0.05 * rng.normal(size=128)).astype(F)
    ang = rng.uniform(0, 100, (M, 64))
    cos, sin = np.cos(ang).astype(F), np.sin(ang).astype(F)
    q8 = torch.zeros((M, 2048), dtype=torch.int8, device=cuda)
    qs = torch.zeros((M, 16), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, 256, q8=q8, qs=qs,
                            nw=dev(nw), cos=dev(cos), sin=dev(sin), inv_hd=F(1 / 128))
    rq, rs = nrq_ref(oracle.gemm_nt_group(a, as_, b, bs, 256), nw, cos, sin, 16)
    assert bits_equal(host(q8), rq), describe_diff(host(q8), rq)
    assert bits_equal(host(qs), rs), describe_diff(host(qs), rs)


def test_norm_rope_quant_heads_unfused(cuda):
    rng = np.random.default_rng(30)
    x = rng.normal(size=(6, 1024)).astype(F)
    nw = (1 + 0.05 * rng.normal(size=128)).astype(F)
    ang = rng.uniform(0, 100, (6, 64))
    cos, sin = np.cos(ang).astype(F), np.sin(ang).astype(F)
    q8 = torch.zeros((6, 1024), dtype=torch.int8, device=cuda)
    qs = torch.zeros((6, 8), dtype=torch.float32, device=cuda)
    ops.norm_rope_quant_heads(dev(x), dev(nw), dev(cos), dev(sin), q8, qs, 8, F(1 / 128), True)
    rq, rs = nrq_ref(x, nw, cos, sin, 8)
    assert bits_equal(host(q8), rq) and bits_equal(host(qs), rs)


def make_pages(rng, kv_len, kv_dim, kv_heads, n_pages, shuffle=True, page_tokens=32):
    table = np.arange(n_pages, dtype=np.uint16)
    if shuffle:
        rng.shuffle(table)
    P = page_tokens
    k8 = rng.integers(-127, 128, (kv_len, kv_dim)).astype(np.int8)
    v8 = rng.integers(-127, 128, (kv_len, kv_dim)).astype(np.int8)
    ks = rng.uniform(1e-3, 5e-2, (kv_len, kv_heads)).astype(F)
    vs = rng.uniform(1e-3, 5e-2, (kv_len, kv_heads)).astype(F)
    kp = rng.integers(-127, 128, (n_pages, P, kv_dim)).astype(np.int8)  # garbage elsewhere
    vp = rng.integers(-127, 128, (n_pages, P, kv_dim)).astype(np.int8)
    ksp = np.full((n_pages, P, kv_heads), np.nan, F)
    vsp = np.full((n_pages, P, kv_heads), np.nan, F)
    t = np.arange(kv_len)
    kp[table[t // P], t % P] = k8
    vp[table[t // P], t % P] = v8
    ksp[table[t // P], t % P] = ks
    vsp[table[t // P], t % P] = vs
    return (k8, v8, ks, vs), (kp, vp, ksp, vsp, table)


@pytest.mark.parametrize("page_tokens", [64, 96, 128])
@pytest.mark.parametrize("rows,kv_len", [(1, 1), (1, 200), (1, 1100), (40, 40), (33, 250),
                                         (100, 700)])
def test_attention_page_sizes(cuda, page_tokens, rows, kv_len):
    """PagedKV.page_tokens other than 32 (kernels/kv_pages.h:13-24; the walk
    divides by it, attention_gqa.h:462-463): 64 and 128 take the
    phase-parallel prefill kernel, 96 the block-order walk (not a power of
    two); one row takes the decode kernel; blocks start mid-page, and pages
    come from a shuffled table with garbage in the unused slots."""
    note(f"attention page_tokens={page_tokens} rows={rows} kv_len={kv_len}")
    rng = np.random.default_rng(page_tokens * 7 + rows * 1000 + kv_len)
    heads, kvh = 16, 8
    n_pages = (kv_len + page_tokens - 1) // page_tokens + 2
    (k8, v8, ks, vs), (kp, vp, ksp, vsp, table) = make_pages(rng, kv_len, kvh * 128, kvh, n_pages,
                                                             page_tokens=page_tokens)
    q8 = rng.integers(-127, 128, (rows, heads * 128)).astype(np.int8)
    qs = rng.uniform(1e-3, 5e-2, (rows, heads)).astype(F)
    kv = ops.paged_kv(dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16)), page_tokens)
    o8 = torch.zeros((rows, heads * 128), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((rows, heads), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(q8), dev(qs), kv, kv_len, o8, os_, heads, kvh, 128,
                                           True, QK)
    attn = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, heads, kvh, 128, True, QK)
    ro8, ros = oracle.quant_rows_heads(attn, 128)
    assert bits_equal(host(o8), ro8), describe_diff(host(o8), ro8)
    assert bits_equal(host(os_), ros), describe_diff(host(os_), ros)


@pytest.mark.parametrize("variant", ["walk", "pair"])
@pytest.mark.parametrize("rows,kv_len,causal", [(512, 512, True), (100, 1000, True), (48, 300, True),
                                                (40, 300, False)])
def test_attention_prefill_variants(cuda, monkeypatch, variant, rows, kv_len, causal):
    """The multi-row attention forms Q3_PREFILL_ATTN selects (read at every
    launch): the block-order walk and the causal pair in one workgroup give
    the oracle's bytes like the default phase-parallel kernel."""
    note(f"attention prefill variant={variant} rows={rows} kv_len={kv_len} causal={causal}")
    monkeypatch.setenv("Q3_PREFILL_ATTN", variant)
    rng = np.random.default_rng(rows * 13 + kv_len)
    heads, kvh = 16, 8
    n_pages = (kv_len + 31) // 32 + 2
    (k8, v8, ks, vs), (kp, vp, ksp, vsp, table) = make_pages(rng, kv_len, kvh * 128, kvh, n_pages)
    q8 = rng.integers(-127, 128, (rows, heads * 128)).astype(np.int8)
    qs = rng.uniform(1e-3, 5e-2, (rows, heads)).astype(F)
    kv = ops.paged_kv(dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16)))
    o8 = torch.zeros((rows, heads * 128), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((rows, heads), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(q8), dev(qs), kv, kv_len, o8, os_, heads, kvh, 128,
                                           causal, QK)
    torch.cuda.synchronize()
    attn = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, heads, kvh, 128, causal, QK)
    ro8, ros = oracle.quant_rows_heads(attn, 128)
    assert bits_equal(host(o8), ro8), describe_diff(host(o8), ro8)
    assert bits_equal(host(os_), ros), describe_diff(host(os_), ros)


@pytest.mark.parametrize("rows,kv_len", [(1, 1), (1, 33), (1, 600), (4, 80), (8, 48),
                                         (40, 40), (33, 97), (512, 512)])
def test_attention_paged(cuda, rows, kv_len):
    note(f"attention rows={rows} kv_len={kv_len}")
    rng = np.random.default_rng(rows * 1000 + kv_len)
    heads, kvh = 16, 8
    n_pages = (kv_len + 31) // 32 + 3
    (k8, v8, ks, vs), (kp, vp, ksp, vsp, table) = make_pages(rng, kv_len, kvh * 128, kvh, n_pages)
    q8 = rng.integers(-127, 128, (rows, heads * 128)).astype(np.int8)
    qs = rng.uniform(1e-3, 5e-2, (rows, heads)).astype(F)
    tk, tv, tks, tvs, tt = dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16))
    kv = ops.paged_kv(tk, tv, tks, tvs, tt)
    o8 = torch.zeros((rows, heads * 128), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((rows, heads), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(q8), dev(qs), kv, kv_len, o8, os_, heads, kvh, 128,
                                           True, QK)
    attn = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, heads, kvh, 128, True, QK)
    ro8, ros = oracle.quant_rows_heads(attn, 128)
    assert bits_equal(host(o8), ro8), describe_diff(host(o8), ro8)
    assert bits_equal(host(os_), ros), describe_diff(host(os_), ros)


@pytest.mark.parametrize("heads,kvh,rows,kv_len,causal", [
    (16, 8, 512, 2048, True),   # a later chunk: 1536 keys of context before the rows
    (16, 8, 100, 1000, True),   # row 0 at position 900 (not a multiple of 16 or 32)
    (16, 8, 48, 300, True),     # 3 query blocks: the middle one walks alone
    (16, 8, 17, 17, True),
    (8, 8, 64, 200, True),      # GQA group 1
    (16, 4, 96, 96, True),      # GQA group 4
    (16, 8, 40, 300, False),    # no mask: every row walks every key
])
def test_attention_prefill_shapes(cuda, heads, kvh, rows, kv_len, causal):
    """Multi-row attention (the phase-parallel prefill kernel) over contexts
    that span several 8-block chunks, unaligned first positions, odd query
    block counts, other GQA groups and the unmasked form."""
    note(f"attention prefill heads={heads}/{kvh} rows={rows} kv_len={kv_len} causal={causal}")
    rng = np.random.default_rng(rows * 7 + kv_len + heads + kvh)
    n_pages = (kv_len + 31) // 32 + 2
    (k8, v8, ks, vs), (kp, vp, ksp, vsp, table) = make_pages(rng, kv_len, kvh * 128, kvh, n_pages)
    q8 = rng.integers(-127, 128, (rows, heads * 128)).astype(np.int8)
    qs = rng.uniform(1e-3, 5e-2, (rows, heads)).astype(F)
    kv = ops.paged_kv(dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16)))
    o8 = torch.zeros((rows, heads * 128), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((rows, heads), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(q8), dev(qs), kv, kv_len, o8, os_, heads, kvh, 128,
                                           causal, QK)
    attn = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, heads, kvh, 128, causal, QK)
    ro8, ros = oracle.quant_rows_heads(attn, 128)
    assert bits_equal(host(o8), ro8), describe_diff(host(o8), ro8)
    assert bits_equal(host(os_), ros), describe_diff(host(os_), ros)


@pytest.mark.parametrize("heads,kvh,kv_len", [(16, 8, 1023), (16, 8, 1025), (16, 8, 2500),
                                              (8, 8, 77), (8, 8, 1100)])
def test_attention_decode_chunks(cuda, heads, kvh, kv_len):
    """One query row (the decode kernel): key counts around and beyond the
    1024-key chunk of the parallel form, GQA groups 2 and 1."""
    note(f"attention decode heads={heads}/{kvh} kv_len={kv_len}")
    rng = np.random.default_rng(kv_len + heads)
    n_pages = (kv_len + 31) // 32 + 2
    (k8, v8, ks, vs), (kp, vp, ksp, vsp, table) = make_pages(rng, kv_len, kvh * 128, kvh, n_pages)
    q8 = rng.integers(-127, 128, (1, heads * 128)).astype(np.int8)
    qs = rng.uniform(1e-3, 5e-2, (1, heads)).astype(F)
    kv = ops.paged_kv(dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16)))
    o8 = torch.zeros((1, heads * 128), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((1, heads), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(q8), dev(qs), kv, kv_len, o8, os_, heads, kvh, 128,
                                           True, QK)
    attn = oracle.attention_heads_gqa_tokscale(q8, qs, k8, ks, v8, vs, heads, kvh, 128, True, QK)
    ro8, ros = oracle.quant_rows_heads(attn, 128)
    assert bits_equal(host(o8), ro8), describe_diff(host(o8), ro8)
    assert bits_equal(host(os_), ros), describe_diff(host(os_), ros)


@pytest.mark.parametrize("case,rows,kv_len", [("pa", 4, 80), ("pm1", 8, 48)])
def test_attention_guest_fixture(cuda, case, rows, kv_len):
    """The reference's paged-attention guest inputs (4 heads / 2 kv heads,
    shuffled page table as in paged_attn.cpp) against its golden outputs."""
    g = golden("ops.npz")
    n_pages = (kv_len + 31) // 32
    table = np.array([2, 0, 1] if n_pages == 3 else list(range(n_pages))[::-1], np.uint16)
    kd = 2 * 128
    kp = np.zeros((n_pages, 32, kd), np.int8)
    vp = np.zeros_like(kp)
    ksp = np.zeros((n_pages, 32, 2), F)
    vsp = np.zeros_like(ksp)
    t = np.arange(kv_len)
    kp[table[t // 32], t % 32] = g[f"{case}_k8"]
    vp[table[t // 32], t % 32] = g[f"{case}_v8"]
    ksp[table[t // 32], t % 32] = g[f"{case}_ks"]
    vsp[table[t // 32], t % 32] = g[f"{case}_vs"]
    kv = ops.paged_kv(dev(kp), dev(vp), dev(ksp), dev(vsp), dev(table.view(np.int16)))
    o8 = torch.zeros((rows, 512), dtype=torch.int8, device=cuda)
    os_ = torch.zeros((rows, 4), dtype=torch.float32, device=cuda)
    ops.attention_heads_gqa_tokscale_paged(dev(g[f"{case}_q8"]), dev(g[f"{case}_qs"]), kv, kv_len,
                                           o8, os_, 4, 2, 128, True, QK)
    assert bits_equal(host(o8), g[f"{case}_o8"]), describe_diff(host(o8), g[f"{case}_o8"])
    assert bits_equal(host(os_), g[f"{case}_os"])


def test_kv_paged_epilogues(cuda):
    """K (norm+RoPE) and V rows written into shuffled pages from a chunk that
    starts mid-page and crosses two page boundaries."""
    rng = np.random.default_rng(40)
    M, pos0, n_pages = 70, 21, 6
    a, as_, bk, bks = rand_gemm(rng, M, 1024, 1024, 256)
    _, _, bv, bvs = rand_gemm(rng, M, 1024, 1024, 256)
    nk = (1 + 0.05 * rng.normal(size=128)).astype(F)
    ang = rng.uniform(0, 100, (M, 64))
    cos, sin = np.cos(ang).astype(F), np.sin(ang).astype(F)
    table = np.array([4, 1, 5, 0, 3, 2], np.uint16)
    kp = torch.zeros((n_pages, 32, 1024), dtype=torch.int8, device=cuda)
    vp = torch.zeros_like(kp)
    ksp = torch.zeros((n_pages, 32, 8), dtype=torch.float32, device=cuda)
    vsp = torch.zeros_like(ksp)
    kv = ops.paged_kv(kp, vp, ksp, vsp, dev(table.view(np.int16)))
    ta, tas = dev(a), dev(as_)
    ops.gemm_nt_group_kv_paged(ta, tas, dev(bv), dev(bvs), 256, kv, pos0, True)
    ops.gemm_nt_group_kv_paged(ta, tas, dev(bk), dev(bks), 256, kv, pos0, False, nw=dev(nk),
                               cos=dev(cos), sin=dev(sin), inv_hd=F(1 / 128))
    rv8, rvs = oracle.quant_rows_heads(oracle.gemm_nt_group(a, as_, bv, bvs, 256), 128)
    rk8, rks = nrq_ref(oracle.gemm_nt_group(a, as_, bk, bks, 256), nk, cos, sin, 8)
    t = pos0 + np.arange(M)
    pg, sl = table[t // 32], t % 32
    assert bits_equal(host(vp)[pg, sl], rv8) and bits_equal(host(vsp)[pg, sl], rvs)
    assert bits_equal(host(kp)[pg, sl], rk8) and bits_equal(host(ksp)[pg, sl], rks)
    # nothing outside the written slots was touched
    mask = np.ones((n_pages, 32), bool)
    mask[pg, sl] = False
    assert not host(kp)[mask].any() and not host(vsp)[mask].any()


@pytest.mark.parametrize("M", [1, 11, 16, 64, 100, 512])
def test_gate_up_swiglu_quant(cuda, M):
    rng = np.random.default_rng(50 + M)
    a, as_, wg, wgs = rand_gemm(rng, M, 1024, 3072, 256)
    _, _, wu, wus = rand_gemm(rng, M, 1024, 3072, 256)
    s8 = torch.zeros((M, 3072), dtype=torch.int8, device=cuda)
    ss = torch.zeros((M, 12), dtype=torch.float32, device=cuda)
    ops.gemm_gate_up_swiglu_quant(dev(a), dev(as_), dev(wg), dev(wgs), dev(wu), dev(wus), s8, ss,
                                  256)
    g = oracle.gemm_nt_group(a, as_, wg, wgs, 256)
    u = oracle.gemm_nt_group(a, as_, wu, wus, 256)
    rs8, rss = oracle.quant_rows_heads(oracle.swiglu(g, u), 256)
    assert bits_equal(host(s8), rs8), describe_diff(host(s8), rs8)
    assert bits_equal(host(ss), rss), describe_diff(host(ss), rss)


def test_gate_up_swiglu_quant_strided_weights_two_streams(cuda):
    """Decode-shaped gate/up (M <= 16): weight rows with padding (the
    per-column-block kernel) and contiguous rows on two streams at once (the
    GEMV through each stream's own workspace) give the oracle's bytes."""
    rng = np.random.default_rng(77)
    M = 5
    a, as_, wg, wgs = rand_gemm(rng, M, 1024, 3072, 256)
    _, _, wu, wus = rand_gemm(rng, M, 1024, 3072, 256)
    g = oracle.gemm_nt_group(a, as_, wg, wgs, 256)
    u = oracle.gemm_nt_group(a, as_, wu, wus, 256)
    rs8, rss = oracle.quant_rows_heads(oracle.swiglu(g, u), 256)
    pad = lambda w: dev(np.concatenate([w, np.full((w.shape[0], 64), 99, np.int8)], axis=1))[:, :1024]
    s8 = torch.zeros((M, 3072), dtype=torch.int8, device=cuda)
    ss = torch.zeros((M, 12), dtype=torch.float32, device=cuda)
    ops.gemm_gate_up_swiglu_quant(dev(a), dev(as_), pad(wg), dev(wgs), pad(wu), dev(wus), s8, ss, 256)
    assert bits_equal(host(s8), rs8) and bits_equal(host(ss), rss)
    outs = []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    args = (dev(a), dev(as_), dev(wg), dev(wgs), dev(wu), dev(wus))
    torch.cuda.synchronize()
    for st in streams:
        o8 = torch.zeros((M, 3072), dtype=torch.int8, device=cuda)
        os_ = torch.zeros((M, 12), dtype=torch.float32, device=cuda)
        with torch.cuda.stream(st):
            for _ in range(4):
                ops.gemm_gate_up_swiglu_quant(*args, o8, os_, 256, stream=st)
        outs.append((o8, os_))
    torch.cuda.synchronize()
    for o8, os_ in outs:
        assert bits_equal(host(o8), rs8) and bits_equal(host(os_), rss)


@pytest.mark.parametrize("M", [1, 16, 64])
def test_gate_up_swiglu_quant_graph_capture_fresh_stream(cuda, M):
    """The decode-shaped gate/up captured in a HIP graph on a stream that has
    never run it (so it has no workspace and must not allocate inside the
    capture: it takes the fused kernel), then replayed three times with eager
    work in between: every replay gives the oracle's bytes."""
    rng = np.random.default_rng(90 + M)
    a, as_, wg, wgs = rand_gemm(rng, M, 1024, 3072, 256)
    _, _, wu, wus = rand_gemm(rng, M, 1024, 3072, 256)
    rs8, rss = oracle.quant_rows_heads(oracle.swiglu(oracle.gemm_nt_group(a, as_, wg, wgs, 256),
                                                     oracle.gemm_nt_group(a, as_, wu, wus, 256)), 256)
    args = (dev(a), dev(as_), dev(wg), dev(wgs), dev(wu), dev(wus))
    s8 = torch.zeros((M, 3072), dtype=torch.int8, device=cuda)
    ss = torch.zeros((M, 12), dtype=torch.float32, device=cuda)
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        ops.gemm_gate_up_swiglu_quant(*args, s8, ss, 256, stream=st)
    for rep in range(3):
        s8.fill_(0)
        ss.fill_(0.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(host(s8), rs8) and bits_equal(host(ss), rss), (M, rep)


def test_gate_up_guest_fixture(cuda):
    g = golden("ops.npz")
    s8 = torch.zeros((32, 256), dtype=torch.int8, device=cuda)
    ss = torch.zeros((32, 1), dtype=torch.float32, device=cuda)
    ops.gemm_gate_up_swiglu_quant(dev(g["gu_a"]), dev(g["gu_as"]), dev(g["gu_wg"]),
                                  dev(g["gu_wgs"]), dev(g["gu_wu"]), dev(g["gu_wus"]), s8, ss, 256)
    assert bits_equal(host(s8), g["gu_s8"]) and bits_equal(host(ss), g["gu_ss"])


@pytest.mark.parametrize("N", [1024, 151936])
def test_lm_argmax(cuda, N):
    rng = np.random.default_rng(N)
    a, as_, b, bs = rand_gemm(rng, 1, 1024, N, 256)
    best = torch.tensor([-3.0e38], dtype=torch.float32, device=cuda)
    bidx = torch.zeros(1, dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best, bidx, 256)
    logits = oracle.gemm_nt_group(a, as_, b, bs, 256)[0]
    assert int(host(bidx)[0]) == int(np.argmax(logits))
    assert bits_equal(host(best), logits.max(keepdims=True))
    # merging into a running (best, idx) that is not beaten keeps it
    best2 = torch.tensor([1e30], dtype=torch.float32, device=cuda)
    bidx2 = torch.tensor([-5], dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best2, bidx2, 256)
    assert int(host(bidx2)[0]) == -5 and host(best2)[0] == np.float32(1e30)


def test_lm_argmax_two_streams(cuda):
    """Two argmax calls in flight at once on two streams (each stream has its
    own key workspace): both results equal the oracle's."""
    rng = np.random.default_rng(123)
    cases = [rand_gemm(rng, M, 1024, 151936, 256) for M in (24, 7)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ins = [tuple(dev(t) for t in c) for c in cases]
    outs = []
    torch.cuda.synchronize()
    for (ta, tas, tb, tbs), st in zip(ins, streams):
        M = ta.shape[0]
        with torch.cuda.stream(st):
            best = torch.full((M,), -3.0e38, dtype=torch.float32, device=cuda)
            bidx = torch.zeros(M, dtype=torch.int32, device=cuda)
            for _ in range(3):  # repeated, so the two streams' launches interleave
                ops.gemm_nt_group_argmax(ta, tas, tb, tbs, best, bidx, 256, stream=st)
            outs.append((best, bidx))
    torch.cuda.synchronize()
    for (a, as_, b, bs), (best, bidx) in zip(cases, outs):
        logits = oracle.gemm_nt_group(a, as_, b, bs, 256)
        assert bidx.cpu().numpy().tolist() == [int(i) for i in np.argmax(logits, axis=1)]
        assert bits_equal(best.cpu().numpy(), logits.max(axis=1))


# 17-64 rows on the GEMV kernel: each way of splitting the rows (one 16-row
# tile per workgroup in grid rows; 2 tiles per workgroup; 4 tiles with the A
# fragments in one batch or, at three groups per wave, in two), at both
# group sizes, with rows past M inside a workgroup's last tile
ROW_TILE_CASES = [
    ("split", 20, 3072, 1024, 256),
    ("mt2", 48, 1024, 4096, 256),
    ("mt2_g128", 33, 1024, 4096, 128),
    ("mt4_two_batches", 64, 3072, 4224, 256),
    ("mt4_g128", 40, 2048, 4224, 128),
]


@pytest.mark.parametrize("case,M,K,N,group", ROW_TILE_CASES)
def test_gemm_row_tiles(cuda, case, M, K, N, group):
    """Store, residual add, per-(row, group) B scales and the argmax key
    epilogue of the row-tiled GEMV against the oracle, bit for bit."""
    note(f"gemm row tiles {case} M={M} K={K} N={N} g={group}")
    rng = np.random.default_rng(131 * M + K + N + group)
    a, as_, b, bs = rand_gemm(rng, M, K, N, group)
    ref = oracle.gemm_nt_group(a, as_, b, bs, group)
    out = torch.zeros((M, N), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), out, group)
    got = host(out)
    assert bits_equal(got, ref), ("store", describe_diff(got, ref))
    x = rng.normal(size=(M, N)).astype(F)
    xt = dev(x)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), None, group, add=xt)
    got = host(xt)
    exp = (ref + x).astype(F)
    assert bits_equal(got, exp), ("residual", describe_diff(got, exp))
    bsg = rng.uniform(1e-3, 1e-1, (N, K // group)).astype(F)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bsg), out, group)
    got = host(out)
    exp = oracle.gemm_nt_group_bg(a, as_, b, bsg, group)
    assert bits_equal(got, exp), ("group B scales", describe_diff(got, exp))
    best = torch.full((M,), -3.0e38, dtype=torch.float32, device=cuda)
    bidx = torch.zeros(M, dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best, bidx, group)
    assert host(bidx).tolist() == [int(i) for i in np.argmax(ref, axis=1)]
    assert bits_equal(host(best), ref.max(axis=1))


@pytest.mark.parametrize("M", [2, 5, 16, 20, 33, 64, 100])
def test_lm_argmax_wide_multirow(cuda, M):
    """lm_head width with several rows: one running key per row and
    workgroup across the column tiles each workgroup walks (M <= 16), one key
    per row and 128-column tile of the LDS-staged tile kernel (M <= 64), and
    the per-32-row kernel beyond."""
    note(f"lm argmax M={M} N=151936")
    rng = np.random.default_rng(40 + M)
    a, as_, b, bs = rand_gemm(rng, M, 1024, 151936, 256)
    best = torch.full((M,), -3.0e38, dtype=torch.float32, device=cuda)
    bidx = torch.zeros(M, dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best, bidx, 256)
    logits = oracle.gemm_nt_group(a, as_, b, bs, 256)
    assert host(bidx).tolist() == [int(i) for i in np.argmax(logits, axis=1)]
    assert bits_equal(host(best), logits.max(axis=1))


def test_lm_argmax_wide_ties_across_tiles(cuda):
    """Copies of the winning row in tiles owned by other workgroups (and in
    the same tile): the earliest index wins."""
    rng = np.random.default_rng(77)
    a, as_, b, bs = rand_gemm(rng, 1, 1024, 151936, 256)
    logits = oracle.gemm_nt_group(a, as_, b, bs, 256)[0]
    w = int(np.argmax(logits))
    copies = [151935, 70001, min(w + 1, 151935), 64 * 513 + 3]
    for c in copies:
        b[c] = b[w]
        bs[c] = bs[w]
    first = min([w] + copies)
    best = torch.tensor([-3.0e38], dtype=torch.float32, device=cuda)
    bidx = torch.zeros(1, dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best, bidx, 256)
    assert int(host(bidx)[0]) == first


@pytest.mark.parametrize("M", [1, 3])
def test_gemm_store_lm_width(cuda, M):
    """Logits mode: the full 151936-wide f32 row(s)."""
    note(f"gemm store M={M} N=151936")
    rng = np.random.default_rng(90 + M)
    a, as_, b, bs = rand_gemm(rng, M, 1024, 151936, 256)
    out = torch.zeros((M, 151936), dtype=torch.float32, device=cuda)
    ops.gemm_nt_group_store(dev(a), dev(as_), dev(b), dev(bs), out, 256)
    ref = oracle.gemm_nt_group(a, as_, b, bs, 256)
    got = host(out)
    assert bits_equal(got, ref), describe_diff(got, ref)


def test_lm_argmax_ties_first_index(cuda):
    """Duplicate the winning weight row at a later index and an earlier one:
    the earliest index of the maximum wins."""
    rng = np.random.default_rng(7)
    a, as_, b, bs = rand_gemm(rng, 1, 1024, 4096, 256)
    logits = oracle.gemm_nt_group(a, as_, b, bs, 256)[0]
    w = int(np.argmax(logits))
    b[3000] = b[w]
    bs[3000] = bs[w]
    b[17] = b[w]
    bs[17] = bs[w]
    best = torch.tensor([-3.0e38], dtype=torch.float32, device=cuda)
    bidx = torch.zeros(1, dtype=torch.int32, device=cuda)
    ops.gemm_nt_group_argmax(dev(a), dev(as_), dev(b), dev(bs), best, bidx, 256)
    assert int(host(bidx)[0]) == min(17, w)


def test_argmax_logits(cuda):
    rng = np.random.default_rng(8)
    v = rng.normal(size=151936).astype(F)
    v[[100, 5000]] = v.max() + 1
    out = torch.zeros(4, dtype=torch.int32, device=cuda)
    ops.argmax_logits(dev(v.reshape(1, -1)), out)
    assert int(host(out)[0]) == oracle.argmax_logits(v) == 100


def test_rows_kernels(cuda):
    rng = np.random.default_rng(9)
    V, H, R = 1024, 1024, 37
    emb = rng.integers(-127, 128, (V, H)).astype(np.int8)
    es = rng.uniform(1e-4, 1e-3, V).astype(F)
    ids = rng.integers(0, V, R).astype(np.int32)
    w = (1 + 0.05 * rng.normal(size=H)).astype(F)
    tmp = torch.zeros((R, H), dtype=torch.float32, device=cuda)
    out = torch.zeros((R, H), dtype=torch.float32, device=cuda)
    ops.embedding_rmsnorm_rows(dev(emb), dev(es), dev(ids.reshape(-1, 1)), tmp, dev(w), out,
                               F(1 / H))
    rh, rx = oracle.embedding_rmsnorm(emb, es, ids, w, F(1 / H))
    assert bits_equal(host(tmp), rx) and bits_equal(host(out), rh), describe_diff(host(out), rh)
    x = rng.normal(size=(R, H)).astype(F)
    ops.rmsnorm_rows(dev(x), dev(w), out, F(1 / H))
    ref = oracle.rmsnorm_rows(x, w, F(1 / H))
    assert bits_equal(host(out), ref), describe_diff(host(out), ref)
    for group in (128, 256):
        q = torch.zeros((R, H), dtype=torch.int8, device=cuda)
        s = torch.zeros((R, H // group), dtype=torch.float32, device=cuda)
        ops.quant_rows_heads(dev(x), q, s, group)
        rq, rs = oracle.quant_rows_heads(x, group)
        assert bits_equal(host(q), rq) and bits_equal(host(s), rs)


def test_quant_guest_fixture(cuda):
    g = golden("ops.npz")
    q = torch.zeros((32, 256), dtype=torch.int8, device=cuda)
    s = torch.zeros((32, 2), dtype=torch.float32, device=cuda)
    ops.quant_rows_heads(dev(g["qh_x"]), q, s, 128)
    assert bits_equal(host(q), g["qh_q"]) and bits_equal(host(s), g["qh_s"])


def test_zero_rows_are_no_ops(cuda):
    """Every row-parallel operator called with 0 rows returns OK and writes
    nothing, as the reference's row loops then do nothing (group_gemm.h:91,
    swiglu_quant.h:164, lm_argmax.h:72, attention_gqa.h:549, rmsnorm.h:34,
    quant.h:89, embedding.h:99).  The 0-row views are empty slices, which
    torch hands over with a NULL data pointer; the outputs they were sliced
    from hold a sentinel that must survive."""
    rng = np.random.default_rng(77)
    K, N, g = 1024, 2048, 256
    a, as_, b, bs = rand_gemm(rng, 4, K, N, g)
    ta, tas, tb, tbs = dev(a)[:0], dev(as_)[:0], dev(b), dev(bs)

    def full(shape, v, dt=torch.float32):
        return torch.full(shape, v, dtype=dt, device=cuda)

    note("zero rows: gemm store / residual / argmax")
    out = full((4, N), 7.0)
    ops.gemm_nt_group_store(ta, tas, tb, tbs, out[:0], g)
    ops.gemm_nt_group_store(ta, tas, tb, tbs, out[:0], g, add=out[:0])
    best, bidx = full((4,), -1.0), full((4,), -5, torch.int32)
    ops.gemm_nt_group_argmax(ta, tas, tb, tbs, best[:0], bidx[:0], g)
    ops.gemm_nt_group_argmax_noalloc(ta, tas, tb, tbs, best[:0], bidx[:0], g)
    torch.cuda.synchronize()
    assert (host(out) == 7.0).all()
    assert (host(best) == -1.0).all() and (host(bidx) == -5).all()

    note("zero rows: gate/up + SwiGLU + quant")
    _, _, wg, wgs = rand_gemm(rng, 1, K, 3072, g)
    _, _, wu, wus = rand_gemm(rng, 1, K, 3072, g)
    s8, ss = full((4, 3072), 5, torch.int8), full((4, 12), 3.0)
    ops.gemm_gate_up_swiglu_quant(ta, tas, dev(wg), dev(wgs), dev(wu), dev(wus), s8[:0], ss[:0], g)
    assert (host(s8) == 5).all() and (host(ss) == 3.0).all()

    note("zero rows: row kernels")
    H = 1024
    x = dev(rng.normal(size=(4, H)).astype(F))
    w = dev((1 + 0.05 * rng.normal(size=H)).astype(F))
    emb = dev(rng.integers(-127, 128, (64, H)).astype(np.int8))
    es = dev(rng.uniform(1e-4, 1e-3, 64).astype(F))
    ids = dev(np.arange(4, dtype=np.int32).reshape(-1, 1))
    tmp, rout = full((4, H), 2.0), full((4, H), 9.0)
    ops.embedding_rmsnorm_rows(emb, es, ids[:0], tmp[:0], w, rout[:0], F(1 / H))
    ops.rmsnorm_rows(x[:0], w, rout[:0], F(1 / H))
    q, s = full((4, H), 4, torch.int8), full((4, H // 128), 6.0)
    ops.quant_rows_heads(x[:0], q[:0], s[:0], 128)
    ang = rng.uniform(0, 100, (4, 64))
    cos, sin = dev(np.cos(ang).astype(F)), dev(np.sin(ang).astype(F))
    nw = dev((1 + 0.05 * rng.normal(size=128)).astype(F))
    ops.norm_rope_quant_heads(x[:0], nw, cos[:0], sin[:0], q[:0], s[:0, :8], 8, F(1 / 128), True)
    assert (host(tmp) == 2.0).all() and (host(rout) == 9.0).all()
    assert (host(q) == 4).all() and (host(s) == 6.0).all()

    note("zero rows: K/V page epilogue and attention")
    table = np.array([2, 0, 1], np.uint16)
    kp, ksp = full((3, 32, 1024), 1, torch.int8), full((3, 32, 8), 8.0)
    vp, vsp = full((3, 32, 1024), 1, torch.int8), full((3, 32, 8), 8.0)
    kv = ops.paged_kv(kp, vp, ksp, vsp, dev(table.view(np.int16)))
    _, _, bv, bvs = rand_gemm(rng, 1, K, 1024, g)
    ops.gemm_nt_group_kv_paged(ta, tas, dev(bv), dev(bvs), g, kv, 5, True)
    q8 = dev(rng.integers(-127, 128, (4, 16 * 128)).astype(np.int8))
    qs = dev(rng.uniform(1e-3, 5e-2, (4, 16)).astype(F))
    o8, os_ = full((4, 16 * 128), 3, torch.int8), full((4, 16), 1.5)
    for causal in (True, False):
        ops.attention_heads_gqa_tokscale_paged(q8[:0], qs[:0], kv, 40, o8[:0], os_[:0], 16, 8, 128,
                                               causal, QK)
    assert (host(kp) == 1).all() and (host(vp) == 1).all()
    assert (host(ksp) == 8.0).all() and (host(vsp) == 8.0).all()
    assert (host(o8) == 3).all() and (host(os_) == 1.5).all()
