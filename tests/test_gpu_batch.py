"""Batched decode of independent sequences (q3_decode_batch) against the
oracle, one sequence at a time.

Each sequence owns its own pages of the paged K/V pool (a per-row page table,
kernels/kv_pages.h paged_kv_scatter_batch; attention over per-row tables as in
tests/guest/paged_attn_multi.cpp) and its own position.  The contexts are
random int8 K/V rows with positive per-head scales written straight into the
pool; the oracle gets the same rows in its dense cache and runs
ref_qwen3.py:366-444 forward_chunk for one row at that sequence's position.
Compared bit for bit, for two consecutive steps: the greedy token, the new
K/V rows of every layer (through the sequence's table) and the last layer's
x / o8 / os / s8 / ss rows.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from conftest import bits_equal, describe_diff

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3ops import Q3Error  # noqa: E402
from q3ops.layout import InitConfig, Layout, ModelShape, init_random_blob  # noqa: E402
from q3ops.model import Model  # noqa: E402

PAGE = 32
Q3_ERR_RANGE = -7  # include/q3ops.h
LD_TABLE = 8  # pages per sequence table (contexts up to 254 tokens + 2 steps)
# Contexts around the batched attention's chunk of 12 blocks of 32 keys
# (384 keys): one short of a chunk, exactly one, one over, two chunks +- 1,
# and config 4's 2048-token contexts (6 chunks, the last one partial after
# the steps); the longest needs 65 table entries.
LONG_CTX = [383, 384, 385, 767, 768, 769, 1535, 2046, 2047, 2048]
LD_TABLE_LONG = 66
SHAPE = ModelShape(layers=2, vocab=1024, seq=96, max_seq=32768)
# config 4's own shape (on 2 layers): 64 rows at 2046-2048 keys, 65 pages
# each, in a pool of 4224 pages (4160 in use) under a random permutation,
# so that page ids far above 1024 are read
SHAPE_CFG4 = ModelShape(layers=2, vocab=1024, seq=96, max_seq=4224 * 32)
INIT = InitConfig(n_prompt=1, n_gen=0, mode=0)
_cache = {}


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def pool_views(lay: Layout, raw: np.ndarray) -> dict[str, np.ndarray]:
    """One layer's K/V pool (raw bytes) as [pages][32][...] arrays."""
    o = lay.offsets
    KW, NKV, MS = lay.kv_width, lay.kv_heads, lay.max_seq
    P = MS // PAGE
    so, vo = o["kKV_SOFF"], o["kKV_VOFF"]
    return {
        "kc": raw[:MS * KW].view(np.int8).reshape(P, PAGE, KW),
        "ks": raw[so:so + 4 * MS * NKV].view(np.float32).reshape(P, PAGE, NKV),
        "vc": raw[vo:vo + MS * KW].view(np.int8).reshape(P, PAGE, KW),
        "vs": raw[vo + so:vo + so + 4 * MS * NKV].view(np.float32).reshape(P, PAGE, NKV),
    }


def make_case(n: int, seed: int, edge: list[int] | None = None, ld_table: int = LD_TABLE,
              shape: ModelShape = SHAPE):
    """Blob with n random contexts in disjoint random pages; per-row positions
    and tables; the contexts in dense form for the oracle."""
    key = (n, seed, tuple(edge or ()), ld_table, shape)
    if key in _cache:
        return _cache[key]
    lay = Layout(shape)
    blob = init_random_blob(lay, INIT)
    rng = np.random.default_rng(seed)
    # edge contexts first: empty, one short of a page, exactly one page, one over
    top = 255
    if edge is None:
        edge = [0, 31, 32, 33, 62, 63, 64, 254]
    else:  # the other rows: random contexts up to the longest edge context
        top = max(edge) + 1
    ctx = np.array((edge + list(rng.integers(1, top, size=max(0, n - len(edge)))))[:n], np.int32)
    assert int(ctx.max()) + 2 <= ld_table * PAGE
    n_pages = lay.max_seq // PAGE
    perm = rng.permutation(n_pages).astype(np.uint16)
    tables = np.full((n, ld_table), 0xFFFF, np.uint16)  # unused slots: out of range on purpose
    need = [(int(c) + 2 + PAGE - 1) // PAGE for c in ctx]
    nxt = 0
    for r in range(n):
        tables[r, :need[r]] = perm[nxt:nxt + need[r]]
        nxt += need[r]
    assert nxt <= n_pages
    KW, NKV, L = lay.kv_width, lay.kv_heads, lay.layers
    o = lay.offsets
    dense = []
    for r in range(n):
        c = int(ctx[r])
        d = {"kc": rng.integers(-127, 128, size=(L, c, KW), dtype=np.int8),
             "vc": rng.integers(-127, 128, size=(L, c, KW), dtype=np.int8),
             "ks": rng.uniform(0.002, 0.03, size=(L, c, NKV)).astype(np.float32),
             "vs": rng.uniform(0.002, 0.03, size=(L, c, NKV)).astype(np.float32)}
        dense.append(d)
        t = np.arange(c)
        pages, slots = tables[r, t // PAGE], t % PAGE
        for li in range(L):
            base = o["kKV_BASE"] + li * o["kKV_STRIDE"]
            pv = pool_views(lay, blob[base:base + o["kKV_STRIDE"]])
            for nm in ("kc", "vc", "ks", "vs"):
                pv[nm][pages, slots] = d[nm][li]
    ids = rng.integers(0, lay.vocab, size=n).astype(np.int32)
    _cache[key] = (lay, blob, ctx, tables, dense, ids)
    return _cache[key]


def oracle_steps(lay: Layout, blob: np.ndarray, ctx, dense, ids, steps: int):
    """Per sequence: load its context into the oracle cache and run `steps`
    one-row forwards (greedy).  Returns per step: ids, new K/V rows, last-layer
    records."""
    om = oracle.OracleModel(blob, lay.offsets, dict(lay.shape.__dict__))
    n = len(ctx)
    out = [{"ids": np.zeros(n, np.int32), "rec": [], "kv": []} for _ in range(steps)]
    for r in range(n):
        om.reset_cache()
        c = int(ctx[r])
        for li in range(lay.layers):
            om.k8[li, :c] = dense[r]["kc"][li]
            om.v8[li, :c] = dense[r]["vc"][li]
            om.k_s[li, :c] = dense[r]["ks"][li]
            om.v_s[li, :c] = dense[r]["vs"][li]
        tok = int(ids[r])
        for st in range(steps):
            p = c + st
            logits, rec = om.forward_chunk(np.array([tok], np.int32), p, 1, True, record=True)
            tok = oracle.argmax_logits(logits)
            out[st]["ids"][r] = tok
            out[st]["rec"].append(rec)
            out[st]["kv"].append({nm: a[:, p].copy() for nm, a in
                                  (("kc", om.k8), ("vc", om.v8), ("ks", om.k_s), ("vs", om.v_s))})
    return out


def gpu_new_rows(m: Model, lay: Layout, tables, pos) -> list[dict]:
    """New K/V rows (at pos[r], through row r's table) of every layer."""
    o = lay.offsets
    per_layer = []
    for li in range(lay.layers):
        raw = m.read(o["kKV_BASE"] + li * o["kKV_STRIDE"], o["kKV_STRIDE"])
        pv = pool_views(lay, raw)
        pages = tables[np.arange(len(pos)), pos // PAGE]
        per_layer.append({nm: a[pages, pos % PAGE] for nm, a in pv.items()})
    return per_layer


def run_batch_case(cuda, n, lay, blob, ctx, tables, dense, ids0):
    steps = 2
    ref = oracle_steps(lay, blob, ctx, dense, ids0, steps)
    m = Model(lay, blob)
    ids = torch.from_numpy(ids0.copy()).to(cuda)
    out = torch.zeros(n, dtype=torch.int32, device=cuda)
    probs = []
    for st in range(steps):
        pos = (ctx + st).astype(np.int32)
        m.decode_batch(ids, pos, tables, out)
        m.synchronize()
        got = out.cpu().numpy()
        exp = ref[st]["ids"]
        if not np.array_equal(got, exp):
            bad = np.nonzero(got != exp)[0]
            probs.append(f"step {st} ids differ at rows {bad.tolist()}: {got[bad]} vs {exp[bad]}")
        rows = gpu_new_rows(m, lay, tables, pos)
        for li in range(lay.layers):
            for nm in ("kc", "ks", "vc", "vs"):
                e = np.stack([ref[st]["kv"][r][nm][li] for r in range(n)])
                if not bits_equal(rows[li][nm], e):
                    probs.append(f"step {st} layer {li} {nm}: {describe_diff(rows[li][nm], e)}")
        for nm in ("x", "o8", "os", "s8", "ss"):
            g = m.stage(nm, n)
            e = np.concatenate([ref[st]["rec"][r][nm] for r in range(n)])
            if not bits_equal(g, e):
                probs.append(f"step {st} {nm}: {describe_diff(g, e)}")
        ids = out.clone()
    m.close()
    assert not probs, probs


@pytest.mark.parametrize("n", [1, 5, 16, 17, 20, 40, 64, 80])
def test_decode_batch_matches_oracle(cuda, n):
    """One batched greedy step of n sequences against the oracle, stage by
    stage.  16/17 straddle the GEMV's one-tile/row-tile boundary; 20 and 40
    leave a workgroup's last row tile partly past n (one 16-row tile per
    workgroup in grid rows for the narrow launches, two per workgroup for
    Q|K|V and gate/up at 40); 80 takes the prefill-shaped GEMMs."""
    note(f"decode_batch n={n}")
    run_batch_case(cuda, n, *make_case(n, seed=100 + n))


@pytest.mark.parametrize("n", [len(LONG_CTX), 24])
def test_decode_batch_long_contexts(cuda, n):
    """Contexts that cross the batched attention's 384-key chunks, up to
    config 4's 2048 tokens: the (maximum, denominator, result) state of both
    query heads of a GQA group carried from chunk to chunk (attention_gqa.h:
    404-547 walks the blocks in one recurrence; the kernel splits it into
    chunks of 12 blocks)."""
    note(f"decode_batch long contexts n={n}")
    run_batch_case(cuda, n, *make_case(n, seed=300 + n, edge=list(LONG_CTX),
                                       ld_table=LD_TABLE_LONG))


def test_decode_batch_cfg4_shape(cuda):
    """BASELINE config 4's batch at its own shape: 64 sequences, every one at
    2046-2048 keys (65 pages of 32 tokens), their pages drawn from a pool of
    4224 through a random permutation (ids up to 4223), two greedy steps:
    ids, every layer's new K/V rows and the last layer's x/o8/os/s8/ss
    against the oracle run one sequence at a time."""
    note("decode_batch config 4 shape: 64 x 2046-2048 keys, 4224-page pool")
    edge = [2046 + r % 3 for r in range(64)]
    case = make_case(64, seed=404, edge=edge, ld_table=LD_TABLE_LONG, shape=SHAPE_CFG4)
    lay, blob, ctx, tables, dense, ids = case
    assert int(tables[tables != 0xFFFF].max()) > 1024
    run_batch_case(cuda, 64, *case)
    _cache.pop((64, 404, tuple(edge), LD_TABLE_LONG, SHAPE_CFG4), None)  # 0.6 GB blob


def test_decode_batch_rejects_bad_rows(cuda):
    """Host-side validation: positions, table entries and row counts out of
    range fail with Q3_ERR_RANGE before anything is launched."""
    lay, blob, ctx, tables, dense, ids0 = make_case(5, seed=105)
    m = Model(lay, blob)
    ids = torch.from_numpy(ids0.copy()).to(cuda)
    out = torch.zeros(5, dtype=torch.int32, device=cuda)
    cases = []
    pos = ctx.copy()
    pos[2] = lay.max_seq
    cases.append(("pos >= max_seq", pos, tables))
    pos = ctx.copy()
    pos[1] = LD_TABLE * PAGE  # beyond the table width
    cases.append(("pos beyond table", pos, tables))
    bad = tables.copy()
    bad[3, ctx[3] // PAGE] = lay.max_seq // PAGE  # page id past the pool
    cases.append(("page out of pool", ctx.copy(), bad))
    for what, pos, tab in cases:
        with pytest.raises(Q3Error) as ei:
            m.decode_batch(ids, pos, tab, out)
        assert ei.value.status == Q3_ERR_RANGE, what
    big = Model(Layout(ModelShape(layers=1, vocab=1024, seq=4, max_seq=256)))
    with pytest.raises(Q3Error):
        big.decode_batch(ids, ctx.copy() % 200, tables[:, :8] % 8, out)
    big.close()
    m.close()
