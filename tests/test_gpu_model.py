"""GPU model path (q3_forward_chunk / q3_generate through the C ABI) against
the reference goldens of tools/ref_qwen3.py and against the oracle."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from conftest import bits_equal, describe_diff
from paritylib import compare_stage, load_cfg, sha

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3ops import LM_ARGMAX, LM_LOGITS, LM_NONE  # noqa: E402
from q3ops.layout import CONFIGS, InitConfig, Layout, ModelShape, init_random_blob  # noqa: E402
from q3ops.model import Model  # noqa: E402

_cache = {}


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def host_blob(name: str, shape: ModelShape | None = None, init: InitConfig | None = None):
    key = (name, shape, init)
    if key not in _cache:
        s0, i0 = CONFIGS[name]
        lay = Layout(shape or s0)
        _cache[key] = (lay, init_random_blob(lay, init or i0))
    return _cache[key]


def stage_problems(g, prefix, m: Model, rows: int, kv_len: int, layer: int,
                   last_row_only: bool) -> list[str]:
    probs = []
    sel = slice(rows - 1, rows) if last_row_only else None
    for st in ("h", "h8", "hs", "x", "s8", "ss", "o8", "os", "q8", "qs"):
        if last_row_only and st in ("q8", "qs"):
            continue  # row 0 doubles as the final-norm scratch (compare.py:49-51)
        got = m.stage(st, rows)
        if st in ("q8", "qs") and not last_row_only:
            # compare.py:197-205: row 0 of q8/qs is reused by the final norm
            got, gold_rows = got[1:], slice(1, None)
            spec = f"{prefix}{st}"
            if spec in g.files:
                exp = g[spec][1:]
                if not bits_equal(got, exp):
                    probs.append(f"{prefix}{st}: {describe_diff(got, exp)}")
            continue
        p = compare_stage(g, prefix, st, got, rows=sel)
        if p:
            probs.append(p)
    caches = m.kv_cache(layer, kv_len)
    for st in ("kc", "ks", "vc", "vs"):
        p = compare_stage(g, prefix, st, caches[st])
        if p:
            probs.append(p)
    return probs


@pytest.mark.parametrize("mode", [0, 1])
def test_cfg0_generate(cuda, mode, gold_meta):
    note(f"cfg0 generate mode={mode}")
    lay, blob = host_blob("cfg0")
    assert sha(blob[lay["kEMB"]:lay["kLOGITS"]]) == gold_meta["cfg0"]["weights_sha256"]
    g = load_cfg("cfg0")
    m = Model(lay, blob)
    m.set_ctrl(40, 2, mode)
    m.generate()
    ids = m.ids()
    assert np.array_equal(ids[40:42], g["generated"]), (ids[40:42], g["generated"])
    gl = g["logits"]
    if mode == 1:
        got = m.stage("logits", 1)[0]
        assert bits_equal(got, gl), describe_diff(got, gl)
    else:
        best, idx = m.argmax()
        assert idx == int(np.argmax(gl)) and bits_equal(np.float32(best), gl.max())
    last = int(g["n_forwards_with_logits"]) - 1
    probs = stage_problems(g, f"f{last}_", m, 1, 42, 0, last_row_only=(mode == 0))
    m.close()
    assert not probs, probs


@pytest.mark.parametrize("fuse_oproj,fuse_qkv", [("0", "1"), ("1", "0"), ("1", "1")])
def test_cfg0_generate_oproj_modes(cuda, gold_meta, fuse_oproj, fuse_qkv, monkeypatch):
    """Decode with the O projection inside the attention kernel (default) and
    as its own GEMV (Q3_DECODE_FUSE_OPROJ=0), and with the Q|K|V projection in
    the attention's launch (default; it needs the fused O projection) or as
    its own GEMV (Q3_DECODE_FUSE_QKV=0), both read when the model opens: the
    generated ids, logits and the last forward's stages match the goldens
    either way, and no bounded wait of the fused launch ran out."""
    note(f"cfg0 generate fuse_oproj={fuse_oproj} fuse_qkv={fuse_qkv}")
    monkeypatch.setenv("Q3_DECODE_FUSE_OPROJ", fuse_oproj)
    monkeypatch.setenv("Q3_DECODE_FUSE_QKV", fuse_qkv)
    lay, blob = host_blob("cfg0")
    g = load_cfg("cfg0")
    m = Model(lay, blob)
    m.set_ctrl(40, 2, 1)
    m.generate()
    assert m.fused_status() == (3 if fuse_qkv == "1" else 0, 0)
    ids = m.ids()
    assert np.array_equal(ids[40:42], g["generated"]), (ids[40:42], g["generated"])
    got = m.stage("logits", 1)[0]
    assert bits_equal(got, g["logits"]), describe_diff(got, g["logits"])
    last = int(g["n_forwards_with_logits"]) - 1
    probs = stage_problems(g, f"f{last}_", m, 1, 42, 0, last_row_only=False)
    m.close()
    assert not probs, probs


def test_cfg0_each_forward(cuda):
    """forward_chunk step by step, non-fused (all rows of the last layer):
    every recorded stage of every forward, bit for bit.  Chunk 0 runs with
    logits on so its last layer is computed in full (with Q3_LM_NONE the
    device stops the last layer after the K/V writes, main_big.cpp:212-220,
    which is covered by the generate tests); the reference has no logits
    for chunk 0, so only its stages are compared."""
    lay, blob = host_blob("cfg0")
    g = load_cfg("cfg0")
    m = Model(lay, blob)
    ids = np.array(g["ids_in"], np.int32).copy()
    ids[40:] = g["generated"]
    m.set_ids(ids)
    for pos, rows, lm, prefix in ((0, 32, LM_LOGITS, "c0_"), (32, 8, LM_LOGITS, "f0_"),
                                  (40, 1, LM_LOGITS, "f1_"), (41, 1, LM_LOGITS, "f2_")):
        note(f"cfg0 forward pos={pos} rows={rows}")
        m.forward_chunk(pos, rows, lm, optimize_tail=False)
        probs = stage_problems(g, prefix, m, rows, pos + rows, 0, last_row_only=False)
        if f"{prefix}logits" in g.files:
            got = m.stage("logits", 1)[0]
            gl = g[f"{prefix}logits"].reshape(-1)
            if not bits_equal(got, gl):
                probs.append(f"{prefix}logits: {describe_diff(got, gl)}")
        assert not probs, (prefix, probs)
    m.close()


def test_cfg0_nonfinal_chunk_writes_kv_only(cuda):
    """Q3_LM_NONE on the last layer: K/V rows are written (bit-exact with the
    reference cache) and the tail is skipped."""
    lay, blob = host_blob("cfg0")
    g = load_cfg("cfg0")
    m = Model(lay, blob)
    m.forward_chunk(0, 32, LM_NONE)
    caches = m.kv_cache(0, 32)
    probs = [p for st in ("kc", "ks", "vc", "vs")
             if (p := compare_stage(g, "c0_", st, caches[st]))]
    m.close()
    assert not probs, probs


def test_cfg0_chunk_and_page_invariance(cuda):
    """One 40-row chunk (seq=64 layout, same weights) and a shuffled page
    table give the reference's ids and logits."""
    g = load_cfg("cfg0")
    shape = ModelShape(layers=1, vocab=1024, seq=64, max_seq=256)
    lay, blob = host_blob("cfg0", shape=shape)
    m = Model(lay, blob)
    rng = np.random.default_rng(3)
    tab = np.arange(lay.max_seq // 32, dtype=np.uint16)
    rng.shuffle(tab)
    m.set_page_table(tab)
    m.set_ctrl(40, 2, 1)
    m.generate()
    assert np.array_equal(m.ids()[40:42], g["generated"])
    got = m.stage("logits", 1)[0]
    assert bits_equal(got, g["logits"]), describe_diff(got, g["logits"])
    m.close()


@pytest.mark.parametrize("seq", [17, 20, 33, 48])
def test_cfg0_prompt_chunk_sizes(cuda, seq):
    """The 40-token prompt in chunks of at most `seq` rows (17+17+6, 20+20,
    33+7, 40): the GEMV row splits of 17-64-row chunks and the single-row
    and block-sized remainders give the reference's ids and logits."""
    g = load_cfg("cfg0")
    shape = ModelShape(layers=1, vocab=1024, seq=seq, max_seq=256)
    lay, blob = host_blob("cfg0", shape=shape)
    m = Model(lay, blob)
    m.set_ctrl(40, 2, 1)
    m.generate()
    assert np.array_equal(m.ids()[40:42], g["generated"])
    got = m.stage("logits", 1)[0]
    assert bits_equal(got, g["logits"]), describe_diff(got, g["logits"])
    m.close()


def test_cfg2_full_depth(cuda, gold_meta):
    note("cfg2 28 layers, 32-token prefill, mode 1")
    lay, blob = host_blob("cfg2")
    assert sha(blob[lay["kEMB"]:lay["kLOGITS"]]) == gold_meta["cfg2"]["weights_sha256"]
    g = load_cfg("cfg2")
    m = Model(lay, blob)
    m.generate()
    got = m.stage("logits", 1)[0]
    assert bits_equal(got, g["logits"]), describe_diff(got, g["logits"])
    probs = stage_problems(g, "f0_", m, 32, 32, lay.layers - 1, last_row_only=False)
    m.close()
    assert not probs, probs


@pytest.mark.parametrize("merge", ["1", "0"])
def test_cfg3_greedy(cuda, gold_meta, merge, monkeypatch):
    """Config 3's greedy generation on the decode graph, with each layer's
    down projection in the next layer's Q|K|V + attention launch (default)
    and on its own (Q3_DECODE_MERGE_DOWN=0)."""
    note(f"cfg3 28 layers, 15-token prompt + 6 greedy tokens, mode 0, merge={merge}")
    monkeypatch.setenv("Q3_DECODE_MERGE_DOWN", merge)
    lay, blob = host_blob("cfg3")
    g = load_cfg("cfg3")
    m = Model(lay, blob)
    m.generate()
    # decode on the fused Q|K|V + attention launch (+ the merged down)
    assert m.fused_status() == (3 if merge == "1" else 1, 0)
    ids = m.ids()
    assert np.array_equal(ids[15:21], g["generated"]), (ids[15:21], g["generated"])
    best, idx = m.argmax()
    gl = g["logits"]
    assert idx == int(np.argmax(gl)) and bits_equal(np.float32(best), gl.max())
    last = int(g["n_forwards_with_logits"]) - 1
    probs = stage_problems(g, f"f{last}_", m, 1, 21, lay.layers - 1, last_row_only=True)
    m.close()
    assert not probs, probs


@pytest.mark.parametrize("pf", ["0", "37"])
def test_cfg3_greedy_prefetch_counts(cuda, gold_meta, pf, monkeypatch):
    """The decode launches with no prefetch workgroups and with an odd count
    of them (Q3_DECODE_PREFETCH_WGS, read at open; the default is 120): the
    prefetch reads only warm the caches, so config 3's greedy ids, fused
    argmax and last-forward stages stay bit-exact and no bounded wait runs
    out."""
    note(f"cfg3 greedy with {pf} prefetch workgroups")
    monkeypatch.setenv("Q3_DECODE_PREFETCH_WGS", pf)
    lay, blob = host_blob("cfg3")
    g = load_cfg("cfg3")
    m = Model(lay, blob)
    m.generate()
    assert m.fused_status() == (3, 0)
    ids = m.ids()
    assert np.array_equal(ids[15:21], g["generated"]), (ids[15:21], g["generated"])
    best, idx = m.argmax()
    assert idx == int(np.argmax(g["logits"])) and bits_equal(np.float32(best), g["logits"].max())
    last = int(g["n_forwards_with_logits"]) - 1
    probs = stage_problems(g, f"f{last}_", m, 1, 21, lay.layers - 1, last_row_only=True)
    m.close()
    assert not probs, probs


@pytest.mark.parametrize("merge", ["0", "1"])
def test_cfg3_greedy_generic_roles(cuda, gold_meta, merge, monkeypatch):
    """The fused decode launches and the prefill attention with the head
    counts read from the kernel arguments (Q3_HEAD_CONSTS=0, as for any head
    configuration other than 16 / 8) instead of the compile-time constants
    of the 16 / 8 shape: config 3's greedy ids, fused argmax and
    last-forward stages stay bit-exact."""
    note(f"cfg3 greedy with argument head counts, merge={merge}")
    monkeypatch.setenv("Q3_HEAD_CONSTS", "0")
    monkeypatch.setenv("Q3_DECODE_MERGE_DOWN", merge)
    lay, blob = host_blob("cfg3")
    g = load_cfg("cfg3")
    m = Model(lay, blob)
    m.generate()
    assert m.fused_status() == (3 if merge == "1" else 1, 0)
    ids = m.ids()
    assert np.array_equal(ids[15:21], g["generated"]), (ids[15:21], g["generated"])
    best, idx = m.argmax()
    assert idx == int(np.argmax(g["logits"])) and bits_equal(np.float32(best), g["logits"].max())
    last = int(g["n_forwards_with_logits"]) - 1
    probs = stage_problems(g, f"f{last}_", m, 1, 21, lay.layers - 1, last_row_only=True)
    m.close()
    assert not probs, probs


def test_cfg3_merged_down_launches(cuda, gold_meta, monkeypatch):
    """The merged launch runs: with kernel timing on (eager launches), the
    down GEMV launches drop by layers - 1 per decode token against
    Q3_DECODE_MERGE_DOWN=0, the fused launches stay, and both runs give the
    golden ids and fused argmax."""
    lay, blob = host_blob("cfg3")
    g = load_cfg("cfg3")
    counts = {}
    for merge in ("1", "0"):
        note(f"cfg3 generate with kernel timing, merge={merge}")
        monkeypatch.setenv("Q3_DECODE_MERGE_DOWN", merge)
        m = Model(lay, blob)
        m.set_kernel_timing(True)
        m.generate()
        counts[merge] = {k: n for k, (_, n) in m.kernel_times().items()}
        assert m.fused_status()[1] == 0
        ids = m.ids()
        assert np.array_equal(ids[15:21], g["generated"]), (merge, ids[15:21], g["generated"])
        best, idx = m.argmax()
        assert idx == int(np.argmax(g["logits"])) and bits_equal(np.float32(best), g["logits"].max())
        m.close()
    on, off = counts["1"], counts["0"]
    assert on["attn_decode"] == off["attn_decode"] > 0
    saved = off["gemv_down"] - on["gemv_down"]
    assert saved > 0 and saved % (lay.layers - 1) == 0, (on, off)
    assert saved // (lay.layers - 1) == on["attn_decode"] // lay.layers, (on, off)


# Config 3's perf prefill as one 512-row chunk (layout seq = 512) on a
# 2-layer, vocab-1024 model with the same seeds; the oracle runs the same
# prompt as sixteen 32-row chunks (a row's arithmetic does not depend on the
# chunk it is computed in: ref_qwen3.py:366-444 is row-wise except for the
# causal attention, which walks the row's keys in the same 32-key blocks).
SHAPE_512 = ModelShape(layers=2, vocab=1024, seq=512, max_seq=640)
INIT_512 = InitConfig(n_prompt=512, n_gen=4, mode=0)


def oracle_512(blob, lay):
    import oracle
    dims = dict(SHAPE_512.__dict__)
    dims["seq"] = 32
    return oracle.OracleModel(blob, lay.offsets, dims)


def test_cfg3_prefill_512_chunk_stages(cuda):
    """One 512-row q3_forward_chunk against the oracle's 16 chunks of 32:
    every recorded stage of the last layer for all 512 rows, both layers'
    K/V pages (all 16 pages, through a shuffled page table) and the logits."""
    note("512-row prefill chunk, 2 layers, stages + K/V pages + logits")
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_512, init=INIT_512)
    om = oracle_512(blob, lay)
    ids = lay.global_views(blob)["ids"][:512].copy()
    recs, logits = [], None
    for c in range(16):
        lg, rec = om.forward_chunk(ids[32 * c:32 * (c + 1)], 32 * c, 32, c == 15, record=True)
        recs.append(rec)
        logits = lg
    ref = {k: np.concatenate([r[k] for r in recs]) for k in recs[0]}
    m = Model(lay, blob)
    tab = np.arange(lay.max_seq // 32, dtype=np.uint16)
    np.random.default_rng(5).shuffle(tab)
    m.set_page_table(tab)
    m.forward_chunk(0, 512, LM_LOGITS, optimize_tail=False)
    probs = []
    got = m.stage("logits", 1)[0]
    if not bits_equal(got, logits):
        probs.append(f"logits: {describe_diff(got, logits)}")
    for st in ("h", "h8", "hs", "q8", "qs", "o8", "os", "s8", "ss", "x"):
        g = m.stage(st, 512)
        e = ref[st]
        if st in ("q8", "qs"):  # row 0 doubles as the final-norm scratch (compare.py:197-205)
            g, e = g[1:], e[1:]
        if not bits_equal(g, e):
            probs.append(f"{st}: {describe_diff(g, e)}")
    for li in range(lay.layers):
        caches = m.kv_cache(li, 512)
        for st, arr in (("kc", om.k8), ("ks", om.k_s), ("vc", om.v8), ("vs", om.v_s)):
            e = arr[li, :512]
            if not bits_equal(caches[st], e):
                probs.append(f"layer {li} {st}: {describe_diff(caches[st], e)}")
    m.close()
    assert not probs, probs


def test_cfg3_prefill_512_generate(cuda):
    """q3_generate with CTRL [512, 4, mode 0]: one 512-row prefill chunk (on
    the weights packed at model open), then four greedy decode steps; ids and
    the fused argmax equal the oracle's.  Three calls on the model's own
    stream: the first captures the decode steps as a graph, the later ones
    replay it, and between calls the device memory is churned (large tensors
    filled and released), so a prefill reading weights that an earlier call
    released would show."""
    note("512-row prefill + 4 greedy tokens, 2 layers, 3 calls")
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_512, init=INIT_512)
    om = oracle_512(blob, lay)
    logits, gen, _, _ = om.generate(lay.global_views(blob)["ids"], 512, 4, record=False)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        m = Model(lay, blob, stream=st)
    m.set_ctrl(512, 4, 0)
    for rep in range(3):
        note(f"generate call {rep}")
        m.generate()
        m.synchronize()
        got = m.ids()[512:516].copy()
        best, idx = m.argmax()
        assert np.array_equal(got, gen), (rep, got, gen)
        assert idx == int(np.argmax(logits)) and bits_equal(np.float32(best), logits.max()), rep
        junk = [torch.full((64 << 20,), -1, dtype=torch.int8, device=cuda) for _ in range(8)]
        torch.cuda.synchronize()
        del junk
        torch.cuda.empty_cache()
    m.close()


def oracle_span(om, ids, pos, rows, record):
    """The oracle over positions [pos, pos + rows) in chunks of at most 32
    rows (its layout's seq), logits of the last row; records concatenated."""
    recs, logits, p = [], None, pos
    while p < pos + rows:
        n = min(32, pos + rows - p)
        last = p + n == pos + rows
        lg, rec = om.forward_chunk(ids[p:p + n], p, n, last, record=record)
        if record:
            recs.append(rec)
        if last:
            logits = lg
        p += n
    ref = {k: np.concatenate([r[k] for r in recs]) for k in recs[0]} if record else None
    return ref, logits


@pytest.mark.parametrize("packed", ["1", "0"])
@pytest.mark.parametrize("pos,rows", [(0, 100), (512, 88)])
def test_prefill_partial_tiles_and_offset(cuda, monkeypatch, packed, pos, rows):
    """Prefill chunks that do not fill the stream GEMM's 32-row tiles (rows
    past the chunk are computed on clamped rows and not stored), at position
    0 and at 512 after a 512-row chunk, on the weights packed at model open
    (default) and on the row-major blob (Q3_PACKED_WEIGHTS=0): every recorded
    stage of the chunk's last layer, both layers' K/V pages and scales for
    all positions so far, and the logits, against the oracle in 32-row chunks."""
    note(f"prefill chunk pos={pos} rows={rows} packed={packed}")
    monkeypatch.setenv("Q3_PACKED_WEIGHTS", packed)
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_512, init=INIT_512)
    om = oracle_512(blob, lay)
    ids = lay.global_views(blob)["ids"][:pos + rows].copy()
    if pos:
        oracle_span(om, ids, 0, pos, record=False)
    ref, logits = oracle_span(om, ids, pos, rows, record=True)
    m = Model(lay, blob)
    tab = np.arange(lay.max_seq // 32, dtype=np.uint16)
    np.random.default_rng(9).shuffle(tab)
    m.set_page_table(tab)
    if pos:
        m.forward_chunk(0, pos, LM_NONE, optimize_tail=False)
    m.forward_chunk(pos, rows, LM_LOGITS, optimize_tail=False)
    probs = []
    got = m.stage("logits", 1)[0]
    if not bits_equal(got, logits):
        probs.append(f"logits: {describe_diff(got, logits)}")
    for st in ("h", "h8", "hs", "q8", "qs", "o8", "os", "s8", "ss", "x"):
        g, e = m.stage(st, rows), ref[st]
        if st in ("q8", "qs"):  # row 0 doubles as the final-norm scratch (compare.py:197-205)
            g, e = g[1:], e[1:]
        if not bits_equal(g, e):
            probs.append(f"{st}: {describe_diff(g, e)}")
    for li in range(lay.layers):
        caches = m.kv_cache(li, pos + rows)
        for st, arr in (("kc", om.k8), ("ks", om.k_s), ("vc", om.v8), ("vs", om.v_s)):
            e = arr[li, :pos + rows]
            if not bits_equal(caches[st], e):
                probs.append(f"layer {li} {st}: {describe_diff(caches[st], e)}")
    m.close()
    assert not probs, probs


def test_repack_after_weight_write(cuda):
    """The packed copy is a snapshot taken at open: after new layer weights
    are written into the device blob, q3_model_repack refreshes it, and a
    100-row prefill chunk (packed path) then equals the oracle on the new
    weights bit for bit, logits and K/V pages."""
    note("weights rewritten after open + q3_model_repack")
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_512, init=INIT_512)
    _, other = host_blob("cfg3_perf", shape=SHAPE_512,
                         init=InitConfig(weight_seed=0x5EED0100, n_prompt=512, n_gen=4, mode=0))
    o = lay.offsets
    w0, w1 = o["kLAYERW_BASE"], o["kLAYERW_BASE"] + lay.layers * o["kLAYERW_STRIDE"]
    hybrid = blob.copy()
    hybrid[w0:w1] = other[w0:w1]
    om = oracle_512(hybrid, lay)
    ids = lay.global_views(hybrid)["ids"][:100].copy()
    _, logits = oracle_span(om, ids, 0, 100, record=False)
    m = Model(lay, blob)
    m.write(w0, other[w0:w1])
    m.repack()
    m.forward_chunk(0, 100, LM_LOGITS, optimize_tail=False)
    got = m.stage("logits", 1)[0]
    caches = [m.kv_cache(li, 100) for li in range(lay.layers)]
    m.close()
    assert bits_equal(got, logits), describe_diff(got, logits)
    for li in range(lay.layers):
        for st, arr in (("kc", om.k8), ("ks", om.k_s), ("vc", om.v8), ("vs", om.v_s)):
            assert bits_equal(caches[li][st], arr[li, :100]), (li, st)


def test_generate_300_token_prompt(cuda):
    """q3_generate with CTRL [300, 4, mode 0]: one 300-row prefill chunk (a
    partial last tile of the stream GEMMs, packed weights) and four greedy
    decode steps: the ids and the fused argmax equal the oracle's."""
    note("300-token prompt + 4 greedy tokens, 2 layers")
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_512, init=INIT_512)
    om = oracle_512(blob, lay)
    logits, gen, _, _ = om.generate(lay.global_views(blob)["ids"], 300, 4, record=False)
    m = Model(lay, blob)
    m.set_ctrl(300, 4, 0)
    m.generate()
    got = m.ids()[300:304].copy()
    best, idx = m.argmax()
    assert m.fused_status() == (3, 0)
    m.close()
    assert np.array_equal(got, gen), (got, gen)
    assert idx == int(np.argmax(logits)) and bits_equal(np.float32(best), logits.max())


SHAPE_1K = ModelShape(layers=2, vocab=1024, seq=512, max_seq=1056)
INIT_1K = InitConfig(weight_seed=0x5EED1000, n_prompt=1000, n_gen=4, mode=0)


def test_generate_1000_token_prompt_two_chunk_decode(cuda):
    """A 1000-token prompt (prefill chunks of 512 + 488) and four greedy
    decode steps at 1000-1003 keys: the fused b = 1 attention walks two
    chunks of key blocks per head (24 + 8), reusing its LDS stages in the
    second chunk and patching the new token's K/V row there.  The ids and the
    fused argmax equal the oracle's."""
    import oracle
    note("1000-token prompt + 4 greedy tokens, 2 layers (two-chunk decode attention)")
    lay, blob = host_blob("cfg3_perf", shape=SHAPE_1K, init=INIT_1K)
    dims = dict(SHAPE_1K.__dict__)
    dims["seq"] = 32
    om = oracle.OracleModel(blob, lay.offsets, dims)
    logits, gen, _, _ = om.generate(lay.global_views(blob)["ids"], 1000, 4, record=False)
    m = Model(lay, blob)
    m.set_ctrl(1000, 4, 0)
    m.generate()
    got = m.ids()[1000:1004].copy()
    best, idx = m.argmax()
    assert m.fused_status() == (3, 0)
    m.close()
    assert np.array_equal(got, gen), (got, gen)
    assert idx == int(np.argmax(logits)) and bits_equal(np.float32(best), logits.max())


def test_generate_decode_graph_replays(cuda, monkeypatch):
    """On a stream of its own, q3_generate captures its decode steps as one
    HIP graph and replays it while CTRL and the page table stay the same.
    Every replay, with eager work and synchronisations in between, gives the
    reference's ids and logits; a new CTRL mode or page table is captured
    anew; the launch-by-launch path (Q3_DECODE_GRAPH=0) agrees."""
    lay, blob = host_blob("cfg0")
    g = load_cfg("cfg0")
    gl = g["logits"]

    def run(m, mode):
        m.set_ctrl(40, 2, mode)
        m.generate()
        m.synchronize()
        ids = m.ids()[40:42].copy()
        if mode == 1:
            return ids, m.stage("logits", 1)[0].copy()
        return ids, m.argmax()

    def check_out(ids, out, mode, what):
        assert np.array_equal(ids, g["generated"]), (what, ids, g["generated"])
        if mode == 1:
            assert bits_equal(out, gl), (what, describe_diff(out, gl))
        else:
            best, idx = out
            assert idx == int(np.argmax(gl)) and bits_equal(np.float32(best), gl.max()), what

    results = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("Q3_DECODE_GRAPH", flag)
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            m = Model(lay, blob, stream=st)
        for rep in range(3):
            note(f"decode graph={flag} replay {rep}")
            ids, out = run(m, 1)
            check_out(ids, out, 1, f"graph={flag} mode 1 call {rep}")
            results.setdefault((flag, 1), []).append(out)
            # eager work on the model's stream and on another stream between replays
            m.forward_chunk(0, 32, LM_NONE)
            torch.randn(4096, device=cuda).sum().item()
            m.synchronize()
        ids, out = run(m, 0)
        check_out(ids, out, 0, f"graph={flag} mode 0")
        tab = np.arange(lay.max_seq // 32, dtype=np.uint16)
        np.random.default_rng(11).shuffle(tab)
        m.set_page_table(tab)
        for rep in range(2):
            ids, out = run(m, 1)
            check_out(ids, out, 1, f"graph={flag} shuffled pages call {rep}")
        m.close()
    assert all(bits_equal(a, b) for a, b in zip(results[("1", 1)], results[("0", 1)]))
