"""Host engine (tools/engine.py) on the CPU: the reference's own engine check
(tools/check_engine.py: mock guest, three requests, chunked prefill, pages
freed), with the exact ids that its mock guest fixes, plus the sampler's and
scheduler's properties."""
from __future__ import annotations

import numpy as np
import pytest

from q3ops.engine import Batch, Engine, PagePool, Request, SamplingParams, Sampler, State


def mock_guest(batch: Batch) -> dict:
    """check_engine.py:12-21: a one-hot logit row whose hot id depends on the
    request id, its generated count and the item's row count."""
    out = {}
    for it in batch.items:
        if it.needs_logits:
            x = np.full(32, -100.0)
            x[(it.req.rid * 7 + len(it.req.generated) + it.rows) % 32] = 100.0
            out[it.req.rid] = x
    return out


def test_reference_engine_check():
    # check_engine.py:24-36
    eng = Engine(mock_guest, num_pages=8, max_rows=32, vocab=32)
    p = SamplingParams(max_new=4, temperature=0)
    a = eng.add_request([1, 2, 3, 4, 5], p)
    b = eng.add_request(list(range(70)), SamplingParams(max_new=4, temperature=0))
    c = eng.add_request(list(range(33)), SamplingParams(max_new=4, temperature=0))
    batches = []
    orig = eng.guest_step

    def spy(batch):
        batches.append([(it.req.rid, it.rows, it.pos, it.prefill, it.needs_logits)
                        for it in batch.items])
        return orig(batch)

    eng.guest_step = spy
    eng.run(max_steps=100)
    outs = eng.outputs()
    assert all(len(outs[r.rid]) == 4 for r in (a, b, c)), outs
    assert eng.pool.free_pages == 8
    assert a.done and b.done and c.done
    # The ids the mock fixes: the first id comes from the last prefill chunk
    # (rows = its size), then one id per decode row (rows = 1, generated g).
    # Batches of 32 rows: a 5 + b 27; a 1 + b 31; a 1 + b 12 + c 19;
    # a 1 + b 1 + c 14; then decode rows only.
    assert batches[0] == [(0, 5, 0, True, True), (1, 27, 0, True, False)]
    assert batches[1] == [(0, 1, 5, False, True), (1, 31, 27, True, False)]
    assert batches[2] == [(0, 1, 6, False, True), (1, 12, 58, True, True), (2, 19, 0, True, False)]
    assert batches[3] == [(0, 1, 7, False, True), (1, 1, 70, False, True), (2, 14, 19, True, True)]
    assert outs[a.rid] == [5, 2, 3, 4]
    assert outs[b.rid] == [(7 + 12) % 32, 9, 10, 11]
    assert outs[c.rid] == [(14 + 14) % 32, 16, 17, 18]
    assert eng.steps == 7
    assert all(sum(r for _, r, *_ in bt) <= 32 for bt in batches)


def test_pool_exhaustion_defers_request():
    """Two pages: b's page request fails while a holds both, so b waits and
    runs only once a has finished and released them."""
    eng = Engine(mock_guest, num_pages=2, max_rows=32, vocab=32)
    a = eng.add_request(list(range(40)), SamplingParams(max_new=4))
    b = eng.add_request(list(range(10)), SamplingParams(max_new=3))
    rids = []
    orig = eng.guest_step
    eng.guest_step = lambda bt: (rids.append({it.req.rid for it in bt.items}), orig(bt))[1]
    eng.run()
    first_b = next(i for i, s in enumerate(rids) if b.rid in s)
    last_a = max(i for i, s in enumerate(rids) if a.rid in s)
    assert first_b > last_a
    assert len(eng.outputs()[a.rid]) == 4 and len(eng.outputs()[b.rid]) == 3
    assert eng.pool.free_pages == 2 and not eng.pool.used


def test_pool_lifo_order():
    pool = PagePool(4)
    r = Request(0, [1] * 70, SamplingParams())
    assert pool.ensure(r, 70) and r.pages == [3, 2, 1]
    s = Request(1, [1], SamplingParams())
    assert pool.ensure(s, 33) is False and s.pages == [0]  # partial, as the reference
    pool.release(r)
    assert pool.free == [3, 2, 1] and pool.free_pages == 3
    assert pool.alloc_page() == 1


def test_max_rows_bounds_chunks():
    eng = Engine(mock_guest, num_pages=16, max_rows=8, vocab=32)
    reqs = [eng.add_request(list(range(n)), SamplingParams(max_new=3)) for n in (20, 9, 3)]
    seen = []
    orig = eng.guest_step
    eng.guest_step = lambda b: (seen.append(b.total_rows), orig(b))[1]
    eng.run()
    assert max(seen) <= 8
    assert all(len(eng.outputs()[r.rid]) == 3 for r in reqs)


def test_stop_token_finishes():
    eng = Engine(mock_guest, num_pages=4, max_rows=32, vocab=32)
    # rid 0, prompt 5: first id (0 + 0 + 5) % 32 = 5, then 2, 3, ...
    r = eng.add_request([9] * 5, SamplingParams(max_new=10, stop_tokens={2}))
    eng.run()
    assert eng.outputs()[r.rid] == [5, 2] and r.state == State.FINISHED


# ---- sampler -----------------------------------------------------------------
def _req(**kw) -> Request:
    return Request(0, [0], SamplingParams(**kw))


def test_sampler_greedy_first_index():
    x = np.array([0.5, 2.0, -1.0, 2.0], np.float32)
    assert Sampler().sample(x, _req(temperature=0.0)) == 1
    assert Sampler().sample(x, _req(temperature=-1.0, top_k=1)) == 1


@pytest.mark.parametrize("seed", range(5))
def test_sampler_reduces_to_argmax(seed):
    rng = np.random.default_rng(100 + seed)
    x = rng.normal(size=257).astype(np.float32)
    best = int(np.argmax(x))
    assert Sampler().sample(x, _req(temperature=0.7, top_k=1, seed=seed)) == best
    assert Sampler().sample(x, _req(temperature=1.3, top_p=1e-9, seed=seed)) == best


def test_sampler_inverse_cdf_draw():
    """temperature 1, no masks: the draw is the inverse CDF of one uniform of
    the request's PCG64 stream (numpy Generator.choice with p)."""
    p = np.array([0.1, 0.25, 0.05, 0.4, 0.2])
    x = np.log(p)
    for seed in range(20):
        got = Sampler().sample(x, _req(temperature=1.0, seed=seed))
        q = np.exp(x - x.max())
        q /= q.sum()
        cdf = np.cumsum(q)
        cdf /= cdf[-1]
        u = np.random.default_rng(seed).random()
        assert got == int(np.searchsorted(cdf, u, side="right"))


def test_sampler_temperature_distribution():
    p = np.array([0.5, 0.3, 0.2])
    x = np.log(p)
    for t, expect in ((1.0, p), (2.0, np.sqrt(p) / np.sqrt(p).sum())):
        r = _req(temperature=t, seed=3)
        n = 20000
        counts = np.bincount([Sampler().sample(x, r) for _ in range(n)], minlength=3)
        assert np.all(np.abs(counts / n - expect) < 0.015), (t, counts / n, expect)


def test_sampler_top_k_and_top_p_support():
    x = np.log(np.array([0.05, 0.4, 0.1, 0.3, 0.15]))
    r = _req(temperature=1.0, top_k=2, seed=1)
    got = {Sampler().sample(x, r) for _ in range(400)}
    assert got == {1, 3}
    # nucleus: sorted masses 0.4, 0.3, 0.15, ... (cumulative 0.4, 0.7, 0.85):
    # top_p 0.75 keeps ids 1 and 3
    r = _req(temperature=1.0, top_p=0.75, seed=2)
    got = {Sampler().sample(x, r) for _ in range(400)}
    assert got == {1, 3}
    # the first id survives even when its own mass exceeds top_p
    r = _req(temperature=1.0, top_p=0.1, seed=2)
    assert {Sampler().sample(x, r) for _ in range(50)} == {1}


def test_sampler_repetition_penalty():
    # positive logit divided, negative logit multiplied (each id once)
    x = np.array([2.0, 1.9, -5.0])
    r = _req(temperature=1.0, top_k=1, repetition_penalty=2.0)
    r.generated = [0, 0]
    assert Sampler().sample(x, r) == 1  # 2.0 / 2 < 1.9
    x = np.array([-1.0, -1.5, -9.0])
    r = _req(temperature=1.0, top_k=1, repetition_penalty=2.0)
    r.generated = [0]
    assert Sampler().sample(x, r) == 1  # -1.0 * 2 < -1.5
    r.generated = []
    assert Sampler().sample(x, r) == 0


def test_engine_rejects_device_id_for_sampled_request():
    def guest(batch):
        return {it.req.rid: 3 for it in batch.items if it.needs_logits}

    eng = Engine(guest, num_pages=2, vocab=32)
    eng.add_request([1, 2], SamplingParams(temperature=0.5))
    with pytest.raises(ValueError):
        eng.run()
