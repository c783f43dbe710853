"""Continuous-batching engine on the device (q3ops.engine.GpuGuest through the
C ABI) against the same engine driven by the oracle.

The oracle guest gives every request its own dense cache and runs
ref_qwen3.py:366-444 forward_chunk for each batch item; the device guest
runs all requests in one shared page pool (each through its own page table),
greedy decode rows batched in q3_decode_batch.  Requests mix greedy and
sampled decoding (temperature, top-k, top-p, repetition penalty, stop ids),
prompt lengths across page and chunk boundaries, and a pool small enough that
one request waits for pages.  Every generated id must be equal, and the
greedy ids must not depend on where the argmax runs.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3ops.engine import Engine, SamplingParams, make_gpu_engine  # noqa: E402
from q3ops.layout import InitConfig, Layout, ModelShape, init_random_blob  # noqa: E402
from q3ops.model import Model  # noqa: E402

SHAPE = ModelShape(layers=2, vocab=1024, seq=32, max_seq=320)  # 10 pages of 32
INIT = InitConfig(n_prompt=1, n_gen=0, mode=0)
_blob = {}


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def blob():
    if not _blob:
        lay = Layout(SHAPE)
        _blob["v"] = (lay, init_random_blob(lay, INIT))
    return _blob["v"]


def requests():
    rng = np.random.default_rng(77)

    def prompt(n):
        return [int(t) for t in rng.integers(0, SHAPE.vocab, size=n)]

    return [
        (prompt(5), SamplingParams(max_new=6)),
        (prompt(70), SamplingParams(max_new=6, temperature=0.8, top_k=40, seed=11)),
        (prompt(33), SamplingParams(max_new=5)),
        (prompt(20), SamplingParams(max_new=7, temperature=1.1, top_p=0.9,
                                    repetition_penalty=1.3, seed=7)),
        (prompt(32), SamplingParams(max_new=4, temperature=0.6, seed=5)),
        (prompt(64), SamplingParams(max_new=6)),
    ]


class OracleGuest:
    """Each request in its own oracle model (dense cache); logits for every
    item that needs them."""

    def __init__(self, lay: Layout, host_blob: np.ndarray):
        self.lay, self.blob = lay, host_blob
        self.models = {}

    def __call__(self, batch):
        out = {}
        for it in batch.items:
            om = self.models.get(it.req.rid)
            if om is None:
                om = self.models[it.req.rid] = oracle.OracleModel(
                    self.blob, self.lay.offsets, dict(SHAPE.__dict__))
            logits, _ = om.forward_chunk(np.array(it.token_ids, np.int32), it.pos, it.rows,
                                         it.needs_logits)
            if it.needs_logits:
                out[it.req.rid] = logits
        return out


def run(engine: Engine) -> dict:
    for p, sp in requests():
        engine.add_request(p, sp)
    engine.run(max_steps=500)
    return engine.outputs()


@pytest.fixture(scope="module")
def oracle_outputs():
    lay, hb = blob()
    eng = Engine(OracleGuest(lay, hb), num_pages=SHAPE.max_seq // 32, max_rows=32,
                 vocab=SHAPE.vocab)
    outs = run(eng)
    note(f"oracle engine: {eng.steps} steps, outputs {outs}")
    assert eng.pool.free_pages == SHAPE.max_seq // 32
    return outs, eng.steps


@pytest.mark.parametrize("greedy_on_device", [True, False])
def test_engine_matches_oracle(oracle_outputs, greedy_on_device):
    lay, hb = blob()
    note(f"engine on device: greedy_on_device={greedy_on_device}")
    m = Model(lay, hb)
    try:
        eng = make_gpu_engine(m, greedy_on_device=greedy_on_device)
        outs = run(eng)
        guest = eng.guest_step
        note(f"device engine: {eng.steps} steps, launches {guest.launches}")
    finally:
        m.close()
    exp, steps = oracle_outputs
    assert outs == exp
    assert eng.steps == steps
    assert eng.pool.free_pages == SHAPE.max_seq // 32
    if greedy_on_device:
        assert guest.launches["decode_batch"] > 0
