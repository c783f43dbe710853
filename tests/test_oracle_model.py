"""The CPU oracle's model path (forward_chunk / generate) against the golden
stage records of tools/ref_qwen3.py on the random-init configs."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import bits_equal, describe_diff
from paritylib import STAGES, compare_stage, load_cfg, sha
from q3ops.layout import CONFIGS, Layout, init_random_blob


@pytest.fixture(scope="module", autouse=True)
def built():
    oracle.build()


_blobs = {}


def model_for(name: str, gold_meta):
    if name not in _blobs:
        shape, init = CONFIGS[name]
        lay = Layout(shape)
        blob = init_random_blob(lay, init)
        assert sha(blob[lay["kEMB"]:lay["kLOGITS"]]) == gold_meta[name]["weights_sha256"]
        dims = dict(shape.__dict__)
        _blobs[name] = (lay, blob, oracle.OracleModel(blob, lay.offsets, dims), init)
    return _blobs[name]


def record_problems(g, prefix: str, rec: dict, caches: dict, kv_len: int) -> list[str]:
    probs = []
    for st in STAGES:
        if st in ("kc", "ks", "vc", "vs"):
            got = caches[st][:kv_len]
        else:
            got = rec[st]
        p = compare_stage(g, prefix, st, got)
        if p:
            probs.append(p)
    return probs


def caches_of(om: oracle.OracleModel, layer: int) -> dict:
    return {"kc": om.k8[layer], "ks": om.k_s[layer], "vc": om.v8[layer], "vs": om.v_s[layer]}


def test_cfg0_generate(gold_meta):
    lay, blob, om, init = model_for("cfg0", gold_meta)
    g = load_cfg("cfg0")
    ids = lay.global_views(blob)["ids"]
    logits, gen, rec, ids_out = om.generate(ids, init.n_prompt, init.n_gen, record=True)
    assert bits_equal(logits.reshape(1, -1)[0], g["logits"]), describe_diff(logits, g["logits"])
    assert np.array_equal(gen, g["generated"])
    total = init.n_prompt + init.n_gen
    last = int(g["n_forwards_with_logits"]) - 1
    probs = record_problems(g, f"f{last}_", rec, caches_of(om, 0), total)
    assert not probs, probs


def test_cfg0_each_forward(gold_meta):
    """Step the reference loop chunk by chunk: chunk 0 (32 rows, no logits),
    chunk 1 (8 rows) and the two decode steps, every last-layer stage."""
    lay, blob, om, init = model_for("cfg0", gold_meta)
    g = load_cfg("cfg0")
    om.reset_cache()
    ids = np.array(g["ids_in"], np.int32).copy()
    ids[init.n_prompt:] = g["generated"]
    steps = [(0, 32, False, "c0_"), (32, 8, True, "f0_"), (40, 1, True, "f1_"),
             (41, 1, True, "f2_")]
    for pos, rows, want, prefix in steps:
        logits, rec = om.forward_chunk(ids[pos:pos + rows], pos, rows, want, record=True)
        probs = record_problems(g, prefix, rec, caches_of(om, 0), pos + rows)
        if want:
            gl = g[f"{prefix}logits"].reshape(-1)
            if not bits_equal(logits, gl):
                probs.append(f"{prefix}logits: {describe_diff(logits, gl)}")
        assert not probs, (prefix, probs)


def test_cfg2_full_depth_logits(gold_meta):
    lay, blob, om, init = model_for("cfg2", gold_meta)
    g = load_cfg("cfg2")
    om.reset_cache()
    ids = lay.global_views(blob)["ids"]
    logits, gen, rec, _ = om.generate(ids, init.n_prompt, init.n_gen, record=True)
    assert bits_equal(logits, g["logits"]), describe_diff(logits, g["logits"])
    probs = record_problems(g, "f0_", rec, caches_of(om, lay.layers - 1), init.n_prompt)
    assert not probs, probs


def test_cfg3_greedy_ids(gold_meta):
    lay, blob, om, init = model_for("cfg3", gold_meta)
    g = load_cfg("cfg3")
    om.reset_cache()
    ids = lay.global_views(blob)["ids"]
    logits, gen, rec, _ = om.generate(ids, init.n_prompt, init.n_gen, record=True)
    assert np.array_equal(gen, g["generated"]), (gen, g["generated"])
    assert bits_equal(logits, g["logits"]), describe_diff(logits, g["logits"])
    last = int(g["n_forwards_with_logits"]) - 1
    probs = record_problems(g, f"f{last}_", rec, caches_of(om, lay.layers - 1),
                            init.n_prompt + init.n_gen)
    assert not probs, probs


def test_chunk_size_invariance_oracle(gold_meta):
    """The 40-token prompt as one 40-row chunk gives the same int8 stages,
    logits and ids as the reference's 32+8 chunking."""
    lay, blob, om, init = model_for("cfg0", gold_meta)
    g = load_cfg("cfg0")
    shape = dict(om.dims)
    shape["seq"] = 64
    big = oracle.OracleModel(blob, lay.offsets, shape)  # same weights, larger chunks
    ids = lay.global_views(blob)["ids"]
    logits, gen, rec, _ = big.generate(ids, init.n_prompt, init.n_gen, record=True)
    assert np.array_equal(gen, g["generated"])
    assert bits_equal(logits, g["logits"])
