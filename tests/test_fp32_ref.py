"""Model-level drift check (q3ops.fp32_ref; tools/fp32_ref.py): an f32 Qwen3
forward from the unquantised checkpoint.

The f32 model shares no code with the int8 path, so its agreement with the
W8A8 oracle up to quantisation noise pins it to the same model (embedding,
norms, RoPE, GQA attention, SwiGLU, lm_head); a mistake planted in the f32
model (RoPE rotating the wrong way) must break that agreement, which shows
the bound can fail.  On the GPU the device logits are compared the same way
(the drift the tool reports).  Float tolerances: cosine >= 0.995 and
relative L2 error <= 0.1 of the last row's logits."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("safetensors")

import oracle  # noqa: E402
from q3ops.convert import convert  # noqa: E402
from q3ops.fp32_ref import F32Model, compare_device, drift_stats  # noqa: E402
from test_convert import make_checkpoint  # noqa: E402

IDS = [3, 517, 88, 1000, 42, 7, 7, 250, 901, 12, 640, 333]
COS_MIN, REL_MAX = 0.995, 0.1


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("f32ckpt")
    make_checkpoint(d, tied=False, seed=9)
    return d


@pytest.fixture(scope="module")
def oracle_last_logits(ckpt):
    lay, blob = convert(ckpt, seq=32, max_seq=256, n_prompt=len(IDS))
    om = oracle.OracleModel(np.ascontiguousarray(blob), lay.offsets, dict(lay.shape.__dict__))
    logits, _ = om.forward_chunk(np.array(IDS, np.int32), 0, len(IDS), True)
    return logits


def test_f32_model_agrees_with_w8a8_oracle(ckpt, oracle_last_logits):
    ref = F32Model(ckpt, device="cpu").forward(IDS)
    assert ref.shape == (len(IDS), 1024) and np.all(np.isfinite(ref))
    st = drift_stats(ref[-1], oracle_last_logits)
    print("f32 vs W8A8 oracle:", st)
    assert st["cosine"] >= COS_MIN and st["rel_l2"] <= REL_MAX, st


def test_planted_rope_mistake_is_caught(ckpt, oracle_last_logits):
    m = F32Model(ckpt, device="cpu")
    m.rope_sign = -1.0
    st = drift_stats(m.forward(IDS)[-1], oracle_last_logits)
    print("planted mistake:", st)
    assert st["cosine"] < COS_MIN or st["rel_l2"] > REL_MAX, st


def test_first_row_is_position_independent(ckpt):
    # row 0 attends to itself only: its logits do not depend on later ids
    m = F32Model(ckpt, device="cpu")
    a, b = m.forward(IDS)[0], m.forward(IDS[:1] + [5] * 7)[0]
    assert np.array_equal(a, b)


def test_drift_stats_identity():
    x = np.linspace(-1, 1, 64)
    st = drift_stats(x, x)
    assert st["max_abs"] == 0 and st["rel_l2"] == 0 and st["top1_equal"] and st["top5_overlap"] == 5
    assert abs(st["cosine"] - 1) < 1e-12


@pytest.mark.gpu
def test_device_drift_report(ckpt):
    print("device W8A8 vs f32 (12-token prompt, 1 layer)", flush=True)
    st = compare_device(ckpt, IDS)
    print("device drift:", st, flush=True)
    assert st["cosine"] >= COS_MIN and st["rel_l2"] <= REL_MAX, st
