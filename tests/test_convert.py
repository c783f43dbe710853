"""PQWF converter (q3ops.convert; tools/convert_pqwf.py, tools/pqwf.py) on a
synthetic Qwen3-shaped checkpoint: BF16 safetensors with the Hugging Face
tensor names, one layer, a 1024-row vocabulary.

Pinned by: a numpy restatement of pqwf.py:344-360's per-row quantiser (its
numpy operations, independent of the C++ quantiser the converter calls), the
quantiser's closed-form properties (|q| <= 127 with 127 reached, error within
half a step plus the quotient rounding, zero rows, ties to even), the placement of every tensor in
the blob (through the layout's typed views, byte offsets pinned by the
layout tests), the RoPE tables' closed form, and on the GPU a generation on
the converted blob equal to the oracle's."""
from __future__ import annotations

import json

import numpy as np
import pytest

torch = pytest.importorskip("torch")
safetensors_torch = pytest.importorskip("safetensors.torch")

from q3ops.convert import convert, parse_ids, rope_tables  # noqa: E402
from q3ops.layout import Layout  # noqa: E402

H, HEADS, KVH, HD, I, V = 1024, 16, 8, 128, 3072, 1024
KINV127 = np.float32(1.0) / np.float32(127.0)


def make_checkpoint(d, tied: bool, seed: int = 5):
    g = torch.Generator().manual_seed(seed)

    def w(rows, cols, std=0.02):
        return (torch.randn(rows, cols, generator=g) * std).to(torch.bfloat16)

    def gain(n):
        return (1 + 0.05 * torch.randn(n, generator=g)).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": w(V, H), "model.norm.weight": gain(H)}
    if not tied:
        t["lm_head.weight"] = w(V, H)
    p = "model.layers.0."
    t[p + "self_attn.q_proj.weight"] = w(HEADS * HD, H)
    t[p + "self_attn.k_proj.weight"] = w(KVH * HD, H)
    t[p + "self_attn.v_proj.weight"] = w(KVH * HD, H)
    t[p + "self_attn.o_proj.weight"] = w(H, HEADS * HD)
    gate = w(I, H)
    gate[0].zero_()                       # zero row: scale 0, all-zero ints
    gate[1] = 0
    gate[1, 0], gate[1, 1] = 127.0, 0.5   # scale 1 -> 0.5 is a tie (to even: 0)
    gate[1, 2] = -2.5                     # tie: -2
    gate[2, 5] = 1e4                      # one dominant value, the rest tiny
    t[p + "mlp.gate_proj.weight"] = gate
    t[p + "mlp.up_proj.weight"] = w(I, H)
    t[p + "mlp.down_proj.weight"] = w(H, I)
    for nm, n in (("input_layernorm", H), ("post_attention_layernorm", H),
                  ("self_attn.q_norm", HD), ("self_attn.k_norm", HD)):
        t[p + nm + ".weight"] = gain(n)
    safetensors_torch.save_file(t, str(d / "model.safetensors"))
    cfg = {"hidden_size": H, "num_hidden_layers": 1, "num_attention_heads": HEADS,
           "num_key_value_heads": KVH, "head_dim": HD, "intermediate_size": I,
           "vocab_size": V, "rope_theta": 1000000.0, "tie_word_embeddings": tied}
    (d / "config.json").write_text(json.dumps(cfg))
    return {k: v.to(torch.float32).numpy() for k, v in t.items()}


def pqwf_quantize(block: np.ndarray):
    """pqwf.py:349-358 in numpy: per-row absmax * (1/127), f32 quotient,
    rint, NaN -> 0, clip."""
    absmax = np.max(np.abs(block), axis=1).astype(np.float32)
    scale = (absmax * KINV127).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        quot = (block / scale[:, None]).astype(np.float32)
    q = np.where(np.isnan(quot), np.float32(0), np.rint(quot))
    return np.clip(q, -127, 127).astype(np.int8), scale


@pytest.fixture(scope="module", params=[False, True], ids=["untied", "tied"])
def converted(request, tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    src = make_checkpoint(d, tied=request.param)
    lay, blob = convert(d, seq=32, max_seq=256, n_prompt=12, n_gen=3, out=d / "blob.bin")
    return request.param, src, lay, np.asarray(blob)


def test_weights_match_pqwf_quantiser(converted):
    tied, src, lay, blob = converted
    w = lay.weight_views(blob, 0)
    g = lay.global_views(blob)
    p = "model.layers.0."
    pairs = [(g["emb8"], g["emb_s"], src["model.embed_tokens.weight"]),
             (g["lm8"], g["lm_s"], src["model.embed_tokens.weight" if tied else "lm_head.weight"])]
    for proj, mod, key in (("q_proj", "self_attn", "wq"), ("k_proj", "self_attn", "wk"),
                           ("v_proj", "self_attn", "wv"), ("o_proj", "self_attn", "wo"),
                           ("gate_proj", "mlp", "wg"), ("up_proj", "mlp", "wu"),
                           ("down_proj", "mlp", "wd")):
        pairs.append((w[key], w[key + "_s"], src[f"{p}{mod}.{proj}.weight"]))
    for q, s, ref in pairs:
        eq, es = pqwf_quantize(ref)
        assert np.array_equal(q, eq)
        assert np.array_equal(s.view(np.uint32), es.view(np.uint32))
    for nm, key in (("input_layernorm", "n1"), ("self_attn.q_norm", "nq"),
                    ("self_attn.k_norm", "nk"), ("post_attention_layernorm", "n2")):
        assert np.array_equal(w[key], src[f"{p}{nm}.weight"])
    assert np.array_equal(g["nf"], src["model.norm.weight"])


def test_quantiser_properties(converted):
    _, src, lay, blob = converted
    w = lay.weight_views(blob, 0)
    q, s = w["wg"].astype(np.int32), w["wg_s"]
    ref = src["model.layers.0.mlp.gate_proj.weight"]
    nz = s > 0
    assert np.all(np.abs(q) <= 127) and np.all(np.abs(q[nz]).max(axis=1) == 127)
    err = np.abs(q * s[:, None].astype(np.float64) - ref)
    # half a step, plus the f32 rounding of the quotient (|q| <= 128 ulps of
    # 2^-24): an f32 quotient of exactly k + 0.5 may stand for a true value
    # just past the midpoint
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 128 * 2.0 ** -24))
    assert s[0] == 0 and not q[0].any()                         # zero row
    assert s[1] == np.float32(np.float32(127) * KINV127)
    assert (q[1, 0], q[1, 1], q[1, 2]) == (127, 0, -2)          # ties to even
    assert q[2, 5] == 127 and np.count_nonzero(q[2]) == 1       # one dominant value


def test_tables_ids_ctrl(converted):
    _, _, lay, blob = converted
    g = lay.global_views(blob)
    cos, sin = g["cos"], g["sin"]
    half = HD // 2
    pos, i = 37, 5
    ang = pos * (1.0 / (1e6 ** (i / half)))
    assert cos[pos, i] == np.float32(np.cos(ang)) and sin[pos, i] == np.float32(np.sin(ang))
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    assert np.allclose(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2, 1, atol=1e-6)
    c2, s2 = rope_tables(256, HD, 1e6)
    assert np.array_equal(cos, c2) and np.array_equal(sin, s2)
    assert list(g["ids"][:15]) == [100 + 10 * k for k in range(15)]
    assert list(g["ctrl"]) == [12, 3, 256, 0]


def test_parse_ids():
    assert parse_ids("", 3) == [100, 110, 120]
    assert parse_ids("5, 6", 4) == [5, 6, 0, 0]
    assert parse_ids("1,2,3", 2) == [1, 2]


@pytest.mark.gpu
def test_converted_blob_generates_like_oracle(converted):
    """The converted model on the device: q3_generate ids and the last
    logits' argmax equal the oracle's on the same blob."""
    import oracle
    from q3ops.model import Model
    tied, _, lay, blob = converted
    host = np.ascontiguousarray(blob[:lay.size])
    print(f"converted ({'tied' if tied else 'untied'}): generate 12 + 3 on the device", flush=True)
    m = Model(lay, host)
    try:
        m.generate()
        ids = m.ids()[:15].copy()
    finally:
        m.close()
    om = oracle.OracleModel(host, lay.offsets, dict(lay.shape.__dict__))
    _, gen, _, _ = om.generate(host[lay["kIDS"]:lay["kIDS"] + 4 * 15].view(np.int32), 12, 3,
                               record=False)
    assert list(ids[12:]) == [int(t) for t in gen]
