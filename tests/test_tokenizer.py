"""Tokenizer (q3ops.tokenizer; tools/tokenizer.py) and the chat path
(q3ops.chat; tools/run_chat.py).

Pinned by: the GPT-2 byte alphabet's known code points, a hand-built
tokenizer.json whose ids follow from its merge ranks by hand, and agreement
with the Hugging Face ``tokenizers`` library (an independent implementation
of the same pipeline) on a byte-level BPE trained here with the Qwen2 split
pattern, over texts that exercise every branch of the pattern, special
tokens and round trips.  On the GPU the chat helper's greedy ids equal the
oracle's for the tokenised ChatML prompt."""
from __future__ import annotations

import json

import numpy as np
import pytest

from q3ops.tokenizer import SPLIT_PATTERN, Tokenizer, byte_alphabet, chatml

tokenizers = pytest.importorskip("tokenizers")

SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
CORPUS = [
    "Hello world! It's a test, isn't it? We'll see; they'd know.",
    "The quick brown fox jumps over the lazy dog 1234567890 times.",
    "def f(x):\n    return x ** 2  # square\n\n\nprint(f(3))\r\n",
    "你好，请用一句话介绍你自己。今天天气很好！",
    "Ünïcödé façade naïve café — “quotes” and ‘apostrophes’ … ✓ 😀🚀",
    "tabs\tand   multiple    spaces   \n  leading and trailing  ",
    "URLs: https://example.com/path?q=1&r=two#frag, emails a.b@c.de",
    "Numbers 3.14159, -42, 1e-6, 0xFF and ১২৩ (Bengali digits) ٣٤٥",
] * 20
TEXTS = [
    "Hello, world!", "It's", "I'M here", "they'RE", "  two spaces", "trailing   ",
    "line\nbreak\r\n\r\nwindows", "x = [1, 2, 3]\n\tindent", "你好世界", "café 😀 ok",
    "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", "123456", "a1b2c3",
    "!!!???...", " ?!x", "\n\n\n", "mixed<|im_end|>special<|endoftext|>end", "",
    "Numbers 3.14159, -42", "emails a.b@c.de https://x.y/z?q=1",
]


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    from tokenizers import Regex, decoders, models, pre_tokenizers, trainers
    tk = tokenizers.Tokenizer(models.BPE())
    tk.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(SPLIT_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tk.decoder = decoders.ByteLevel()
    tr = trainers.BpeTrainer(vocab_size=900, special_tokens=SPECIALS,
                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                             show_progress=False)
    tk.train_from_iterator(CORPUS, trainer=tr)
    path = tmp_path_factory.mktemp("tok") / "tokenizer.json"
    tk.save(str(path))
    return path, tk


def test_byte_alphabet_known_points():
    a = byte_alphabet()
    assert len(set(a.values())) == 256
    assert a[ord("A")] == "A" and a[0xA1] == "\xa1" and a[0xFF] == "\xff"
    assert a[0x20] == "Ġ" and a[0x0A] == "Ċ" and a[0x00] == "Ā"
    assert a[0xAD] == "Ń"  # the 68th and last remapped byte


def test_hand_built_merges(tmp_path):
    a = byte_alphabet()
    vocab = {a[b]: b for b in range(256)}
    for t in ("he", "ll", "hell", "Ġw", "or"):
        vocab[t] = len(vocab)
    vocab["<|im_end|>"] = len(vocab)
    spec = {"model": {"type": "BPE", "vocab": vocab,
                      "merges": ["h e", "l l", "he ll", "Ġ w", "o r"]},
            "added_tokens": [{"id": vocab["<|im_end|>"], "content": "<|im_end|>"}]}
    p = tmp_path / "tokenizer.json"
    p.write_text(json.dumps(spec))
    tok = Tokenizer(p)
    # "hello" -> h e l l o -> he l l o -> he ll o -> hell o
    # " world" -> Ġ w o r l d -> Ġw o r l d -> Ġw or l d
    assert tok.encode("hello world<|im_end|>") == [
        vocab["hell"], ord("o"), vocab["Ġw"], vocab["or"], ord("l"), ord("d"),
        vocab["<|im_end|>"]]
    assert tok.decode(tok.encode("hello world<|im_end|>")) == "hello world<|im_end|>"


def test_matches_hf_tokenizers(trained):
    path, hf = trained
    tok = Tokenizer(path)
    for t in TEXTS + CORPUS[:8]:
        assert tok.encode(t) == hf.encode(t).ids, t
        assert tok.decode(tok.encode(t)) == t


def test_chat_template_tokens(trained):
    path, _ = trained
    tok = Tokenizer(path)
    ids = tok.encode(chatml("hi"))
    sp = {s: tok.special[s] for s in SPECIALS}
    assert ids[0] == sp["<|im_start|>"] and sp["<|im_end|>"] in ids
    assert tok.eos_id == sp["<|im_end|>"]


@pytest.mark.gpu
def test_chat_generates_like_oracle(trained, tmp_path):
    """ChatML prompt -> ids -> q3_generate on a converted synthetic
    checkpoint; the greedy ids equal the oracle's."""
    import oracle
    from q3ops.chat import generate_ids
    from q3ops.convert import convert
    from q3ops.model import Model
    from test_convert import make_checkpoint
    path, _ = trained
    make_checkpoint(tmp_path, tied=True, seed=21)
    tok = Tokenizer(path)
    prompt = tok.encode(chatml("What is 2 + 2? Answer briefly."))
    assert max(prompt) < 1024
    lay, blob = convert(tmp_path, seq=32, max_seq=256)
    host = np.ascontiguousarray(blob[:lay.size])
    print(f"chat: prompt of {len(prompt)} ids, 6 new", flush=True)
    m = Model(lay, host)
    try:
        got = generate_ids(m, prompt, 6)
    finally:
        m.close()
    om = oracle.OracleModel(host, lay.offsets, dict(lay.shape.__dict__))
    _, gen, _, _ = om.generate(np.array(prompt, np.int32), len(prompt), 6, record=False)
    assert got == [int(t) for t in gen]
    assert isinstance(tok.decode([t for t in got if t < 900]), str)
