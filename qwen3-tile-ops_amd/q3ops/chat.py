"""Text in / text out on the device model (tools/run_chat.py).

The prompt is wrapped in the ChatML user turn (unless raw), tokenised, and
written with CTRL = [n_prompt, max_new, max_seq, 0] into the blob; q3_generate
then runs the chunked prefill and the greedy decode loop on the device (the
lm_head argmax stays there) and the host decodes the ids up to the first
end-of-turn id.

    python -m q3ops.chat "text" --model-dir DIR [--tokenizer DIR/tokenizer.json]
        [--blob converted.bin] [--max-new 16] [--max-seq 1024] [--raw | --ids 1,2]
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np

__all__ = ["EOS_IDS", "generate_ids", "main"]

EOS_IDS = {151645, 151643}  # <|im_end|>, <|endoftext|> (run_chat.py:25)


def generate_ids(model, prompt_ids, max_new: int) -> list:
    """Greedy continuation of prompt_ids on the device (q3_generate)."""
    L = model.layout
    n = len(prompt_ids)
    if n < 1 or n + max_new > L.max_seq:
        raise ValueError(f"prompt {n} + max_new {max_new} must fit max_seq {L.max_seq}")
    model.set_ids(list(prompt_ids))
    model.set_ctrl(n, max_new, 0)
    model.generate()
    return [int(t) for t in model.ids()[n:n + max_new]]


def cut_at_eos(ids, eos=EOS_IDS) -> list:
    out = []
    for t in ids:
        if t in eos:
            break
        out.append(t)
    return out


def main(argv=None) -> int:
    from .convert import convert
    from .layout import Layout, ModelShape
    from .model import Model
    from .tokenizer import Tokenizer, chatml
    ap = argparse.ArgumentParser(description="greedy chat on the device model")
    ap.add_argument("text", nargs="?", default="Hello, who are you?")
    ap.add_argument("--model-dir", required=True, help="Hugging Face checkpoint directory")
    ap.add_argument("--tokenizer", default="", help="tokenizer.json (default: in --model-dir)")
    ap.add_argument("--blob", default="", help="a blob converted with the same --seq/--max-seq")
    ap.add_argument("--seq", type=int, default=32)
    ap.add_argument("--max-seq", type=int, default=1024)
    ap.add_argument("--max-new", type=int, default=16)
    ap.add_argument("--raw", action="store_true", help="do not wrap the text in ChatML")
    ap.add_argument("--ids", default="", help="prompt ids instead of the text")
    a = ap.parse_args(argv)
    tok = Tokenizer(a.tokenizer or Path(a.model_dir) / "tokenizer.json")
    if a.ids:
        prompt = [int(t) for t in a.ids.split(",") if t.strip()]
    else:
        prompt = tok.encode(a.text if a.raw else chatml(a.text))
    if a.blob:
        import json
        cfg = json.loads((Path(a.model_dir) / "config.json").read_text())
        lay = Layout(ModelShape(hidden=cfg["hidden_size"], layers=cfg["num_hidden_layers"],
                                heads=cfg["num_attention_heads"],
                                kv_heads=cfg["num_key_value_heads"], head_dim=cfg["head_dim"],
                                inter=cfg["intermediate_size"], vocab=cfg["vocab_size"],
                                seq=a.seq, max_seq=a.max_seq))
        blob = np.fromfile(a.blob, dtype=np.uint8)
        if blob.size < lay.size:
            print(f"error: {a.blob} holds {blob.size} bytes, the layout needs {lay.size}",
                  file=sys.stderr)
            return 2
    else:
        lay, blob = convert(a.model_dir, seq=a.seq, max_seq=a.max_seq)
    m = Model(lay, np.ascontiguousarray(blob[:lay.size]))
    try:
        gen = generate_ids(m, prompt, a.max_new)
    finally:
        m.close()
    kept = cut_at_eos(gen)
    print(f"prompt ids ({len(prompt)}): {prompt}")
    print(f"generated ids: {gen}")
    print(tok.decode(kept))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
