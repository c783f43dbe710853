"""Qwen3 byte-level BPE tokenizer over a Hugging Face tokenizer.json
(tools/tokenizer.py:39-173).

Pipeline, as the reference's (which restates the Hugging Face fast
tokenizer for Qwen2/Qwen3):

1. special tokens (``added_tokens``) are matched literally, leftmost and
   longest first, and become their ids;
2. the text between them is split by the Qwen2 pre-tokenizer pattern
   (contractions, letter runs with one optional leading non-letter, single
   digits, symbol runs with trailing newlines, newline runs, spaces);
3. each piece is UTF-8 encoded and mapped byte by byte to the GPT-2
   printable alphabet;
4. BPE: the adjacent pair with the lowest merge rank is merged until none
   applies; the pieces are looked up in the vocabulary.

Decoding joins the token strings and maps the alphabet back to bytes
(invalid UTF-8 becomes U+FFFD).  As in the reference there is no Unicode
normaliser step.  The split pattern uses the ``regex`` module's Unicode
classes (\\p{L}, \\p{N}).
"""
from __future__ import annotations

import json
from functools import lru_cache
from pathlib import Path

import regex

__all__ = ["Tokenizer", "SPLIT_PATTERN", "byte_alphabet", "CHAT_TEMPLATE", "chatml"]

SPLIT_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}"
                 r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
CHAT_TEMPLATE = "<|im_start|>user\n{text}<|im_end|>\n<|im_start|>assistant\n"


def chatml(text: str) -> str:
    """One user turn and the assistant prefix (run_chat.py:45)."""
    return CHAT_TEMPLATE.format(text=text)


@lru_cache(maxsize=1)
def byte_alphabet() -> dict:
    """GPT-2's byte -> printable character map: the printable Latin-1 bytes
    stand for themselves, the other 68 take code points 256, 257, ... in
    byte order."""
    keep = [b for b in range(256)
            if 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or 0xAE <= b <= 0xFF]
    table, extra = {}, 0
    for b in range(256):
        if b in keep:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + extra)
            extra += 1
    return table


class Tokenizer:
    def __init__(self, path: str | Path):
        tk = json.loads(Path(path).read_text(encoding="utf-8"))
        model = tk["model"]
        self.vocab: dict = dict(model["vocab"])
        self.id_to_token = {i: t for t, i in self.vocab.items()}
        self.ranks = {}
        for r, m in enumerate(model["merges"]):
            a, b = m.split(" ") if isinstance(m, str) else m
            self.ranks[(a, b)] = r
        self.special = {}
        for t in tk.get("added_tokens", []):
            self.special[t["content"]] = int(t["id"])
            self.id_to_token[int(t["id"])] = t["content"]
        self._special_ids = set(self.special.values())
        self.eos_id = self.special.get("<|im_end|>", 151645)
        self._enc = byte_alphabet()
        self._dec = {c: b for b, c in self._enc.items()}
        self._split = regex.compile(SPLIT_PATTERN)
        self._special_re = (regex.compile("|".join(regex.escape(s) for s in
                                                    sorted(self.special, key=len, reverse=True)))
                            if self.special else None)
        self._cache: dict = {}

    def _bpe(self, piece: str) -> list:
        hit = self._cache.get(piece)
        if hit is not None:
            return hit
        word = list(piece)
        while len(word) > 1:
            pairs = [(self.ranks.get((word[k], word[k + 1])), k) for k in range(len(word) - 1)]
            pairs = [p for p in pairs if p[0] is not None]
            if not pairs:
                break
            _, k = min(pairs)
            word[k:k + 2] = [word[k] + word[k + 1]]
        ids = [self.vocab[t] for t in word]
        if len(self._cache) < 65536:
            self._cache[piece] = ids
        return ids

    def _encode_plain(self, text: str, out: list) -> None:
        for piece in self._split.findall(text):
            out.extend(self._bpe("".join(self._enc[b] for b in piece.encode("utf-8"))))

    def encode(self, text: str) -> list:
        out: list = []
        pos = 0
        if self._special_re is not None:
            for m in self._special_re.finditer(text):
                self._encode_plain(text[pos:m.start()], out)
                out.append(self.special[m.group(0)])
                pos = m.end()
        self._encode_plain(text[pos:], out)
        return out

    def decode(self, ids) -> str:
        parts = []
        for i in ids:
            t = self.id_to_token[int(i)]
            if int(i) in self._special_ids:
                parts.append(t.encode("utf-8"))
            else:
                parts.append(bytes(self._dec[c] for c in t))
        return b"".join(parts).decode("utf-8", errors="replace")
