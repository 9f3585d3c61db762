"""Oracle (test infrastructure only): a restatement of Vortex-RT's Gemma 3 tokenizer.

Index (src/gemma3.cpp:289-454): pieces of token type 1 or 4 keyed by their string (a later
duplicate replaces an earlier one only with a strictly higher fp32 score), byte pieces
"<0xHH>" of type 6 (the last id of a byte wins), the longest piece length, add_space_prefix,
and the unknown / BOS / EOS ids (defaults 3 / 2 / 1).

Tokenize (:1920-2062): every run of ' ', '\\t', '\\r', '\\n' becomes one U+2581 marker (plus a
leading marker when add_space_prefix is set and the text does not start with one); a dynamic
programme over byte positions keeps, per end position, the first strictly best fp32 score
best[i] + score(piece) over the pieces starting at i (lengths ascending); at a position where
no piece starts, one byte is consumed by its byte piece (or the unknown id) at score -100.
Backtracking yields the ids, BOS first when requested.

decode_piece (:1251-1299): ids 0..3 print nothing, "<0xHH>" prints its byte, U+2581 prints
as a space.

Pinned in tests/test_tokenizer.py by brute force over every segmentation of short strings,
hand-worked cases (whitespace runs, prefix, byte fallback, unknown id) and the C++
implementation.
"""
from __future__ import annotations

import numpy as np

MARKER = "▁".encode("utf-8")


def _byte_piece(p: str):
    if len(p) == 6 and p[0] == "<" and p[1] == "0" and p[2] == "x" and p[5] == ">":
        try:
            return int(p[3:5], 16)
        except ValueError:
            return None
    return None


class Tokenizer:
    def __init__(self, pieces, scores, types, bos=2, eos=1, unk=3, add_space_prefix=False):
        n = len(pieces)
        if len(scores) != n or len(types) != n:
            raise ValueError("Gemma 3 tokenizer metadata is incomplete")
        self.pieces = list(pieces)
        self.index = {}
        self.byte_tokens = [None] * 256
        self.max_len = 0
        for i, (p, s, t) in enumerate(zip(pieces, scores, types)):
            if t == 6:
                b = _byte_piece(p)
                if b is not None:
                    self.byte_tokens[b] = i
                    continue
            if t not in (1, 4):
                continue
            key = p.encode("utf-8")
            s32 = np.float32(s)
            if key not in self.index or s32 > self.index[key][1]:
                self.index[key] = (i, s32)
            self.max_len = max(self.max_len, len(key))
        self.unk = min(unk, n - 1)
        if bos >= n:
            raise ValueError("Gemma 3 BOS token id is out of range")
        self.bos, self.eos = bos, eos
        self.add_space_prefix = add_space_prefix

    def normalize(self, text: str) -> bytes:
        out = bytearray()
        in_space = False
        for c in text.encode("utf-8"):
            if c in (0x20, 0x09, 0x0D, 0x0A):
                if not in_space:
                    out += MARKER
                in_space = True
            else:
                out.append(c)
                in_space = False
        if self.add_space_prefix and out and not out.startswith(MARKER):
            out = bytearray(MARKER) + out
        return bytes(out)

    def tokenize(self, text: str, add_bos: bool = True):
        s = self.normalize(text)
        n = len(s)
        neg = np.float32(-np.inf)
        best = [neg] * (n + 1)
        frm = [None] * (n + 1)
        via = [None] * (n + 1)
        best[0] = np.float32(0.0)
        for i in range(n):
            if not np.isfinite(best[i]):
                continue
            any_piece = False
            for ln in range(1, min(self.max_len, n - i) + 1):
                hit = self.index.get(s[i:i + ln])
                if hit is None:
                    continue
                any_piece = True
                cand = np.float32(best[i] + hit[1])
                if cand > best[i + ln]:
                    best[i + ln], frm[i + ln], via[i + ln] = cand, i, hit[0]
            if not any_piece:
                tid = self.byte_tokens[s[i]]
                if tid is None:
                    tid = self.unk
                cand = np.float32(best[i] - np.float32(100.0))
                if cand > best[i + 1]:
                    best[i + 1], frm[i + 1], via[i + 1] = cand, i, tid
        if n and not np.isfinite(best[n]):
            raise ValueError("Gemma 3 tokenizer could not segment prompt")
        ids = []
        at = n
        while at:
            ids.append(via[at])
            at = frm[at]
        ids.reverse()
        return ([self.bos] if add_bos else []) + ids

    def decode_piece(self, tid: int) -> bytes:
        if tid <= 3:
            return b""
        p = self.pieces[tid] if tid < len(self.pieces) else ""
        b = _byte_piece(p)
        if b is not None:
            return bytes([b])
        return p.encode("utf-8").replace(MARKER, b" ")

    def best_score(self, text: str):
        """The fp32 score of the segmentation tokenize() returns (for the brute-force pin)."""
        s = self.normalize(text)
        ids = self.tokenize(text, add_bos=False)
        total = np.float32(0.0)
        at = 0
        for tid in ids:
            p = self.pieces[tid].encode("utf-8")
            if self.index.get(p, (None,))[0] == tid and s[at:at + len(p)] == p:
                total = np.float32(total + self.index[p][1])
                at += len(p)
            else:
                total = np.float32(total - np.float32(100.0))
                at += 1
        return total
