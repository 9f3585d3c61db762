"""The Gemma 3 tokenizer (src/gemma3.cpp:289-454, :1237-1299, :1920-2062): the oracle's
restatement pinned by brute force and hand-worked cases, then the C++ Gemma3Tokenizer
(libvortexrt.so, host only) against the oracle. No GPU."""
import itertools
import json
import os
import subprocess

import numpy as np
import pytest

import synth
from tokenizer import MARKER, Tokenizer

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "_build", "tokenizer_test")
M = "▁"
CONTROL = (["<pad>", "<eos>", "<bos>", "<unk>"], [0.0] * 4, [3, 3, 3, 2])


def _vocab(pieces, scores, types=None, with_bytes=True):
    p, s, t = (list(x) for x in CONTROL)
    if with_bytes:
        p += [f"<0x{b:02X}>" for b in range(256)]
        s += [0.0] * 256
        t += [6] * 256
    p += pieces
    s += scores
    t += types if types is not None else [1] * len(pieces)
    return p, s, t


def _brute(tok, text):
    """Best fp32 score over every segmentation of the normalised text: any vocabulary piece may
    start a step; a byte step (-100) only where no piece starts."""
    s = tok.normalize(text)
    best = None

    def walk(i, total):
        nonlocal best
        if i == len(s):
            best = total if best is None or total > best else best
            return
        starts = [ln for ln in range(1, len(s) - i + 1) if s[i:i + ln] in tok.index]
        if not starts:
            walk(i + 1, np.float32(total - np.float32(100.0)))
        for ln in starts:
            walk(i + ln, np.float32(total + tok.index[s[i:i + ln]][1]))

    walk(0, np.float32(0.0))
    return best


def test_oracle_matches_brute_force():
    rng = np.random.default_rng(7)
    alphabet = ["a", "b", "c", M]
    for trial in range(30):
        pieces = sorted({"".join(rng.choice(alphabet, size=rng.integers(1, 4))) for _ in range(12)})
        scores = list(rng.uniform(-8.0, -0.5, size=len(pieces)))
        tok = Tokenizer(*_vocab(pieces, scores))
        for _ in range(12):
            text = "".join(rng.choice(["a", "b", "c", " ", "d"], size=rng.integers(0, 9)))
            got = tok.best_score(text)
            want = _brute(tok, text)
            if want is None:   # empty text
                assert tok.tokenize(text, False) == []
                continue
            assert got == want, (trial, text, pieces)


def test_oracle_hand_cases():
    pieces = [M + "Hello", M + "H", "ello", "ell", "o", M, "H", M + "world", "wor", "ld"]
    scores = [-1.0, -3.0, -2.5, -2.0, -1.5, -4.0, -5.0, -1.2, -3.0, -2.0]
    p, s, t = _vocab(pieces, scores)
    base = 4 + 256
    ids = {x: base + i for i, x in enumerate(pieces)}
    tok = Tokenizer(p, s, t, add_space_prefix=True)
    # the leading marker makes "▁Hello" one piece; the space run becomes one marker
    assert tok.tokenize("Hello  \t world") == [2, ids[M + "Hello"], ids[M + "world"]]
    assert tok.tokenize("Hello", add_bos=False) == [ids[M + "Hello"]]
    # without the prefix "Hello" splits as H + ello (-7.5) rather than H + ell + o (-8.5)
    tok2 = Tokenizer(p, s, t, add_space_prefix=False)
    assert tok2.tokenize("Hello", add_bos=False) == [ids["H"], ids["ello"]]
    # byte fallback: "é" (C3 A9) has no piece -> its two byte pieces; "Z" too
    assert tok2.tokenize("éZ", add_bos=False) == [4 + 0xC3, 4 + 0xA9, 4 + ord("Z")]
    # no byte pieces at all -> the unknown id (3) per byte
    tok3 = Tokenizer(*_vocab(pieces, scores, with_bytes=False))
    assert tok3.tokenize("Zo", add_bos=False) == [3, 4 + pieces.index("o")]
    # an empty prompt is BOS alone
    assert tok.tokenize("") == [2]
    # decode: control ids print nothing, byte pieces their byte, the marker a space
    assert tok.decode_piece(2) == b"" and tok.decode_piece(4 + 0x41) == b"A"
    assert tok.decode_piece(ids[M + "world"]) == b" world"


def test_oracle_duplicate_and_type_rules():
    # a duplicate piece keeps the strictly higher score; ties keep the first id; types other
    # than 1 and 4 are not pieces
    pieces = ["ab", "ab", "ab", "x", "y"]
    scores = [-2.0, -1.0, -1.0, -1.0, -1.0]
    types = [1, 1, 4, 2, 5]
    p, s, t = _vocab(pieces, scores, types)
    tok = Tokenizer(p, s, t)
    base = 4 + 256
    assert tok.index["ab".encode()][0] == base + 1
    assert "x".encode() not in tok.index and "y".encode() not in tok.index
    assert tok.tokenize("xab", add_bos=False) == [4 + ord("x"), base + 1]


def _hex(text):
    return text.encode("utf-8").hex()


def _run_cpp(path, vocab, texts):
    assert os.path.exists(BIN), f"{BIN} not built (vortex-rt_amd/build.py)"
    r = subprocess.run([BIN, path, str(vocab)] + [_hex(t) for t in texts], capture_output=True, text=True, timeout=120)
    return r.returncode, json.loads(r.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("prefix", [None, True, False])
def test_cpp_tokenizer_matches_oracle(tmp_path, prefix):
    rng = np.random.default_rng(11 if prefix is None else (12 if prefix else 13))
    alphabet = ["a", "b", "c", "é", M, "ab", "ca"]
    pieces = sorted({"".join(rng.choice(alphabet, size=rng.integers(1, 4))) for _ in range(40)})
    scores = list(np.round(rng.uniform(-10.0, -0.25, size=len(pieces)), 3))
    types = list(rng.choice([1, 1, 1, 4, 2], size=len(pieces)))
    p, s, t = _vocab(pieces, scores, types)
    path = str(tmp_path / "tok.gguf")
    synth.write_tokenizer_gguf(path, p, s, t, add_space_prefix=prefix)
    texts = ["", "abc", "  a b\tc\n", "éab cab", "zzz", "ca ca  ab é", "a" * 40] + \
            ["".join(rng.choice(["a", "b", "c", " ", "é", "q"], size=rng.integers(1, 30))) for _ in range(40)]
    rc, got = _run_cpp(path, len(p), texts)
    assert rc == 0, got
    tok = Tokenizer(p, s, t, add_space_prefix=bool(prefix))
    assert (got["bos"], got["eos"], got["unk"], got["prefix"]) == (2, 1, 3, int(bool(prefix)))
    assert got["pieces"] == len(tok.index)
    for text, ids, ids_nobos in zip(texts, got["ids"], got["ids_nobos"]):
        assert ids == tok.tokenize(text, True), text
        assert ids_nobos == tok.tokenize(text, False), text
    for i, h in enumerate(got["decoded"]):
        assert bytes.fromhex(h) == tok.decode_piece(i), i


def test_cpp_tokenizer_rejects_incomplete_metadata(tmp_path):
    p, s, t = _vocab(["a", "b"], [-1.0, -2.0])
    path = str(tmp_path / "short.gguf")
    synth.write_tokenizer_gguf(path, p, s[:-1], t)
    rc, got = _run_cpp(path, len(p), ["a"])
    assert rc == 1 and "incomplete" in got["error"]
    path2 = str(tmp_path / "badbos.gguf")
    synth.write_tokenizer_gguf(path2, p, s, t, bos=len(p))
    rc, got = _run_cpp(path2, len(p), ["a"])
    assert rc == 1 and "BOS" in got["error"]


def test_model_vocab_tokenizes(tmp_path):
    """The synthetic models' vocabulary (control ids, 256 byte pieces, '▁t<i>' pieces)."""
    vocab = 1000
    pieces = ["<pad>", "<eos>", "<bos>", "<unk>"] + [f"<0x{b:02X}>" for b in range(256)]
    pieces += [f"{M}t{i}" for i in range(len(pieces), vocab)]
    types = [3, 3, 3, 2] + [6] * 256 + [1] * (vocab - 260)
    scores = list(np.linspace(0, -1, vocab, dtype=np.float32))
    path = str(tmp_path / "model_vocab.gguf")
    synth.write_tokenizer_gguf(path, pieces, scores, types)
    texts = ["Hello world", " t300 t417  t999", "t300", " t5"]
    rc, got = _run_cpp(path, vocab, texts)
    assert rc == 0
    tok = Tokenizer(pieces, scores, types)
    assert got["ids"] == [tok.tokenize(x) for x in texts]
    # whole pieces where the vocabulary has them; " t5" has none ("\u2581t<i>" exists for i >= 260)
    assert tok.tokenize(" t300 t417  t999") == [2, 300, 417, 999]
    assert tok.tokenize(" t5") == [2, 4 + 0xE2, 4 + 0x96, 4 + 0x81, 4 + ord("t"), 4 + ord("5")]
