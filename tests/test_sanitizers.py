"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU): the CPU oracle
(oracle/vrt_oracle.c, driven by tests/cpp/oracle_sanitize.c), the C++ GGUF reader and the
Gemma 3 tokenizer (vortex-rt_amd/csrc/host/{gguf,tokenizer}.cpp, driven by the same test
programs as their parity tests). Each is built here with g++/gcc (host code only) and run on a
tiny synthetic model, a tokenizer vocabulary and corrupted files; any sanitizer report aborts
the program and fails the test."""
import os
import shutil
import subprocess

import pytest

import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(REPO, "tests", "cpp")
HOST = os.path.join(REPO, "vortex-rt_amd", "csrc", "host")
OUT = os.path.join(CPP, "_build", "san")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")


def _build(name, cmd):
    os.makedirs(OUT, exist_ok=True)
    exe = os.path.join(OUT, name)
    r = subprocess.run(cmd + ["-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


@pytest.fixture(scope="module")
def bins():
    if shutil.which("g++") is None or shutil.which("gcc") is None:
        pytest.skip("no host compiler")
    if os.environ.get("LD_PRELOAD"):
        pytest.skip("a preloaded library would precede the sanitizer runtime")
    inc = ["-I" + os.path.join(REPO, "include")]
    return {
        "oracle": _build("oracle_sanitize", ["gcc", "-std=gnu11", "-ffp-contract=off"] + SAN +
                         ["-I" + os.path.join(REPO, "oracle"), os.path.join(CPP, "oracle_sanitize.c"),
                          os.path.join(REPO, "oracle", "vrt_oracle.c"), "-lm"]),
        "gguf": _build("gguf_test", ["g++", "-std=c++20"] + SAN + inc +
                       [os.path.join(CPP, "gguf_test.cpp"), os.path.join(HOST, "gguf.cpp")]),
        "tok": _build("tokenizer_test", ["g++", "-std=c++20"] + SAN + inc +
                      [os.path.join(CPP, "tokenizer_test.cpp"), os.path.join(HOST, "tokenizer.cpp"),
                       os.path.join(HOST, "gguf.cpp")]),
    }


def _run(args):
    r = subprocess.run(args, capture_output=True, text=True, env=ENV, timeout=300)
    report = "AddressSanitizer" in r.stderr or "runtime error:" in r.stderr or "LeakSanitizer" in r.stderr
    return r, report


def test_oracle_under_sanitizers(bins, tmp_path):
    good = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(good, seed=3, **synth.TINY)
    bad = str(tmp_path / "trunc.gguf")
    open(bad, "wb").write(open(good, "rb").read()[:300])
    r, report = _run([bins["oracle"], good, bad])
    assert not report, r.stderr[-3000:]
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.stdout, r.stderr[-2000:])


def test_gguf_reader_under_sanitizers(bins, tmp_path):
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=4, **synth.TINY)
    r, report = _run([bins["gguf"], p, "token_embd.weight", "7", "blk.1.ffn_down.weight", "3"])
    assert not report and r.returncode == 0, r.stderr[-3000:]
    raw = open(p, "rb").read()
    for name, data in (("magic", b"XXXX" + raw[4:]), ("version", raw[:4] + (9).to_bytes(4, "little") + raw[8:]),
                       ("trunc", raw[:200]), ("header", raw[:24]), ("empty", b"")):
        q = str(tmp_path / f"{name}.gguf")
        open(q, "wb").write(data)
        r, report = _run([bins["gguf"], q])
        assert not report, (name, r.stderr[-3000:])
        assert r.returncode == 1, (name, r.stdout, r.stderr[-1000:])


def test_tokenizer_under_sanitizers(bins, tmp_path):
    pieces = ["a", "b", "ab", "ca", "é", "▁a", "▁", "abc", "▁▁"]
    p = ["<pad>", "<eos>", "<bos>", "<unk>"] + [f"<0x{b:02X}>" for b in range(256)] + pieces
    s = [0.0] * (4 + 256) + [-1.0, -1.5, -0.5, -2.0, -1.0, -0.75, -3.0, -0.25, -4.0]
    t = [3, 3, 3, 2] + [6] * 256 + [1] * len(pieces)
    path = str(tmp_path / "tok.gguf")
    synth.write_tokenizer_gguf(path, p, s, t, add_space_prefix=True)
    texts = ["", "abc", "  a b\tc\n", "éab cab", "zzz \x00 q", "ca ca  ab é", "a" * 300, "▁▁x"]
    r, report = _run([bins["tok"], path, str(len(p))] + [x.encode("utf-8").hex() for x in texts])
    assert not report and r.returncode == 0, r.stderr[-3000:]
    # a vocabulary size that does not match the metadata is rejected cleanly
    r, report = _run([bins["tok"], path, str(len(p) + 5), "61"])
    assert not report, r.stderr[-3000:]
