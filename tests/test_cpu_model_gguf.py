"""CPU tests: the whole-model oracle (src/gemma3.cpp restated), the GGUF reader/writer, and the
C-ABI library's exported surface. None of these needs a GPU."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import gguf
import oracle
import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_PROBE = os.path.join(REPO, "oracle", "_ref", "ref_gguf_probe")


@pytest.fixture(scope="module")
def zero_proj_model(tmp_path_factory):
    """Every block projection is zero, the embedding is not: each block then leaves the
    residual stream unchanged (zero q/k/v -> uniform softmax over zero values -> zero
    attention; zero gate/up -> gelu(0) * 0 = 0), so the model reduces to
    logits = W_embd . (RMSNorm(embedding(t) * sqrt(d)) * w_out)."""
    p = str(tmp_path_factory.mktemp("m") / "zero.gguf")
    synth.write_gemma3_gguf(p, seed=5, weight_std=0.0, embd_std=0.02, **synth.TINY)
    return p


def test_zero_projection_closed_form(zero_proj_model):
    m = oracle.Model(zero_proj_model)
    f = gguf.GgufFile.open(zero_proj_model)
    d = m.info.embedding_length
    emb = f.tensor_bytes("token_embd.weight")
    w_out = f.read_f32("output_norm.weight").astype(np.float64)
    deq = synth.dequantize_q8_0(emb).reshape(m.info.vocab_size, d).astype(np.float64)
    for pos, tok in enumerate([7, 999, 2, 501]):
        r = m.decode(tok, pos, want_logits=True, logits=True)
        h = deq[tok] * np.sqrt(np.float32(d), dtype=np.float32)
        ref_hidden = h / np.sqrt(np.mean(h ** 2) + 1e-6) * w_out
        assert np.max(np.abs(r["hidden"] - ref_hidden)) <= 1e-6 * np.max(np.abs(ref_hidden))
        ref_logits = deq @ ref_hidden
        assert np.max(np.abs(r["logits"] - ref_logits)) <= 1e-5 * np.max(np.abs(ref_logits))
        top2 = np.sort(ref_logits)[-2:]
        if top2[1] - top2[0] > 1e-4 * abs(top2[1]):
            assert r["index"] == int(np.argmax(ref_logits))
    f.close()
    m.close()


def test_sliding_window_eviction(tmp_path):
    """One local block, window 4: a position's attention sees only the last 4 keys/values, and
    at block 0 those depend on their own tokens only, so changing token 0 must not change
    anything from position 4 on (src/gemma3.cpp:1590-1600), and must change position 3."""
    p = str(tmp_path / "w4.gguf")
    kw = dict(synth.TINY)
    kw.update(n_layers=1, window=4)
    synth.write_gemma3_gguf(p, seed=9, **kw)
    a = [17, 40, 41, 42, 43, 44, 45]
    b = [900] + a[1:]
    ma, mb = oracle.Model(p), oracle.Model(p)
    for pos in range(len(a)):
        ra = ma.decode(a[pos], pos, want_logits=False)
        rb = mb.decode(b[pos], pos, want_logits=False)
        same = np.array_equal(ra["hidden"], rb["hidden"])
        assert same == (pos >= 4), f"position {pos}"
    ma.close()
    mb.close()


def test_decode_state_errors(tmp_path):
    """src/gemma3.cpp:1467-1474 and :1878-1881: contiguous positions, context limit, token
    range, and the cache reset after a failure."""
    p = str(tmp_path / "tiny.gguf")
    kw = dict(synth.TINY)
    kw.update(context=6)
    synth.write_gemma3_gguf(p, seed=2, **kw)
    m = oracle.Model(p)
    m.decode(5, 0)
    with pytest.raises(RuntimeError, match="contiguous"):
        m.decode(5, 2)
    with pytest.raises(RuntimeError, match="vocabulary"):
        m.decode(1000, 1)
    m.decode(5, 0)                       # the failure reset the cache: position 0 again
    for pos in range(1, 6):
        m.decode(5, pos, want_logits=False)
    with pytest.raises(RuntimeError, match="context length"):
        m.decode(5, 6)
    m.close()


def test_generate_stops_after_eos(tmp_path):
    """generate_greedy_tokens appends EOS then stops (src/gemma3.cpp:2134-2141); a prompt of n
    tokens plus N new tokens takes n + N - 1 steps."""
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=11, **synth.TINY)
    m = oracle.Model(p)
    prompt = synth.uniform_ids(5, 5, 2, 1000)
    toks = m.generate(prompt, 12)
    assert toks.size == 12 or toks[-1] == m.info.eos_id
    # the same tokens step by step through decode
    m.reset()
    for i, t in enumerate(prompt):
        r = m.decode(int(t), i, want_logits=(i == prompt.size - 1))
    seq = [r["index"]]
    for j in range(1, toks.size):
        r = m.decode(seq[-1], prompt.size + j - 1)
        seq.append(r["index"])
    assert np.array_equal(np.array(seq, np.uint32), toks)
    m.close()


# ---- GGUF ---------------------------------------------------------------------------------

def test_gguf_roundtrip(tmp_path):
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=1, **synth.TINY)
    f = gguf.GgufFile.open(p)
    assert f.version == 3 and f.alignment == 32 and f.data_offset % 32 == 0
    assert f.meta_str("general.architecture") == "gemma3"
    assert f.meta_u64("gemma3.block_count") == 6
    assert f.meta_array_len("tokenizer.ggml.tokens") == 1000
    t = f.tensors["blk.3.ffn_down.weight"]
    assert t.dims == [256, 128] and t.type == gguf.GGML_Q8_0 and t.offset % 32 == 0
    assert np.array_equal(f.tensor_bytes("blk.3.ffn_down.weight"), synth.q8_matrix(1, "blk.3.ffn_down.weight", 128, 256))
    f.validate()
    f.close()


def test_gguf_rejects_corruption(tmp_path):
    """src/gguf.cpp:321-403 and :640-664: bad magic, bad version, truncation."""
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=1, **synth.TINY)
    raw = open(p, "rb").read()
    for name, data, pat in (("magic", b"XXXX" + raw[4:], "magic"),
                            ("version", raw[:4] + (9).to_bytes(4, "little") + raw[8:], "version"),
                            ("trunc", raw[:200], "")):
        q = str(tmp_path / f"{name}.gguf")
        open(q, "wb").write(data)
        with pytest.raises(gguf.GgufError, match=pat or None):
            gguf.GgufFile.open(q).validate()
        err_o = None
        try:
            oracle.Model(q)
        except RuntimeError as e:
            err_o = str(e)
        assert err_o is not None


@pytest.mark.skipif(not os.path.exists(REF_PROBE), reason="reference GGUF parser probe not built (oracle/Makefile ref)")
def test_gguf_against_reference_parser(tmp_path):
    """The reference's own GgufFile (src/gguf.cpp, compiled by oracle/Makefile) reads our file:
    same header, tensor directory and Q8_0 row dequant bits (src/gguf.cpp:546-638)."""
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=4, **synth.TINY)
    out = subprocess.run([REF_PROBE, p, "token_embd.weight", "0", "token_embd.weight", "777",
                          "blk.5.attn_q.weight", "127"], capture_output=True, text=True, check=True).stdout
    f = gguf.GgufFile.open(p)
    lines = out.splitlines()
    head = lines[0].split()
    assert head[0] == "header" and int(head[1]) == 3 and int(head[2]) == f.data_offset and int(head[3]) == 32
    assert int(head[5]) == len(f.tensors)
    tens = {l.split()[1]: l.split() for l in lines if l.startswith("tensor ")}
    for name, t in f.tensors.items():
        row = tens[name]
        assert int(row[2]) == t.type and int(row[3]) == t.offset and int(row[4]) == t.nbytes()
        assert [int(x) for x in row[5:]] == t.dims
    for l in lines:
        if l.startswith("row "):
            _, name, r, *bits = l.split()
            t = f.tensors[name]
            k = t.dims[0]
            blk = f.tensor_bytes(name)[int(r) * (k // 32) * 34:(int(r) + 1) * (k // 32) * 34]
            ref = np.array([int(b, 16) for b in bits], dtype=np.uint32)
            assert np.array_equal(oracle.dequant(blk).view(np.uint32), ref)
    f.close()


def _header_only(path, n_tensors=0, array_count=None):
    """A GGUF v3 header that ends early: n_tensors tensors announced, and when array_count is
    given one metadata key "a" announcing a u32 array of that many elements."""
    import struct
    b = struct.pack("<IIQQ", 0x46554747, 3, n_tensors, 1 if array_count is not None else 0)
    if array_count is not None:
        b += struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", 9, 4, array_count)
    open(path, "wb").write(b)
    return path


def _limit_errors(tmp_path, run):
    """run(path) -> error text, for headers just inside and just past the reference's limits:
    arrays of 2^28 elements (src/gguf.cpp:16, :105-107), 1,000,000 tensors (:334-336)."""
    out = {}
    for name, kw in (("array_ok", dict(array_count=1 << 28)), ("array_over", dict(array_count=(1 << 28) + 1)),
                     ("count_ok", dict(n_tensors=1000000)), ("count_over", dict(n_tensors=1000001))):
        out[name] = run(_header_only(str(tmp_path / f"{name}.gguf"), **kw))
    return out


def test_cpp_gguf_limits_match_reference(tmp_path):
    """The C++ reader applies the reference's array-length and header-count limits: a header one
    past either limit is rejected with the reference's message, one at the limit gets past the
    check (and then fails at the end of the file)."""
    def run(p):
        r = subprocess.run([_cpp("gguf_test"), p], capture_output=True, text=True)
        assert r.returncode == 1, r.stdout
        return r.stdout
    e = _limit_errors(tmp_path, run)
    assert "GGUF array length exceeds safety limit" in e["array_over"]
    assert "safety limit" not in e["array_ok"] and "end of GGUF file" in e["array_ok"]
    assert "GGUF header counts exceed safety limits" in e["count_over"]
    assert "safety limit" not in e["count_ok"] and "end of GGUF file" in e["count_ok"]


@pytest.mark.skipif(not os.path.exists(REF_PROBE), reason="reference GGUF parser probe not built (oracle/Makefile ref)")
def test_gguf_limits_reference_parser(tmp_path):
    """The reference's own parser rejects the two over-limit headers with the same messages (the
    at-limit array is not run through it: it reserves the announced count, 2^28 values)."""
    for name, kw, msg in (("array_over", dict(array_count=(1 << 28) + 1), "GGUF array length exceeds safety limit"),
                          ("count_over", dict(n_tensors=1000001), "GGUF header counts exceed safety limits")):
        p = _header_only(str(tmp_path / f"{name}.gguf"), **kw)
        r = subprocess.run([REF_PROBE, p], capture_output=True, text=True)
        assert r.returncode == 1 and msg in r.stdout, (name, r.stdout)


# ---- C ABI ---------------------------------------------------------------------------------

def _declared_symbols():
    txt = open(os.path.join(REPO, "include", "vrt_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(vrt_[a-z0-9_]+)\s*\(", txt)))


def test_abi_library_exports_declared_symbols():
    """libvrt_hip.so loads without a GPU and exports every function include/vrt_hip.h declares
    (no compute call is made here)."""
    import vrt
    if not os.path.exists(vrt.LIB_PATH):
        pytest.skip("libvrt_hip.so not built")
    lib = ctypes.CDLL(vrt.LIB_PATH)
    syms = _declared_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert set(syms) == set(vrt.SIGNATURES), "ctypes binding and header disagree"
    nm = subprocess.run(["nm", "-D", "--defined-only", vrt.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in nm.splitlines() if " T " in l}
    assert exported == set(syms), f"unexpected exports: {sorted(exported - set(syms))}"


# ---- C++ surface (vortexrt::GgufFile) -------------------------------------------------------

CPP_BIN = os.path.join(REPO, "tests", "cpp", "_build")


def _cpp(name):
    exe = os.path.join(CPP_BIN, name)
    if not os.path.exists(exe):
        pytest.skip(f"{name} not built (vortex-rt_amd/build.py)")
    return exe


def test_cpp_gguf_reader_matches(tmp_path):
    """The C++ GgufFile reads our writer's file like gguf.py does, and its Q8_0 row dequant
    equals the oracle's bit for bit."""
    import json
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=4, **synth.TINY)
    out = subprocess.run([_cpp("gguf_test"), p, "token_embd.weight", "999", "blk.2.ffn_down.weight", "5"],
                         capture_output=True, text=True, check=True).stdout
    got = json.loads(out)
    f = gguf.GgufFile.open(p)
    assert got["version"] == f.version and got["data_offset"] == f.data_offset and got["alignment"] == f.alignment
    assert got["arch"] == "gemma3" and len(got["tensors"]) == len(f.tensors)
    for name, t in f.tensors.items():
        typ, off, nbytes, *dims = got["tensors"][name]
        assert (typ, off, nbytes, dims) == (t.type, t.offset, t.nbytes(), t.dims)
    for (name, r), row in zip((("token_embd.weight", 999), ("blk.2.ffn_down.weight", 5)), got["rows"]):
        t = f.tensors[name]
        nb = t.dims[0] // 32
        blk = f.tensor_bytes(name)[r * nb * 34:(r + 1) * nb * 34]
        assert np.array_equal(np.array(row, dtype=np.float32), oracle.dequant(blk))
    f.close()


def test_cpp_gguf_reader_rejects_corruption(tmp_path):
    p = str(tmp_path / "tiny.gguf")
    synth.write_gemma3_gguf(p, seed=1, **synth.TINY)
    raw = open(p, "rb").read()
    for name, data, pat in (("magic", b"XXXX" + raw[4:], "Invalid GGUF magic"),
                            ("version", raw[:4] + (9).to_bytes(4, "little") + raw[8:], "Unsupported GGUF version"),
                            ("trunc", raw[:200], "end of GGUF file")):
        q = str(tmp_path / f"{name}.gguf")
        open(q, "wb").write(data)
        r = subprocess.run([_cpp("gguf_test"), q], capture_output=True, text=True)
        assert r.returncode == 1 and pat in r.stdout, (name, r.stdout)
