"""CPU pins of the oracle (oracle/vrt_oracle.c) against checks independent of its own code.

The reference ships no expected outputs for this path (its tests compute their references at
run time and assert tolerances), so each oracle function is pinned by something that does not
restate its formula: IEEE conversions in numpy, exact float64 arithmetic, closed forms and
invariants, and the reference tests' own fixtures and tolerances
(src/q8_test_main.cpp:80-317, src/ffn_test_main.cpp:254-441, src/gelu_test_main.cpp:34-138).
"""
import numpy as np
import pytest

import oracle
import synth

RNG = np.random.default_rng(20261201)


# ---- fp16 codec --------------------------------------------------------------------------

def test_f16_decode_exhaustive_vs_ieee():
    """src/gguf.cpp:203-235 is an exact IEEE half -> float: all 65536 codes against numpy."""
    h = np.arange(65536, dtype=np.uint16)
    blocks = np.zeros((65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    blocks[:, 2] = 1                                   # q = 1 -> value == scale
    got = oracle.dequant(blocks.reshape(-1)).reshape(65536, 32)[:, 0]
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))


def _ieee_half_model(x: np.ndarray) -> np.ndarray:
    """The quantiser's encode described relative to IEEE round-to-nearest-even (numpy):
    identical except that (a) an exact tie rounds the magnitude up instead of to even, and
    (b) when rounding carries out of the mantissa into an odd biased exponent the carry is
    lost, leaving 2^(e-15) (half the correctly rounded value)."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    mant = bits & 0x7FFFFF
    e = ((bits >> 23) & 0xFF) - 127 + 15
    rne = np.abs(x).astype(np.float16).view(np.uint16).astype(np.int64)
    out = rne.copy()
    normal = (e >= 1) & (e <= 30)
    tie = normal & ((mant & 0x1FFF) == 0x1000)
    # half-up on a tie: the next code above the truncated one
    trunc = (e << 10) | (mant >> 13)
    out = np.where(tie, trunc + 1, out)
    carry = normal & (mant + 0x1000 >= 0x800000)
    out = np.where(carry & (e % 2 == 1), e << 10, out)
    out = np.where(carry & (e % 2 == 0), (e + 1) << 10, out)
    return (out | sign).astype(np.uint16)


def test_f16_encode_against_ieee_model():
    """src/q8_test_main.cpp:18-41 on normal-range scales (every block scale amax/127 of the
    workloads lies there): random values plus constructed ties and carries."""
    v = (RNG.standard_normal(200000) * 10.0 ** RNG.uniform(-4, 4, 200000)).astype(np.float32)
    v = v[(np.abs(v) >= 2.0 ** -14) & (np.abs(v) < 65504.0)]
    # constructed ties: mantissa low 13 bits == 0x1000, both parities of the kept lsb
    e = RNG.integers(100, 140, 4000)
    m = (RNG.integers(0, 1 << 10, 4000) << 13) | 0x1000
    ties = ((e << 23) | m).astype(np.uint32).view(np.float32)
    # constructed carries: mantissa >= 0x7ff000, odd and even biased fp16 exponents
    e2 = np.arange(113, 142)
    m2 = 0x7FF000 + RNG.integers(0, 0x1000, e2.size)
    carries = ((e2 << 23) | m2).astype(np.uint32).view(np.float32)
    x = np.concatenate([v, ties, -ties[:100], carries, -carries])
    got = np.array([oracle.f32_to_f16(float(t)) for t in x], dtype=np.uint16)
    assert np.array_equal(got, _ieee_half_model(x))
    # the carry-loss really halves: 0x40FFFFFF (7.9999995, fp16 biased exponent 17, odd)
    # rounds to 8.0 in IEEE but keeps exponent 17 here, i.e. 4.0
    odd = float(np.uint32(0x40FFFFFF).view(np.float32))
    assert oracle.f16_to_f32(oracle.f32_to_f16(odd)) == 4.0


def test_f16_rne_against_numpy():
    """or_f32_to_f16_rne (the fp16 KV rounding) against numpy's float32 -> float16 cast, an
    independent IEEE round-to-nearest-even implementation: every half value, every midpoint
    between neighbouring halves (ties) and its float32 neighbours, the subnormal and overflow
    boundaries, signed zeros, infinities, and 4M random bit patterns."""
    halves = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    mids = (halves[:-1].astype(np.float64) + halves[1:].astype(np.float64)) / 2.0
    mids = mids.astype(np.float32)   # exact: two neighbouring halves differ in 11 significant bits
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))])
    edges = np.array([0.0, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25, 2.0 ** -14, 65504.0, 65519.996, 65520.0,
                      65536.0, 1e30, np.inf, 2.0 ** -26, 3e-8], dtype=np.float32)
    rng = np.random.default_rng(11)
    rand = rng.integers(0, 2 ** 32, size=1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([halves, mids, near, edges, rand])
    x = np.concatenate([x, -x])
    got = oracle.f32_to_f16_rne(x)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)


def _bf16_nearest(x: np.ndarray) -> np.ndarray:
    """bfloat16 bits of finite float32 values by the definition of round to nearest even: of
    the two bf16 values around x (its top 16 bits, and one ulp further from zero, with 2^128 in
    place of the value past the largest finite one), the nearer in exact float64 arithmetic, the
    one with an even last bit on a tie."""
    bits = x.view(np.uint32)
    lo = (bits >> 16).astype(np.uint32)
    hi = lo + 1
    mag = np.abs(x.astype(np.float64))
    v_lo = np.abs((lo << 16).view(np.float32).astype(np.float64))
    hi_bits = (hi << 16).astype(np.uint32)
    v_hi = np.where((hi & 0x7fff) == 0x7f80, 2.0 ** 128, np.abs(hi_bits.view(np.float32).astype(np.float64)))
    d_lo, d_hi = mag - v_lo, v_hi - mag
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((lo & 1) == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def test_bf16_rne_against_definition():
    """or_f32_to_bf16_rne (the bf16 KV rounding) against the definition of round to nearest
    even, computed independently in float64 (_bf16_nearest): every midpoint between neighbouring
    bf16 values of a sweep of exponents (ties, to the even neighbour) and its float32 neighbours,
    the carry into the exponent, the largest finite values (rounding to infinity), subnormals,
    signed zeros, infinities and 4M random bit patterns; NaN stays a quiet NaN. or_bf16_to_f32
    is the exact 16-bit shift for every bf16 bit pattern."""
    rng = np.random.default_rng(12)
    top = rng.integers(0, 0x7f80, size=1 << 16, dtype=np.uint32)
    mids = ((top << 16) | 0x8000).astype(np.uint32).view(np.float32)          # exact ties
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))])
    edges = np.array([0x00000000, 0x00008000, 0x00018000, 0x00007fff, 0x3f7fffff, 0x3f7f8000, 0x3f7f7fff,
                      0x7f7f7fff, 0x7f7f8000, 0x7f7fffff, 0x7f800000, 0x00800000, 0x007fffff],
                     dtype=np.uint32).view(np.float32)
    rand = rng.integers(0, 2 ** 32, size=1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([mids, near, edges, rand])
    x = np.concatenate([x, -x])
    got = oracle.f32_to_bf16_rne(x)
    nan = np.isnan(x)
    fin = np.isfinite(x)
    assert np.array_equal(got[fin], _bf16_nearest(x[fin]))
    inf = ~fin & ~nan
    assert np.array_equal(got[inf], (x[inf].view(np.uint32) >> 16).astype(np.uint16))
    assert np.all((got[nan] & 0x7f80) == 0x7f80) and np.all((got[nan] & 0x40) != 0)
    # a tie rounds to the even neighbour: 1 + 2^-8 (between 1 and 1 + 2^-7) -> 1; the odd one up
    assert oracle.f32_to_bf16_rne(np.array([1 + 2.0 ** -8], np.float32))[0] == 0x3f80
    assert oracle.f32_to_bf16_rne(np.array([1 + 3 * 2.0 ** -8], np.float32))[0] == 0x3f82
    for h in range(1 << 16):
        f = np.float32(oracle.bf16_to_f32(h))
        if np.isnan(f):
            assert (h & 0x7f80) == 0x7f80 and (h & 0x7f) != 0
        else:
            assert int(f.view(np.uint32)) == h << 16, h


def test_f16_encode_golden():
    """Hand-derived codes (ties, carries, subnormals, overflow) kept in tests/golden."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "f16_encode_cases.json")) as fp:
        cases = json.load(fp)["cases"]
    for c in cases:
        x = np.uint32(int(c["f32_bits"], 16)).view(np.float32)
        assert oracle.f32_to_f16(float(x)) == int(c["f16_bits"], 16), c["why"]


# ---- Q8_0 quantiser ----------------------------------------------------------------------

def test_quantiser_properties():
    """q = nearbyint(v / (amax/127)) in fp32 (src/q8_test_main.cpp:106-124): the amax element
    maps to +-127, |q| <= 127, and every q equals numpy's IEEE fp32 division + rint."""
    w = synth.normal_f32(7, 32 * 5000, 0.02)
    blk = oracle.quantize(w).reshape(-1, 34)
    v = w.reshape(-1, 32)
    q = blk[:, 2:].view(np.int8).astype(np.int32)
    amax = np.max(np.abs(v), axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    ref_q = np.rint((v / scale[:, None]).astype(np.float32)).astype(np.int32)
    assert np.array_equal(q, np.clip(ref_q, -127, 127))
    imax = np.argmax(np.abs(v), axis=1)
    assert np.all(np.abs(q[np.arange(q.shape[0]), imax]) == 127)
    half = blk[:, 0:2].copy().view(np.uint16).reshape(-1)
    assert np.array_equal(half, _ieee_half_model(scale))


def test_quantiser_variant_b_and_zero_block():
    """src/ffn_test_main.cpp:169-196 divides by the decoded fp16 scale and maps amax == 0 to
    scale 1; variant A's 0/0 on an all-zero block gives q = -127 (x86 cvttss2si of NaN, then
    the clamp), which still dequantises to zero."""
    v = np.zeros(64, dtype=np.float32)
    v[32:] = np.linspace(-1, 1, 32, dtype=np.float32)
    a = oracle.quantize(v, "a").reshape(-1, 34)
    b = oracle.quantize(v, "b").reshape(-1, 34)
    assert a[0, 0] == 0 and a[0, 1] == 0 and np.all(a[0, 2:].view(np.int8) == -127)
    assert np.all(oracle.dequant(a[0]) == 0)
    assert b[0, 0:2].copy().view(np.uint16)[0] == 0x3C00 and np.all(b[0, 2:] == 0)
    s16 = np.float32(b[1, 0:2].copy().view(np.float16)[0])
    ref = np.clip(np.rint((v[32:] / s16).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(b[1, 2:].view(np.int8), ref)


def test_quantiser_numpy_writer_matches_oracle():
    """synth's numpy quantiser (used to write the model files) equals the C oracle byte for byte."""
    parts = [synth.normal_f32(2, 32 * 3000, 0.02),
             (RNG.standard_normal(32 * 2000) * 10.0 ** RNG.integers(-8, 6, 32 * 2000)).astype(np.float32)]
    edge = np.zeros(32 * 6, dtype=np.float32)
    edge[32:64] = 1e-41
    edge[64:96] = 65504.0 * 127
    edge[96:128] = np.nan
    edge[128] = np.inf
    edge[160:192] = (1.0 + 2.0 ** -11) * 127
    parts.append(edge)
    x = np.concatenate(parts).astype(np.float32)
    for var in ("a", "b"):
        assert np.array_equal(synth.quantize_q8_0(x, var), oracle.quantize(x, var))


def test_dequant_exhaustive():
    """src/gguf.cpp:620-635 over every fp16 scale x every int8 value, against numpy."""
    h = np.arange(65536, dtype=np.uint32)
    blocks = np.zeros((65536 * 8, 34), dtype=np.uint8)
    q = np.arange(256, dtype=np.uint8).reshape(8, 32)
    blocks[:, 0] = np.repeat(h & 0xFF, 8)
    blocks[:, 1] = np.repeat(h >> 8, 8)
    blocks[:, 2:] = np.tile(q, (65536, 1))
    got = oracle.dequant(blocks.reshape(-1))
    scale = np.repeat(h.astype(np.uint16).view(np.float16).astype(np.float32), 8 * 32)
    qq = np.tile(q.reshape(-1).view(np.int8).astype(np.float32), 65536)
    ref = (scale * qq).astype(np.float32)
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]))


# ---- Q8_0 matvec -------------------------------------------------------------------------

@pytest.mark.parametrize("lanes", [8, 16, 32, 64])
def test_matvec_lanes_vs_exact(lanes):
    rows, k = 300, 2048
    w = synth.q8_matrix(4, "pin", rows, k)
    x = synth.normal_f32(5, k)
    deq = synth.dequantize_q8_0(w).reshape(rows, k).astype(np.float64)
    exact = deq @ x.astype(np.float64)                 # every product exact in float64
    got = oracle.matvec_lanes(w, x, rows, lanes)
    assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))
    assert np.max(np.abs(oracle.matvec_f64(w, x, rows) - exact)) <= 1e-12 * np.max(np.abs(exact))


def test_matvec_reference_fixture():
    """src/q8_test_main.cpp:80-131 fixture with its 2e-3 bound (:311-317)."""
    k, rows = 640, 257
    i = np.arange(k, dtype=np.float32)
    x = (np.sin(i * np.float32(0.031)) * np.float32(0.75)).astype(np.float32)
    r = np.arange(rows)[:, None]
    c = np.arange(k)[None, :]
    W = (np.cos(((r * 13 + c).astype(np.float32)) * np.float32(0.017)) * np.float32(0.5)).astype(np.float32)
    wq = oracle.quantize(W)
    reference = (synth.dequantize_q8_0(wq).reshape(rows, k).astype(np.float64) @ x.astype(np.float64))
    for lanes in (8, 16, 32, 64):
        assert np.max(np.abs(oracle.matvec_lanes(wq, x, rows, lanes) - reference)) <= 2e-3


# ---- elementwise ---------------------------------------------------------------------------

def test_gelu_reference_fixture_and_identities():
    """src/gelu_test_main.cpp:34-138 (n = 4096, 5e-5 abs against the float64 closed form)."""
    n = 4096
    i = np.arange(n, dtype=np.float32)
    gate = (np.sin(i * np.float32(0.0137)) * np.float32(5.0)).astype(np.float32)
    up = (np.cos(i * np.float32(0.0211)) * np.float32(3.0)).astype(np.float32)
    got = oracle.gelu_mul(gate, up)
    g = gate.astype(np.float64)
    closed = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * up
    assert np.max(np.abs(got - closed)) <= 5e-5
    assert oracle.gelu_mul(np.zeros(1), np.ones(1))[0] == 0.0
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    gp = oracle.gelu_mul(x, np.ones_like(x))
    gm = oracle.gelu_mul(-x, np.ones_like(x))
    assert np.max(np.abs((gp - gm) - x)) <= 2e-6 * 6      # gelu(x) - gelu(-x) = x


def test_argmax_rules():
    """shaders/argmax.comp:30-43: NaN never wins, larger wins, ties -> lowest index."""
    v = RNG.standard_normal(262144).astype(np.float32)
    assert oracle.argmax(v)[0] == int(np.argmax(v))
    v[[9, 100, 262000]] = 50.0
    assert oracle.argmax(v) == (9, 50.0)
    w = v.copy()
    w[3] = np.nan
    w[::5] = np.nan
    idx, val = oracle.argmax(w)
    clean = np.where(np.isnan(w), -np.inf, w)
    assert idx == int(np.argmax(clean)) and val == clean[idx]
    assert oracle.argmax(np.full(10, -np.inf, np.float32)) == (0, -np.inf)
    i, val = oracle.argmax(np.full(10, np.nan, np.float32))
    assert i == 0xFFFFFFFF and val == -np.inf


# ---- norms, RoPE, attention ------------------------------------------------------------------

def test_rms_norm_closed_forms():
    """src/gemma3.cpp:948-1043: all-ones input gives w / sqrt(1 + eps); scaling the input by a
    power of two scales nothing when eps is negligible; random input vs float64."""
    w = synth.normal_f32(3, 640, 0.1, 1.0)
    ones = np.ones(640, dtype=np.float32)
    s = np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(1e-6))
    assert np.array_equal(oracle.rms_norm_into(ones, w), (ones * s * w).astype(np.float32))
    x = synth.normal_f32(4, 640)
    y = oracle.rms_norm_into(x, w)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(y - ref)) <= 1e-6 * np.max(np.abs(ref))
    assert np.array_equal(oracle.rms_norm_into(x * np.float32(1024.0), w, 0.0), oracle.rms_norm_into(x, w, 0.0))
    # rms_norm_inplace multiplies by (scale * w) (src/gemma3.cpp:1036-1042), rms_norm_into
    # by scale then w (:991-996): the two differ by at most an ulp
    assert np.max(np.abs(oracle.rms_norm_inplace(x, w) - y) / np.abs(y)) <= 2.0 ** -22
    heads = oracle.rms_norm_heads(np.tile(x[:256], 4), w[:256], 4)
    assert np.array_equal(heads, np.tile(oracle.rms_norm_inplace(x[:256], w[:256]), 4))


def test_rope_identities():
    """src/gemma3.cpp:1309-1424: inverse frequencies vs float64, position 0 is the identity,
    rotation preserves each (i, i+128) pair's norm."""
    for theta in (1e4, 1e6):
        inv = oracle.rope_inv_freq(256, theta)
        ref = 1.0 / theta ** (np.arange(128) * 2 / 256.0)
        assert np.max(np.abs(inv - ref) / ref) <= 1e-6
        x = synth.normal_f32(8, 4 * 256)
        c, s = oracle.rope_table(inv, 0)
        assert np.array_equal(oracle.apply_rope(x, 4, 256, c, s), x)
        c, s = oracle.rope_table(inv, 777)
        y = oracle.apply_rope(x, 4, 256, c, s).reshape(4, 2, 128).astype(np.float64)
        xr = x.reshape(4, 2, 128).astype(np.float64)
        assert np.allclose(np.hypot(y[:, 0], y[:, 1]), np.hypot(xr[:, 0], xr[:, 1]), rtol=1e-6)


def test_attention_closed_forms():
    """src/gemma3.cpp:1609-1696: one position returns v exactly; identical keys give the mean
    of V; random case vs a float64 softmax."""
    hd, H = 256, 4
    q = synth.normal_f32(1, H * hd)
    k1 = synth.normal_f32(2, hd).reshape(1, hd)
    v1 = synth.normal_f32(3, hd).reshape(1, hd)
    assert np.array_equal(oracle.attention(q, k1, v1, H, hd, 0.0625), np.tile(v1[0], H))
    keys = np.tile(k1, (37, 1))
    vals = synth.normal_f32(4, 37 * hd).reshape(37, hd)
    out = oracle.attention(q, keys, vals, H, hd, 0.0625).reshape(H, hd)
    assert np.allclose(out, np.tile(vals.astype(np.float64).mean(0), (H, 1)), atol=2e-6)
    keys = synth.normal_f32(5, 300 * hd).reshape(300, hd)
    out = oracle.attention(q, keys, vals.repeat(9, 0)[:300], H, hd, 0.0625).reshape(H, hd)
    s = (q.reshape(H, hd).astype(np.float64) @ keys.T.astype(np.float64)) * 0.0625
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.max(np.abs(out - p @ vals.repeat(9, 0)[:300].astype(np.float64))) <= 1e-5
