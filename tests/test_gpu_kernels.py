"""GPU parity of the standalone Q8_0 kernels (C ABI) against the CPU oracle.

Bars: quantiser bytes, dequant floats and argmax (index, value) bit-exact; matvec y within the
derived per-row error bound of the activation-limb arithmetic (_limb_bound) of the exact float64
oracle (and of the 8-lane reference order plus that order's own fp32 error); the reference
tests' own fixtures and tolerances (src/q8_test_main.cpp:80-317 2e-3 abs,
src/ffn_test_main.cpp:254-441 5e-3 abs, src/gelu_test_main.cpp:34-138 5e-5 abs).
"""
import numpy as np
import pytest

import oracle
import synth
import vrt

pytestmark = pytest.mark.gpu

U = 2.0 ** -24   # fp32 unit roundoff


def _limb_bound(w, x, rows):
    """Per-row bound on |y_gpu - y_exact| for the matvec on activation limbs (vrt_q8_device.hpp):
    x_k = s_b (a + b/254 + c/254^2) with s_b = amax_b / 127 errs by at most 3.0e-7 amax_b per
    element (fp32 rounding of 127/amax and of x * (127/amax): 2u each in units of 127; the third
    limb's rounding 0.5/254^2; the scale's own rounding 2u), taken as 4.8e-7 amax_b; the fp32
    block products d_w s_b t and the lane and DPP sums add at most (nblk + 4) u of the absolute
    sum, taken twice."""
    k = x.size
    nb = k // 32
    blk = np.asarray(w, dtype=np.uint8)[: rows * nb * 34].reshape(rows, nb, 34)
    d = np.abs(blk[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float64))
    q = np.abs(blk[:, :, 2:].view(np.int8).astype(np.float64))
    xb = np.abs(x.astype(np.float64)).reshape(nb, 32)
    amax = xb.max(axis=1)
    limb = (d * (q.sum(axis=2) * amax[None, :])).sum(axis=1) * 4.8e-7
    abs_sum = (d * (q * xb[None]).sum(axis=2)).sum(axis=1)
    return limb + 2.0 * (nb + 4) * U * abs_sum, abs_sum


def _check_matvec(y, w, x, rows, lanes=None):
    ref = oracle.matvec_f64(w, x, rows)
    bound, abs_sum = _limb_bound(w, x, rows)
    err = np.abs(y.astype(np.float64) - ref)
    worst = int(np.argmax(err / np.maximum(bound, 1e-300)))
    assert np.all(err <= bound + 1e-30), f"row {worst}: |dy| {err[worst]:.3e} > bound {bound[worst]:.3e}"
    if lanes is not None:   # the reference's 8-lane fp32 order errs by up to (K + 8) u of |terms| itself
        err_l = np.abs(y.astype(np.float64) - lanes.astype(np.float64))
        assert np.all(err_l <= bound + (x.size + 8) * U * abs_sum + 1e-30)


def _mv(ctx, wbytes, x, rows, off=0, pad_to=None):
    k = x.size
    buf = np.zeros(pad_to if pad_to else off + wbytes.size, dtype=np.uint8)
    buf[off:off + wbytes.size] = wbytes
    w = ctx.upload(buf)
    xd = ctx.upload(x.astype(np.float32))
    yd = ctx.alloc(rows * 4)
    vrt.q8_matvec(ctx, w, off, xd, yd, k, rows, w_bytes=buf.size)
    ctx.sync()
    return yd.read(np.float32, rows)


def _rel_err(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("rows,k", [(2048, 640), (640, 2048), (1536, 640), (640, 1024), (257, 640),
                                    (1, 32), (3, 64), (96, 96), (5, 3072), (7, 8192)])
def test_matvec_vs_exact(ctx, rows, k):
    print(f"[matvec] rows={rows} k={k}", flush=True)
    w = synth.q8_matrix(0, f"mv{rows}x{k}", rows, k, 0.02)
    x = synth.normal_f32(1, k, 1.0)
    y = _mv(ctx, w, x, rows)
    _check_matvec(y, w, x, rows, lanes=oracle.matvec_lanes(w, x, rows, 8))


def test_matvec_config0_seed0(ctx):
    """Config 0: W [2048 x 640] ~ N(0, 0.02) seed 0, x ~ N(0,1); and the [640 x 2048] down shape."""
    for rows, k in ((2048, 640), (640, 2048)):
        w32 = synth.normal_f32(0, rows * k, 0.02)
        wq = synth.quantize_q8_0(w32)
        assert np.array_equal(wq, oracle.quantize(w32))            # quantiser bytes bit-exact
        x = synth.normal_f32(100, k, 1.0)
        y = _mv(ctx, wq, x, rows)
        _check_matvec(y, wq, x, rows)


def test_matvec_offsets_and_tight_end(ctx):
    """4-byte (not 8) aligned offsets, odd block counts (2-byte aligned rows) and a buffer that
    ends exactly at the matrix end."""
    for rows, k, off in ((33, 96, 4), (17, 32, 12), (64, 160, 36)):
        w = synth.q8_matrix(3, f"off{rows}", rows, k)
        x = synth.normal_f32(4, k)
        y = _mv(ctx, w, x, rows, off=off, pad_to=off + w.size)
        _check_matvec(y, w, x, rows)


def test_reference_q8_fixture_and_multi(ctx):
    """src/q8_test_main.cpp fixture (640 x 257, cos/sin), run / pair / triplet packing and
    replay stability."""
    k, rows = 640, 257
    i = np.arange(k, dtype=np.float32)
    x = (np.sin(i * np.float32(0.031)) * np.float32(0.75)).astype(np.float32)
    r = np.arange(rows)[:, None]
    c = np.arange(k)[None, :]
    W = (np.cos(((r * 13 + c).astype(np.float32)) * np.float32(0.017)) * np.float32(0.5)).astype(np.float32)
    wq = synth.quantize_q8_0(W)
    deq = synth.dequantize_q8_0(wq).reshape(rows, k)
    reference = (deq.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    y = _mv(ctx, wq, x, rows)
    assert np.max(np.abs(y - reference)) <= 2e-3
    triple = np.concatenate([wq, wq, wq])
    wd = ctx.upload(triple)
    xd = ctx.upload(x)
    yd = ctx.alloc(3 * rows * 4)
    s = wq.size
    vrt.q8_matvec_multi(ctx, wd, [0, s, 2 * s], [rows] * 3, k, xd, yd)
    ctx.sync()
    packed = yd.read(np.float32, 3 * rows)
    for copy in range(3):
        assert np.max(np.abs(packed[copy * rows:(copy + 1) * rows] - reference)) <= 2e-3
    vrt.q8_matvec_multi(ctx, wd, [0, s], [rows] * 2, k, xd, yd)
    ctx.sync()
    pair = yd.read(np.float32, 2 * rows)
    assert np.array_equal(pair[:rows], packed[:rows])               # replay bit-stable
    assert np.array_equal(pair[rows:], packed[rows:2 * rows])


def test_config1_qkv_ffn(ctx):
    """Config 1: RMSNorm(x) then fused QKV [1024|256|256] x 640 and the FFN 2048/640."""
    d, ffn = 640, 2048
    x = synth.normal_f32(5, d, 1.0)
    wn = synth.normal_f32(6, d, 0.1, 1.0)
    xn = oracle.rms_norm_into(x, wn, 1e-6)
    names = [("q", 1024, d), ("k", 256, d), ("v", 256, d), ("gate", ffn, d), ("up", ffn, d), ("down", d, ffn)]
    mats = {n: synth.q8_matrix(1, n, r, kk) for n, r, kk in names}
    blob, offs = [], {}
    pos = 0
    for n, _, _ in names:
        offs[n] = pos
        blob.append(mats[n])
        pos += mats[n].size
        pad = (-pos) % 32
        blob.append(np.zeros(pad, np.uint8))
        pos += pad
    arena = np.concatenate(blob)
    wd = ctx.upload(arena)
    xd = ctx.upload(xn)
    qkv = ctx.alloc(1536 * 4)
    vrt.q8_matvec_multi(ctx, wd, [offs["q"], offs["k"], offs["v"]], [1024, 256, 256], d, xd, qkv)
    ws = ctx.alloc(2 * ffn * 4)
    y = ctx.alloc(d * 4)
    vrt.q8_ffn(ctx, wd, offs["gate"], offs["up"], offs["down"], d, ffn, d, xd, ws, y)
    ctx.sync()
    got_qkv = qkv.read(np.float32, 1536)
    o = 0
    for n, r in (("q", 1024), ("k", 256), ("v", 256)):   # packed in call order, each within the limb bound
        _check_matvec(got_qkv[o:o + r], mats[n], xn, r)
        o += r
    gate = oracle.matvec_f64(mats["gate"], xn, ffn).astype(np.float32)
    up = oracle.matvec_f64(mats["up"], xn, ffn).astype(np.float32)
    h = oracle.gelu_mul(gate, up)
    ref = oracle.matvec_f64(mats["down"], h, d)
    # the workspace holds [gelu(gate) * up | up] (each gate/up row within its limb bound)
    wsv = ws.read(np.float32, 2 * ffn)
    _check_matvec(wsv[ffn:], mats["up"], xn, ffn)
    assert _rel_err(wsv[:ffn], h.astype(np.float64)) <= 1e-5
    assert _rel_err(y.read(np.float32, d), ref) <= 2e-4


def test_reference_ffn_fixture(ctx):
    """src/ffn_test_main.cpp:254-441: 64 -> 96 -> 64, variant-B quantiser, 5e-3 abs, replay 1e-6."""
    def mat(k, rows, seed):
        r = np.arange(rows)[:, None].astype(np.uint32)
        c = np.arange(k)[None, :].astype(np.uint32)
        phase = (seed * 97 + r * 131 + c * 17).astype(np.float32)
        v = (np.sin(phase * np.float32(0.0031)) * np.float32(0.45) +
             np.cos(phase * np.float32(0.0017)) * np.float32(0.15)).astype(np.float32)
        return synth.quantize_q8_0(v, "b")
    g, u, dn = mat(64, 96, 1), mat(64, 96, 2), mat(96, 64, 3)
    arena = np.concatenate([g, u, dn])
    x = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.071)) * np.float32(0.8)).astype(np.float32)
    gate = oracle.matvec_f64(g, x, 96).astype(np.float32)
    up = oracle.matvec_f64(u, x, 96).astype(np.float32)
    ref = oracle.matvec_f64(dn, oracle.gelu_mul(gate, up), 64).astype(np.float32)
    wd = ctx.upload(arena)
    xd = ctx.upload(x)
    ws = ctx.alloc(2 * 96 * 4)
    y = ctx.alloc(64 * 4)
    vrt.q8_ffn(ctx, wd, 0, g.size, g.size + u.size, 64, 96, 64, xd, ws, y)
    ctx.sync()
    a = y.read(np.float32, 64)
    vrt.q8_ffn(ctx, wd, 0, g.size, g.size + u.size, 64, 96, 64, xd, ws, y)
    ctx.sync()
    b = y.read(np.float32, 64)
    assert np.max(np.abs(a - ref)) <= 5e-3
    assert np.max(np.abs(a - b)) <= 1e-6


def test_gelu_fixture(ctx):
    """src/gelu_test_main.cpp:34-138: n = 4096, 5e-5 abs against float tanh."""
    n = 4096
    i = np.arange(n, dtype=np.float32)
    gate = (np.sin(i * np.float32(0.0137)) * np.float32(5.0)).astype(np.float32)
    up = (np.cos(i * np.float32(0.0211)) * np.float32(3.0)).astype(np.float32)
    ref = oracle.gelu_mul(gate, up)
    gd, ud = ctx.upload(gate), ctx.upload(up)
    vrt.gelu_mul(ctx, gd, ud, n)
    ctx.sync()
    got = gd.read(np.float32, n)
    assert np.max(np.abs(got - ref)) <= 5e-5
    # and against the float64 closed form of the same expression
    x = gate.astype(np.float64)
    closed = 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3))) * up
    assert np.max(np.abs(got - closed)) <= 5e-5


def _argmax_gpu(ctx, v):
    xd = ctx.upload(np.ascontiguousarray(v, dtype=np.float32))
    out = ctx.alloc(8)
    vrt.argmax(ctx, xd, v.size, out)
    ctx.sync()
    r = out.read(np.uint32, 2)
    return int(r[0]), float(r[1:2].view(np.float32)[0])


def test_argmax_rules(ctx):
    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(262144).astype(np.float32), rng.standard_normal(1).astype(np.float32),
             rng.standard_normal(1000).astype(np.float32)]
    t = rng.standard_normal(262144).astype(np.float32)
    t[[5, 77, 262143]] = 9.0                     # tie -> lowest index
    cases.append(t)
    nanv = rng.standard_normal(5000).astype(np.float32)
    nanv[::7] = np.nan                          # NaN never wins
    nanv[3] = np.nan
    cases.append(nanv)
    cases.append(np.full(300, -np.inf, dtype=np.float32))   # all -inf -> index 0
    z = np.zeros(513, dtype=np.float32)
    z[:10] = -0.0                               # -0 == +0: lowest index
    cases.append(z)
    cases.append(np.full(17, np.nan, dtype=np.float32))     # nothing qualifies
    for v in cases:
        gi, gv = _argmax_gpu(ctx, v)
        oi, ov = oracle.argmax(v)
        assert gi == oi and (np.float32(gv).tobytes() == np.float32(ov).tobytes())


def test_quantize_bit_exact(ctx):
    rng = np.random.default_rng(9)
    parts = [synth.normal_f32(2, 32 * 20000, 0.02),
             (rng.standard_normal(32 * 4000) * 10.0 ** rng.integers(-8, 6, 32 * 4000)).astype(np.float32)]
    edge = np.zeros(32 * 8, dtype=np.float32)
    edge[32:64] = 1e-41                         # subnormal block
    edge[64:96] = np.linspace(-3, 3, 32)
    edge[96:128] = 65504.0 * 127                # scale overflows fp16 -> inf
    edge[128:160] = np.nan                      # NaN block
    edge[160] = np.inf
    edge[192:224] = (1.0 + 2.0 ** -11) * 127    # scale tie case
    parts.append(edge)
    x = np.concatenate(parts).astype(np.float32)
    xd = ctx.upload(x)
    for variant, name in ((0, "a"), (1, "b")):
        out = ctx.alloc(x.size // 32 * 34)
        vrt.q8_quantize(ctx, xd, x.size, variant, out)
        ctx.sync()
        got = out.read(np.uint8, x.size // 32 * 34)
        ref = oracle.quantize(x, name)
        bad = np.nonzero((got != ref).reshape(-1, 34).any(axis=1))[0]
        assert bad.size == 0, f"variant {name}: {bad.size} blocks differ, first {bad[:8]} " \
                              f"x={x.reshape(-1, 32)[bad[0]][:4]} gpu={got.reshape(-1, 34)[bad[0]][:6]} " \
                              f"ref={ref.reshape(-1, 34)[bad[0]][:6]}"
        assert np.array_equal(got, synth.quantize_q8_0(x, name))


def test_dequantize_exhaustive(ctx):
    """Every fp16 scale against every int8 value (65536 x 256)."""
    h = np.arange(65536, dtype=np.uint32)
    blocks = np.zeros((65536 * 8, 34), dtype=np.uint8)
    q = np.arange(256, dtype=np.uint8).reshape(8, 32)
    blocks[:, 0] = np.repeat(h & 0xFF, 8)
    blocks[:, 1] = np.repeat(h >> 8, 8)
    blocks[:, 2:] = np.tile(q, (65536, 1))
    flat = blocks.reshape(-1)
    bd = ctx.upload(flat)
    out = ctx.alloc(65536 * 8 * 32 * 4)
    vrt.q8_dequantize(ctx, bd, 65536 * 8, out)
    ctx.sync()
    got = out.read(np.float32, 65536 * 8 * 32)
    ref = oracle.dequant(flat)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_argument_errors(ctx):
    w = ctx.alloc(1024)
    x = ctx.alloc(256)
    y = ctx.alloc(256)
    with pytest.raises(vrt.VrtError, match="divisible by 32"):
        vrt.q8_matvec(ctx, w, 0, x, y, 33, 1)
    with pytest.raises(vrt.VrtError, match="4-byte aligned"):
        vrt.q8_matvec(ctx, w, 2, x, y, 32, 1)
    with pytest.raises(vrt.VrtError, match="too small"):
        vrt.q8_matvec(ctx, w, 0, x, y, 32, 1000, w_bytes=1024)
    with pytest.raises(vrt.VrtError, match="non-zero"):
        vrt.argmax(ctx, x, 0, y)
