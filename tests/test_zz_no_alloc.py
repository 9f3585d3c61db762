"""vrt_q8_ffn_noalloc (the FFN entry point that allocates nothing: its [h | up] workspace is a
static per-device array of the library) against vrt_q8_ffn on a caller-allocated workspace:
bit-identical outputs on two calls in a row, the second with a smaller shape, and a clear error
past the static workspace's limit."""
import numpy as np
import pytest

import synth
import vrt

pytestmark = pytest.mark.gpu


def _ffn_weights(seed, k, ffn, out):
    mats = [synth.q8_matrix(seed, n, r, c) for n, r, c in (("gate", ffn, k), ("up", ffn, k), ("down", out, ffn))]
    offs, pos, blob = [], 0, []
    for m in mats:
        offs.append(pos)
        blob.append(m)
        pos += m.size
        pad = (-pos) % 32
        blob.append(np.zeros(pad, np.uint8))
        pos += pad
    return np.concatenate(blob), offs


@pytest.mark.parametrize("shapes", [((640, 2048, 640), (128, 256, 96))])
def test_noalloc_ffn_matches_workspace_ffn(ctx, shapes):
    for i, (k, ffn, out) in enumerate(shapes):
        print(f"[noalloc] call {i}: k={k} ffn={ffn} out={out}", flush=True)
        arena, offs = _ffn_weights(10 + i, k, ffn, out)
        wd = ctx.upload(arena)
        xd = ctx.upload(synth.normal_f32(20 + i, k))
        ws = ctx.alloc(2 * ffn * 4)
        y_ref = ctx.alloc(out * 4)
        y = ctx.alloc(out * 4)
        vrt.q8_ffn(ctx, wd, offs[0], offs[1], offs[2], k, ffn, out, xd, ws, y_ref)
        vrt.q8_ffn_noalloc(ctx, wd, offs[0], offs[1], offs[2], k, ffn, out, xd, y)
        ctx.sync()
        a = y_ref.read(np.float32, out)
        b = y.read(np.float32, out)
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {i}"


def test_noalloc_ffn_rejects_oversize(ctx):
    arena, offs = _ffn_weights(3, 32, 32, 32)
    wd = ctx.upload(arena)
    xd = ctx.upload(synth.normal_f32(4, 32))
    y = ctx.alloc(32 * 4)
    with pytest.raises(vrt.VrtError, match="static workspace"):
        vrt.q8_ffn_noalloc(ctx, wd, offs[0], offs[1], offs[2], 32, 16384 + 32, 32, xd, y)
