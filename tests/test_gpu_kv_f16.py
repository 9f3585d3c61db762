"""The 16-bit KV cache options, fp16 (VRT_G3_OPT_KV_F16) and bf16 (VRT_G3_OPT_KV_BF16), against
the oracle's matching KV modes, in which keys and values are rounded to IEEE fp16 or bfloat16
(nearest even) as they enter the cache and every position's attention, the current one's
included, reads the rounded values. The reference lists an fp16/bf16 cache as a roadmap item
(README.md:190-192) without an implementation, so the oracle's modes are the specification; its
roundings are pinned against numpy's float16 and against the definition of round to nearest
even to bfloat16 (test_oracle_pins.py).

Bars: teacher-forced greedy tokens identical, logits and hidden state within the format's
resolution of their max |value| (fp16 1e-3 = 2^-10, bf16 4e-3 ~ 2^-8), on the persistent kernel,
the multi-kernel path and the batched prefill. The bars are the 16-bit resolution rather than
the fp32 cache's 1e-4: the GPU's and the oracle's fp32 keys and values agree to ~1e-7 relative,
so now and then one lies on the other side of a rounding boundary and the two caches hold
values one 16-bit ulp apart. Each option must change the results (it is not a no-op), the two
formats must differ from each other, and switching resets the cache."""
import os

import numpy as np
import pytest

import oracle
import synth
import vrt

pytestmark = pytest.mark.gpu

LOGIT_TOL = {"f16": 1e-3, "bf16": 4e-3}    # the format's resolution, see above
HIDDEN_TOL = {"f16": 1e-3, "bf16": 4e-3}
FORMATS = ["f16", "bf16"]
MEDIUM = dict(n_layers=6, d_model=512, n_heads=4, head_dim=128, ffn=1024, vocab=2000, context=2048, window=64)


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / max(np.max(np.abs(b)), 1e-30))


def _oracle_steps(path, tokens, first, fmt="f16"):
    m = oracle.Model(path, kv_f16=fmt == "f16", kv_bf16=fmt == "bf16")
    try:
        return [m.decode(int(t), i, want_logits=i >= first, logits=i >= first) for i, t in enumerate(tokens)]
    finally:
        m.close()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "multikernel"])
def test_kv_f16_decode_vs_oracle(ctx, tiny_model, persistent, fmt):
    toks = synth.uniform_ids(61, 40, 2, 1000)
    first = 4
    ref = _oracle_steps(tiny_model, toks, first, fmt)
    g = vrt.Gemma3(ctx, tiny_model)
    try:
        g.set_persistent(persistent)
        g.set_kv_format(fmt)
        assert g.kv_format() == fmt
        print(f"[kv16] tiny model, {toks.size} steps, {fmt}, persistent={persistent}", flush=True)
        for i, t in enumerate(toks):
            (idx, _), hid = g.decode(int(t), i, top_k=8 if i >= first else 1, hidden=i >= first)
            if i >= first:
                assert idx == ref[i]["index"], f"step {i}"
                assert _rel(g.logits(), ref[i]["logits"]) <= LOGIT_TOL[fmt], f"step {i}"
                assert _rel(hid, ref[i]["hidden"]) <= HIDDEN_TOL[fmt], f"step {i}"
    finally:
        g.close()


def test_kv_f16_changes_results_and_resets(ctx, tiny_model):
    toks = synth.uniform_ids(62, 24, 2, 1000)
    g = vrt.Gemma3(ctx, tiny_model)

    def run():
        for i, t in enumerate(toks):
            g.decode(int(t), i, top_k=8 if i + 1 == toks.size else 1)   # top_k > 1 keeps the logits
        return g.logits()

    try:
        l32 = run()
        out = {}
        for fmt, on in (("f16", g.set_kv_f16), ("bf16", g.set_kv_bf16)):
            on(True)   # resets: the next position is 0 again
            assert g.kv_format() == fmt
            with pytest.raises(RuntimeError, match="contiguous"):
                g.decode(int(toks[0]), 5, top_k=1)
            out[fmt] = run()
            assert not np.array_equal(l32, out[fmt]), fmt
            assert _rel(out[fmt], l32) <= (1e-2 if fmt == "f16" else 3e-2), fmt
            on(False)
            assert g.kv_format() == "f32"
            assert np.array_equal(run(), l32), fmt
        assert not np.array_equal(out["f16"], out["bf16"])
        # one format replaces the other; clearing the one not in use changes nothing
        g.set_kv_f16(True)
        g.set_kv_bf16(True)
        assert g.kv_format() == "bf16"
        assert np.array_equal(run(), out["bf16"])
        check = vrt.lib().vrt_g3_set_option(g.h, vrt.OPT_KV_F16, 0)
        assert check == vrt.VRT_OK and g.kv_format() == "bf16"
    finally:
        g.close()


@pytest.mark.parametrize("fmt", FORMATS)
def test_kv_f16_prefill_vs_oracle(ctx, tiny_model, fmt):
    """The batched prefill with a 16-bit cache against the oracle's serial loop in that mode,
    and decoding on from the prefilled cache."""
    prompt = synth.uniform_ids(63, 45, 2, 1000)
    ref = _oracle_steps(tiny_model, prompt, prompt.size - 1, fmt)
    g = vrt.Gemma3(ctx, tiny_model)
    m = oracle.Model(tiny_model, kv_f16=fmt == "f16", kv_bf16=fmt == "bf16")
    try:
        g.set_kv_format(fmt)
        (idx, _), hid = g.prefill(prompt, top_k=8, hidden=True)   # top_k > 1 keeps the logits
        assert idx == ref[-1]["index"]
        assert _rel(g.logits(), ref[-1]["logits"]) <= LOGIT_TOL[fmt]
        assert _rel(hid, ref[-1]["hidden"]) <= HIDDEN_TOL[fmt]
        for i, t in enumerate(prompt):
            m.decode(int(t), i, want_logits=False)
        tok, pos = ref[-1]["index"], prompt.size
        for _ in range(6):
            (gi, _), _ = g.decode(tok, pos, top_k=1)
            ro = m.decode(tok, pos, want_logits=True)
            assert gi == ro["index"], f"position {pos}"
            tok, pos = ro["index"], pos + 1
    finally:
        m.close()
        g.close()


@pytest.mark.parametrize("fmt", FORMATS)
def test_kv_f16_long_history(ctx, model_dir, fmt):
    """Chunked attention over 16-bit entries: a global block over 300 positions (several chunks),
    local blocks over their 64-slot ring, on both decode paths (the team kernel takes the steps
    below its history limit)."""
    path = os.path.join(str(model_dir), "medium.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=21, **MEDIUM)
    toks = synth.uniform_ids(64, 300, 2, MEDIUM["vocab"])
    first = toks.size - 4
    ref = _oracle_steps(path, toks, first, fmt)
    for persistent in (True, False):
        g = vrt.Gemma3(ctx, path)
        try:
            g.set_persistent(persistent)
            g.set_kv_format(fmt)
            print(f"[kv16] medium model, {toks.size} forced steps, {fmt}, persistent={persistent}", flush=True)
            got = g.forced(toks, first)
        finally:
            g.close()
        for i in range(first, toks.size):
            assert got["index"][i] == ref[i]["index"], f"step {i}"
            assert abs(got["value"][i] - ref[i]["value"]) <= LOGIT_TOL[fmt] * np.max(np.abs(ref[i]["logits"]))
