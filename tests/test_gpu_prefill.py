"""Batched MFMA prefill (vrt_g3_prefill) against the oracle's serial prompt loop
(src/gemma3.cpp:2099-2111): last-position logits within 1e-3 of max|logit|, the same greedy
token, the hidden state within 1e-4, and decoding that continues from the prefilled KV cache
with the oracle's greedy tokens."""
import os

import numpy as np
import pytest

import oracle
import synth
import vrt

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
HIDDEN_TOL = 1e-4
MEDIUM = dict(n_layers=6, d_model=512, n_heads=4, head_dim=128, ffn=1024, vocab=2000, context=2048, window=64)


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / max(np.max(np.abs(b)), 1e-30))


def _check(ctx, path, prompt, n_cont, top2_margin=1e-4, kv_f16=False):
    g = vrt.Gemma3(ctx, path)
    m = oracle.Model(path, kv_f16=kv_f16)
    try:
        if kv_f16:
            g.set_kv_f16(True)
        print(f"[pf] {os.path.basename(path)}: prefill of {prompt.size} positions", flush=True)
        (idx, val), hid = g.prefill(prompt, top_k=8, hidden=True)
        logits = g.logits()
        for i, t in enumerate(prompt):
            last = i == prompt.size - 1
            r = m.decode(int(t), i, want_logits=last, logits=last)
        assert _rel(hid, r["hidden"]) <= HIDDEN_TOL
        assert _rel(logits, r["logits"]) <= LOGIT_TOL
        top = np.sort(r["logits"])[-2:]
        if top[1] - top[0] > top2_margin * abs(top[1]):
            assert idx == r["index"]
        # decoding continues from the prefilled cache
        tok, pos = r["index"], prompt.size
        for _ in range(n_cont):
            (gi, _), _ = g.decode(tok, pos, top_k=1)
            ro = m.decode(tok, pos, want_logits=True)
            assert gi == ro["index"], f"position {pos}"
            tok, pos = ro["index"], pos + 1
    finally:
        m.close()
        g.close()


def test_prefill_tiny(ctx, tiny_model):
    """6 blocks, window 8: local blocks mask keys outside the window and keep only the last 8
    positions in their KV ring."""
    _check(ctx, tiny_model, synth.uniform_ids(31, 45, 2, 1000), 12)


def test_prefill_tiny_short_prompts(ctx, tiny_model):
    for n in (1, 2, 7, 33):
        _check(ctx, tiny_model, synth.uniform_ids(100 + n, n, 2, 1000), 3)


def test_prefill_medium(ctx, model_dir):
    path = os.path.join(str(model_dir), "medium.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=21, **MEDIUM)
    _check(ctx, path, synth.uniform_ids(8, 300, 2, MEDIUM["vocab"]), 6)


LONG = dict(n_layers=6, d_model=256, n_heads=2, head_dim=64, ffn=512, vocab=1000, context=8192, window=64)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_prefill_segments(ctx, model_dir, kv_f16):
    """A prompt longer than the batched workspace (2048 positions) runs as segments of 2048,
    2048 and 404 positions: a segment's global blocks attend to every earlier position through
    the KV cache and its local blocks to the window's start rounded down to 32."""
    path = os.path.join(str(model_dir), "long8k.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=23, **LONG)
    _check(ctx, path, synth.uniform_ids(9, 4500, 2, LONG["vocab"]), 4, kv_f16=kv_f16)


LC_MODEL = dict(synth.GEMMA3_270M, n_layers=6, vocab=4096, context=8448)


def test_prefill_segments_long_context_golden(ctx, model_dir):
    """An 8192-token prompt at the Gemma-3-270M block shape (6 blocks, window 512, block 5
    global; head_dim 256) prefilled in four segments of 2048, then 16 teacher-forced decode steps
    against the oracle's vectors in tests/golden/long_context_6blk.npz (tests/golden/
    make_long_context.py, the long-context decode test's fixture): greedy ids identical, their
    logits within the tolerance, the last step's logits and hidden state within the tolerances.
    The segments' global attention reads up to 6144 earlier positions from the cache, the local
    blocks' their last 512."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "long_context_6blk.npz"))
    path = os.path.join(str(model_dir), "lc6.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=7, **LC_MODEL)
    n_check = gold["index"].size
    toks = synth.uniform_ids(8, 8192 + n_check, 2, LC_MODEL["vocab"])
    scale = np.max(np.abs(gold["last_logits"]))
    g = vrt.Gemma3(ctx, path)
    try:
        print("[pf] 8192-token prefill in segments at the 270M block shape", flush=True)
        g.prefill(toks[:8192], top_k=0)
        hid = None
        for j in range(n_check):
            p, last = 8192 + j, j == n_check - 1
            (idx, val), hid = g.decode(int(toks[p]), p, top_k=8 if last else 1, hidden=last)
            assert idx == int(gold["index"][j]), f"position {p}"
            assert abs(val - float(gold["value"][j])) <= LOGIT_TOL * scale, f"position {p}"
        assert _rel(g.logits(), gold["last_logits"]) <= LOGIT_TOL
        assert _rel(hid, gold["last_hidden"]) <= HIDDEN_TOL
    finally:
        g.close()


def test_prefill_full_shape_512(ctx, full_model):
    """The 512-token prefill workload at the Gemma-3-270M shape."""
    _check(ctx, full_model, synth.uniform_ids(4, 512, 2, 262144), 2)


def test_prefill_errors(ctx, tiny_model):
    g = vrt.Gemma3(ctx, tiny_model)
    try:
        with pytest.raises(RuntimeError, match="no input tokens"):
            g.prefill(np.zeros(0, np.uint32))
        with pytest.raises(RuntimeError, match="vocabulary"):
            g.prefill(np.array([5, 1000, 7], np.uint32))
        g.decode(5, 0, top_k=0)   # the failure reset the cache: position 0 again
    finally:
        g.close()
