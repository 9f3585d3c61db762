"""Batched greedy decode (vrt_g3_batch_*) against the oracle's single-sequence loop
(src/gemma3.cpp:1462-1882, one oracle model per sequence). The batched path computes every
projection and the LM head as MFMA GEMMs over the step's rows (the numerics of the prefill), so
its logits are held to the prefill's bound: within 1e-3 of max|logit|. The sequences are driven
with the oracle's own tokens (teacher forcing) and every greedy token must be identical to the
oracle's, as on the single-sequence path. (The oracle's smallest top-2 margin over these rows is
7.1e-4 of the top logit in the tiny-model cases and 2.9e-3 at the full shape; each row's margin
is printed with the failure.) Sequences join at different steps, so every step mixes rows at
different positions, local windows and chunk counts."""
import numpy as np
import pytest

import oracle
import synth
import vrt

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3     # of max|logit|, as for the prefill (the same GEMMs and hi/lo activation split)


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / max(np.max(np.abs(b)), 1e-30))


def _oracle_runs(path, prompts, n_new):
    """Per sequence: the tokens fed (prompt + greedy continuation) and the oracle's result at
    every position (index, value, top-2 margin, logits)."""
    runs = []
    m = oracle.Model(path)
    try:
        for pr in prompts:
            m.reset()
            feed, res = [], []
            tok = None
            for pos in range(len(pr) + n_new - 1):
                tok = int(pr[pos]) if pos < len(pr) else res[-1]["index"]
                feed.append(tok)
                r = m.decode(tok, pos, want_logits=True, logits=True)
                top = np.sort(r["logits"])[-2:]
                res.append(dict(index=r["index"], value=r["value"], logits=r["logits"],
                                margin=float(top[1] - top[0]) / max(abs(float(top[1])), 1e-30)))
            runs.append((feed, res))
    finally:
        m.close()
    return runs


def _drive(b, runs, starts, check_logits_every=1):
    """Feeds each sequence its oracle tokens, sequence i joining at step starts[i]; compares every
    row of every step with the oracle. Returns the number of rows checked."""
    n = len(runs)
    nxt = [0] * n
    step, checked = 0, 0
    while any(nxt[i] < len(runs[i][0]) for i in range(n)):
        rows = [i for i in range(n) if step >= starts[i] and nxt[i] < len(runs[i][0])]
        if rows:
            toks = [runs[i][0][nxt[i]] for i in rows]
            idx, val = b.step(rows, toks)
            for r, i in enumerate(rows):
                o = runs[i][1][nxt[i]]
                where = (f"sequence {i} position {nxt[i]} (step {step}, {len(rows)} rows; "
                         f"oracle top-2 margin {o['margin']:.3g})")
                assert int(idx[r]) == o["index"], where
                assert abs(float(val[r]) - o["value"]) <= LOGIT_TOL * float(np.max(np.abs(o["logits"]))), where
                if checked % check_logits_every == 0:
                    assert _rel(b.logits(r), o["logits"]) <= LOGIT_TOL, where
                assert b.position(i) == nxt[i] + 1
                nxt[i] += 1
                checked += 1
        step += 1
    return checked


def test_batch_tiny_staggered(ctx, tiny_model):
    """Six sequences of the 6-block model (window 8, one global block): prompts of 1..9 tokens
    joining at steps 0..11, 14 new tokens each; histories pass the window and a 64-position
    chunk boundary of the global block."""
    prompts = [synth.uniform_ids(200 + i, 1 + (i * 3) % 9, 2, 1000) for i in range(6)]
    runs = _oracle_runs(tiny_model, prompts, 14)
    g = vrt.Gemma3(ctx, tiny_model)
    b = vrt.Gemma3Batch(g, 8, 128)
    try:
        print("[batch] tiny: 6 sequences", flush=True)
        assert _drive(b, runs, starts=[0, 0, 2, 5, 7, 11]) == sum(len(r[0]) for r in runs)
    finally:
        b.close()
        g.close()


def test_batch_tiny_long_history(ctx, tiny_model):
    """Two sequences past 130 positions: the global block's history spans three chunks."""
    prompts = [synth.uniform_ids(301, 5, 2, 1000), synth.uniform_ids(302, 70, 2, 1000)]
    runs = _oracle_runs(tiny_model, prompts, 70)
    g = vrt.Gemma3(ctx, tiny_model)
    b = vrt.Gemma3Batch(g, 2, 256)
    try:
        print("[batch] tiny: long histories", flush=True)
        _drive(b, runs, starts=[0, 3], check_logits_every=7)
    finally:
        b.close()
        g.close()


def test_batch_full_shape(ctx, full_model):
    """Four sequences at the Gemma-3-270M shape (18 blocks, vocab 262144)."""
    prompts = [synth.uniform_ids(400 + i, 2 + i, 2, 262144) for i in range(4)]
    runs = _oracle_runs(full_model, prompts, 4)
    g = vrt.Gemma3(ctx, full_model)
    b = vrt.Gemma3Batch(g, 4, 64)
    try:
        print("[batch] full shape: 4 sequences", flush=True)
        _drive(b, runs, starts=[0, 1, 1, 2], check_logits_every=3)
    finally:
        b.close()
        g.close()


def test_batch_free_running_matches_single(ctx, tiny_model):
    """generate() with continuous batching gives each sequence the tokens the single-sequence
    executor generates for its prompt."""
    prompts = [synth.uniform_ids(500 + i, 3 + i, 2, 1000) for i in range(5)]
    g = vrt.Gemma3(ctx, tiny_model)
    b = vrt.Gemma3Batch(g, 5, 64)
    try:
        got = b.generate(prompts, 10, starts=[0, 2, 2, 4, 9])
        for i, pr in enumerate(prompts):
            want = g.generate(pr, 10)
            n = min(len(want), len(got[i]))
            np.testing.assert_array_equal(got[i][:n], want[:n], err_msg=f"sequence {i}")
    finally:
        b.close()
        g.close()


def test_batch_reset_and_reuse(ctx, tiny_model):
    """A sequence slot restarts at position 0 after reset and repeats its results; the other
    slots keep their positions."""
    g = vrt.Gemma3(ctx, tiny_model)
    b = vrt.Gemma3Batch(g, 3, 32)
    try:
        toks = synth.uniform_ids(600, 6, 2, 1000)
        first = [b.step([0, 1], [int(t), int(t)])[0].copy() for t in toks]
        assert b.position(0) == 6 and b.position(1) == 6 and b.position(2) == 0
        b.reset(0)
        assert b.position(0) == 0 and b.position(1) == 6
        again = [b.step([0], [int(t)])[0].copy() for t in toks]
        for a, c in zip(first, again):
            assert int(a[0]) == int(c[0]) == int(a[1])
        b.reset()
        assert all(b.position(i) == 0 for i in range(3))
    finally:
        b.close()
        g.close()


def test_batch_destroy_order(ctx, tiny_model):
    """The executor refuses to be destroyed while a batch over it is alive (the batch reads its
    weights and stream), and is destroyed once the batch is gone."""
    g = vrt.Gemma3(ctx, tiny_model)
    b = vrt.Gemma3Batch(g, 2, 16)
    try:
        b.step([0], [5])
        L = vrt.lib()
        assert L.vrt_g3_destroy(g.h) == vrt.VRT_ERR_STATE
        assert "batched decoder" in L.vrt_last_error().decode()
        idx, _ = b.step([0], [6])          # the batch still runs on the live executor
        assert 0 <= int(idx[0]) < 1000
    finally:
        b.close()
    g.close()                              # checks vrt_g3_destroy's status
    assert g.h is None


def test_batch_errors(ctx, tiny_model):
    g = vrt.Gemma3(ctx, tiny_model)
    try:
        with pytest.raises(RuntimeError, match="max_seqs"):
            vrt.Gemma3Batch(g, 0, 16)
        with pytest.raises(RuntimeError, match="max_ctx"):
            vrt.Gemma3Batch(g, 2, g.config.context_length + 1)
        b = vrt.Gemma3Batch(g, 2, 4)
        try:
            with pytest.raises(RuntimeError, match="twice"):
                b.step([1, 1], [5, 6])
            with pytest.raises(RuntimeError, match="out of range"):
                b.step([2], [5])
            b.step([0, 1], [5, 6])
            with pytest.raises(RuntimeError, match="vocabulary"):
                b.step([0, 1], [5, 1000])
            # the failed step reset both sequences
            assert b.position(0) == 0 and b.position(1) == 0
            for _ in range(4):
                b.step([0], [7])
            with pytest.raises(RuntimeError, match="context length"):
                b.step([0], [7])
            with pytest.raises(RuntimeError, match="row"):
                b.logits(1)
        finally:
            b.close()
    finally:
        g.close()
