"""GPU parity of the Gemma 3 executor (vrt_g3_*) against the CPU oracle's restatement of
src/gemma3.cpp.

Bars: teacher-forced greedy tokens identical; logits within 1e-3 of max|logit| (the relative
tolerance the workload states for fp32 logits); final hidden within 1e-4 of max|hidden|;
graph replay bit-identical to eager launches.
"""
import os

import numpy as np
import pytest

import oracle
import synth
import vrt

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
HIDDEN_TOL = 1e-4


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64))) / max(np.max(np.abs(b)), 1e-30))


def _oracle_forced(path, tokens, first_logit):
    m = oracle.Model(path)
    out = []
    for i, t in enumerate(tokens):
        r = m.decode(int(t), i, want_logits=i >= first_logit, logits=i >= first_logit)
        out.append(r)
    m.close()
    return out


def _top2_gap(logits):
    s = np.sort(logits)
    return float(s[-1] - s[-2])


@pytest.fixture(scope="module")
def tiny_g3(ctx, tiny_model):
    g = vrt.Gemma3(ctx, tiny_model)
    yield g
    g.close()


def test_tiny_teacher_forced_tokens_and_logits(ctx, tiny_model, tiny_g3):
    """40 positions with window 8: local layers evict, the global layer (block 5) keeps all."""
    toks = synth.uniform_ids(21, 40, 2, 1000)
    print(f"[g3] tiny forced n={toks.size}", flush=True)
    got = tiny_g3.forced(toks, 0)
    ref = _oracle_forced(tiny_model, toks, 0)
    for i, r in enumerate(ref):
        assert got["index"][i] == r["index"], f"step {i}: gpu {got['index'][i]} oracle {r['index']} gap {_top2_gap(r['logits'])}"
    # logits through the decode_token path (top_k > 1 keeps them)
    tiny_g3.reset()
    for i, t in enumerate(toks[:12]):
        (idx, val), hid = tiny_g3.decode(int(t), i, top_k=8, hidden=True)
        lg = tiny_g3.logits()
        assert _rel(lg, ref[i]["logits"]) <= LOGIT_TOL
        assert _rel(hid, ref[i]["hidden"]) <= HIDDEN_TOL
        assert idx == ref[i]["index"]


def test_tiny_generate_matches_oracle(ctx, tiny_model, tiny_g3):
    prompt = synth.uniform_ids(5, 5, 2, 1000)
    got = tiny_g3.generate(prompt, 30)
    m = oracle.Model(tiny_model)
    ref = m.generate(prompt, 30)
    m.close()
    assert np.array_equal(got, ref)


def test_generate_stops_at_eos(ctx, tiny_model, tmp_path):
    """EOS is appended and then ends the generation (src/gemma3.cpp:2134-2141), on the
    persistent kernel and on the multi-kernel path: the same weights with EOS set to a token
    the greedy loop produces stop right after it."""
    prompt = synth.uniform_ids(5, 5, 2, 1000)
    m = oracle.Model(tiny_model)
    free = m.generate(prompt, 30)
    m.close()
    k = next(i for i in range(3, free.size) if free[i] not in free[:i])
    path = str(tmp_path / "tiny_eos.gguf")
    synth.write_gemma3_gguf(path, seed=11, eos=int(free[k]), **synth.TINY)
    m = oracle.Model(path)
    ref = m.generate(prompt, 30)
    m.close()
    assert np.array_equal(ref, free[:k + 1])
    g = vrt.Gemma3(ctx, path)
    try:
        for persistent in (True, False):
            if persistent and not g.persistent_available():
                continue
            g.set_persistent(persistent)
            assert np.array_equal(g.generate(prompt, 30), ref), f"persistent={persistent}"
    finally:
        g.close()


def test_graph_replay_equals_eager(ctx, tiny_g3):
    toks = synth.uniform_ids(8, 20, 2, 1000)
    tiny_g3.set_graph(True)
    a = tiny_g3.forced(toks, 0)
    tiny_g3.set_graph(False)
    b = tiny_g3.forced(toks, 0)
    tiny_g3.set_graph(True)
    c = tiny_g3.forced(toks, 0)
    assert np.array_equal(a["index"], b["index"]) and np.array_equal(a["value"].view(np.uint32), b["value"].view(np.uint32))
    assert np.array_equal(a["value"].view(np.uint32), c["value"].view(np.uint32))


def test_no_window_keeps_full_history(ctx, tiny_model_nowindow):
    g = vrt.Gemma3(ctx, tiny_model_nowindow)
    toks = synth.uniform_ids(31, 24, 2, 1000)
    got = g.forced(toks, 4)
    ref = _oracle_forced(tiny_model_nowindow, toks, 4)
    g.close()
    for i in range(4, toks.size):
        assert got["index"][i] == ref[i]["index"]


def test_decode_errors_reset(ctx, tiny_g3):
    tiny_g3.reset()
    tiny_g3.decode(5, 0, top_k=1)
    with pytest.raises(vrt.VrtError, match="contiguous"):
        tiny_g3.decode(5, 2, top_k=1)
    with pytest.raises(vrt.VrtError, match="vocabulary"):
        tiny_g3.decode(1000, 1, top_k=1)
    # the vocabulary error reset the cache: position 0 is next again
    tiny_g3.decode(5, 0, top_k=0)
    with pytest.raises(vrt.VrtError, match="context length"):
        tiny_g3.generate(np.arange(2, 200, dtype=np.uint32), 100)


def test_full_shape_greedy_and_logits(ctx, full_model):
    """Config 2 in full: 8-token prompt, all 128 greedy tokens compared with the oracle's, then a
    teacher-forced pass over the same 135 positions comparing every hidden state and the last
    step's logits (positions 8..135: the chunked attention merge runs at histories of 33 and up)."""
    g = vrt.Gemma3(ctx, full_model)
    assert g.persistent_available(), "the Gemma-3-270M shape must run on the persistent decode kernel"
    prompt = synth.uniform_ids(0, 8, 2, 262144)
    n_new = 128
    print("[g3] full-shape generate", flush=True)
    got = g.generate(prompt, n_new)
    m = oracle.Model(full_model)
    ref = m.generate(prompt, n_new)
    assert np.array_equal(got, ref), f"gpu {got} oracle {ref}"
    # teacher-forced logits at the last position
    seq = np.concatenate([prompt, ref[:-1]]).astype(np.uint32)
    m.reset()
    g.reset()
    for i, t in enumerate(seq):
        last = i == seq.size - 1
        r = m.decode(int(t), i, want_logits=last, logits=last)
        (idx, _), hid = g.decode(int(t), i, top_k=8 if last else 0, hidden=True)
        assert _rel(hid, r["hidden"]) <= HIDDEN_TOL
    assert _rel(g.logits(), r["logits"]) <= LOGIT_TOL
    assert idx == r["index"]
    m.close()
    g.close()


def test_persistent_matches_multikernel(ctx, tiny_model):
    """The persistent decode kernel and the multi-kernel step agree on tokens; their logits
    agree within the logit tolerance (the attention split differs between them)."""
    g = vrt.Gemma3(ctx, tiny_model)
    assert g.persistent_available(), "persistent decode kernel not available for the test shape"
    toks = synth.uniform_ids(77, 48, 2, 1000)
    g.set_persistent(True)
    a = g.forced(toks, 0)
    g.set_persistent(False)
    b = g.forced(toks, 0)
    assert np.array_equal(a["index"], b["index"])
    assert np.max(np.abs(a["value"] - b["value"])) <= LOGIT_TOL * np.max(np.abs(b["value"]))
    g.set_persistent(True)
    prompt = synth.uniform_ids(3, 6, 2, 1000)
    p1 = g.generate(prompt, 40)
    g.set_persistent(False)
    p2 = g.generate(prompt, 40)
    g.close()
    assert np.array_equal(p1, p2)


def test_unfused_sequence_equals_fused(ctx, tiny_model):
    """Projection fusion off runs q, k, v, gate and up as launches of their own and the GELU
    product as a launch after them (src/gemma3.cpp:1529-1541, :1783-1847). Each row is computed
    as in the fused multi-kernel step, so a teacher-forced run gives bit-identical greedy
    results; the option reads back and switching it drops nothing else."""
    g = vrt.Gemma3(ctx, tiny_model)
    toks = synth.uniform_ids(5, 40, 2, 1000)
    g.set_persistent(False)
    a = g.forced(toks, 0)
    g.set_persistent(True)
    g.set_fusion(False)
    assert g.get_option(vrt.OPT_FUSION) == 0
    b = g.forced(toks, 0)
    g.set_fusion(True)
    c = g.forced(toks, 0)   # back on the persistent kernels
    g.close()
    assert np.array_equal(a["index"], b["index"]) and np.array_equal(a["value"], b["value"])
    assert np.array_equal(a["index"], c["index"])


CI_LANE_FUSION = [(64, False), (32, False), (16, False), (8, False), (8, True)]


def test_full_shape_lane_fusion_loop(ctx, full_model):
    """The reference CI's lane x fusion loop (.github/workflows/build.yml:105-123) at the 270M
    shape: each lane width with fusion off, then 8 lanes with it on. The embedding-width
    projections run with the requested lanes (20 blocks per row: 3 blocks per lane at 8), and
    the greedy tokens equal the oracle's."""
    g = vrt.Gemma3(ctx, full_model)
    prompt = synth.uniform_ids(0, 8, 2, 262144)
    m = oracle.Model(full_model)
    ref = m.generate(prompt, 4)
    m.close()
    auto = g.q8_lanes()
    for lanes, fusion in CI_LANE_FUSION:
        print(f"[g3] lanes {lanes} fusion {fusion}", flush=True)
        g.set_q8_lanes(lanes)
        g.set_fusion(fusion)
        assert g.q8_lanes() == lanes and g.get_option(vrt.OPT_Q8_LANES) == lanes
        got = g.generate(prompt, 4)
        assert np.array_equal(got, ref), (lanes, fusion, got, ref)
    with pytest.raises(vrt.VrtError):
        g.set_q8_lanes(12)
    g.set_q8_lanes(0)
    g.set_fusion(True)
    assert g.q8_lanes() == auto
    assert np.array_equal(g.generate(prompt, 4), ref)
    g.close()


def test_team_kernel_matches_allworkgroup_kernel(ctx, tiny_model):
    """The phase-team kernel holds the first 64 history positions in registers and the rest in
    LDS (passes of 64, an online softmax per wave); at head_dim 64 the tiny model's whole
    256-position context fits, so every step runs on it. Teacher-forced over 250 positions (the
    register pass and three LDS passes, the current position in each), team on and off give the
    same greedy tokens and logits within the logit tolerance (float sums with v_rsq and the
    deferred norms against double sums), with fp32, fp16 and bf16 entries; a generation gives
    the same tokens."""
    g = vrt.Gemma3(ctx, tiny_model)
    assert g.team_available(), "team kernel not built for the test shape"
    assert g.team_positions() == 256, g.team_positions()
    toks = synth.uniform_ids(91, 250, 2, 1000)
    for fmt in ("f32", "f16", "bf16"):
        g.set_kv_format(fmt)
        g.set_team(True)
        a = g.forced(toks, 0)
        g.set_team(False)
        b = g.forced(toks, 0)
        assert np.array_equal(a["index"], b["index"]), fmt
        assert np.max(np.abs(a["value"] - b["value"])) <= LOGIT_TOL * np.max(np.abs(b["value"])), fmt
    g.set_kv_format("f32")
    prompt = synth.uniform_ids(92, 20, 2, 1000)
    g.set_team(False)
    mk = g.generate(prompt, 150)
    g.set_team(True)
    tk = g.generate(prompt, 150)
    g.close()
    assert np.array_equal(tk, mk)


def test_team_kernel_history_modes_full_shape(ctx, full_model):
    """At the Gemma-3-270M shape every workgroup of a head holds the whole history on chip up
    to 136 positions with fp32 entries (64 in registers, 72 in LDS) and 208 with fp16 or bf16
    ones; longer histories split into 16 chunks per head whose partials the head's workgroups
    exchange and merge, so the team kernel takes every position. Teacher-forced across the
    switch, team on and off (the all-workgroup kernel) give the same greedy tokens and logits
    within the tolerance."""
    g = vrt.Gemma3(ctx, full_model)
    try:
        assert g.team_available()
        for fmt, switch in (("f32", 136), ("f16", 208), ("bf16", 208)):
            g.set_kv_format(fmt)
            assert g.team_positions() == int(g.config.context_length), (fmt, g.team_positions())
            assert g.team_chunked_from() == switch, (fmt, g.team_chunked_from())
            toks = synth.uniform_ids(94, switch + 12, 2, 262144)
            print(f"[g3] full shape, {toks.size} forced steps, {fmt} KV, team on/off", flush=True)
            g.set_team(True)
            a = g.forced(toks, 0)
            g.set_team(False)
            b = g.forced(toks, 0)
            assert np.array_equal(a["index"], b["index"]), fmt
            assert np.max(np.abs(a["value"] - b["value"])) <= LOGIT_TOL * np.max(np.abs(b["value"])), fmt
    finally:
        g.close()


RAGGED_VOCAB = dict(synth.GEMMA3_270M, n_layers=3, vocab=4099, context=512)


def test_team_lm_head_ragged_vocab(ctx, model_dir):
    """The team kernel's LM head at the 270M block width streams the table in 16-row tiles, each
    wave its own. With 4099 rows the last tile holds 3 rows, and most workgroups have no tile.
    Teacher-forced over 40 positions against the oracle: the greedy token, every logit and the
    hidden state of each step."""
    path = os.path.join(str(model_dir), "ragged_vocab.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=33, **RAGGED_VOCAB)
    toks = synth.uniform_ids(35, 40, 2, RAGGED_VOCAB["vocab"])
    g = vrt.Gemma3(ctx, path)
    m = oracle.Model(path)
    try:
        assert g.team_available(), "team kernel not built for the 270M block width"
        print(f"[g3] ragged vocabulary ({RAGGED_VOCAB['vocab']} rows), {toks.size} forced steps", flush=True)
        for i, t in enumerate(toks):
            r = m.decode(int(t), i, want_logits=True, logits=True)
            (idx, _), hid = g.decode(int(t), i, top_k=8, hidden=True)
            assert idx == r["index"], f"step {i}: gpu {idx} oracle {r['index']}"
            assert _rel(g.logits(), r["logits"]) <= LOGIT_TOL, f"step {i}"
            assert _rel(hid, r["hidden"]) <= HIDDEN_TOL, f"step {i}"
    finally:
        m.close()
        g.close()


def test_team_phase_trace(ctx, tiny_model):
    """The team kernel's phase trace of a launch whose first step runs the LM head: every
    workgroup stamps its team's input and publish of every block in order, the final norm and
    the LM head after the blocks, and the slots match the documented layout (2L + 3 + 8)."""
    g = vrt.Gemma3(ctx, tiny_model)
    L = int(g.config.block_count)
    g.set_trace(True)
    g.generate(synth.uniform_ids(93, 1, 2, 1000), 4)   # the traced first step runs the LM head
    tr = g.read_trace().astype(np.int64)
    g.set_trace(False)
    g.close()
    nwg, slots = tr.shape
    assert slots == 2 * L + 3 + 8, slots
    assert nwg % 8 == 0
    for w in range(nwg):
        ins, pubs = tr[w, :L], tr[w, L:2 * L]
        assert np.all(ins > 0) and np.all(pubs >= ins), w
        assert np.all(np.diff(ins) > 0) and np.all(np.diff(pubs) > 0), w
        start, fold, lm = tr[w, 2 * L], tr[w, 2 * L + 1], tr[w, 2 * L + 2]
        assert start <= ins[0] and pubs[-1] <= fold <= lm, w


def test_persistent_split_launches(ctx, tiny_model):
    """A generation split over several persistent launches equals one launch."""
    g = vrt.Gemma3(ctx, tiny_model)
    prompt = synth.uniform_ids(9, 7, 2, 1000)
    whole = g.generate(prompt, 30)
    g.start(prompt, 30)
    for n in (3, 1, 10, 7, 15):
        g.step(n)
    parts = g.collect()
    g.close()
    assert np.array_equal(whole, parts)


def test_exchange_buffers_read_back(ctx, tiny_model):
    """vrt_g3_read_exchange returns each all-workgroup persistent-kernel exchange buffer in row
    order: after a generation on that kernel (the team kernel off), the last block's q|k|v,
    gelu(gate)*up and down-projection words all carry that block's tag, and the down projection
    (one 64-byte line per four-row producer on the device) comes back compacted to d words."""
    g = vrt.Gemma3(ctx, tiny_model)
    try:
        if not g.persistent_available():
            pytest.skip("persistent kernel unavailable")
        g.set_team(False)
        g.generate(synth.uniform_ids(5, 6, 2, 1000), 4)
        cfg = g.config
        sizes = {0: cfg.head_count * cfg.head_dim + 2 * cfg.head_dim, 3: cfg.feed_forward_length,
                 4: cfg.embedding_length}
        for which, n in sizes.items():
            vals, tags = g.read_exchange(which)
            assert vals.size == n, which
            assert tags[0] != 0 and np.all(tags == tags[0]), (which, np.unique(tags))
            assert np.all(np.isfinite(vals)) and np.any(vals != 0.0), which
    finally:
        g.close()


MEDIUM = dict(n_layers=6, d_model=512, n_heads=4, head_dim=128, ffn=1024, vocab=2000, context=2048, window=64)


def test_long_history_chunked_attention(ctx, model_dir):
    """Histories far past one chunk: the global block attends over 700 positions (16 chunks of
    44, several 32-position groups each; the merge gathers its partials in two rounds), the
    local ones over their 64-position window. Teacher-forced tokens and logits of the last
    steps against the oracle."""
    path = os.path.join(str(model_dir), "medium.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=21, **MEDIUM)
    toks = synth.uniform_ids(5, 700, 2, MEDIUM["vocab"])
    first = toks.size - 6
    g = vrt.Gemma3(ctx, path)
    try:
        assert g.persistent_available()
        print("[g3] medium model, 700 forced steps", flush=True)
        got = g.forced(toks, first)
    finally:
        g.close()
    ref = _oracle_forced(path, toks, first)
    for i in range(first, toks.size):
        assert got["index"][i] == ref[i]["index"], f"step {i}"
        assert abs(got["value"][i] - ref[i]["value"]) <= LOGIT_TOL * np.max(np.abs(ref[i]["logits"]))


def test_long_context_full_shape(ctx, full_model):
    """Config 3 shape: an 8192-token prompt, then greedy steps, on the persistent kernel and on
    the multi-kernel step (an independent attention implementation): the same greedy tokens and
    argmax logits within the tolerance. Global blocks attend over up to 8200 positions."""
    g = vrt.Gemma3(ctx, full_model)
    toks = synth.uniform_ids(1, 8200, 2, 262144)
    first = 8192 - 1
    try:
        print("[g3] 8200 forced steps, persistent", flush=True)
        g.set_persistent(True)
        a = g.forced(toks, first)
        print("[g3] 8200 forced steps, multi-kernel", flush=True)
        g.set_persistent(False)
        b = g.forced(toks, first)
    finally:
        g.close()
    assert np.array_equal(a["index"][first:], b["index"][first:])
    scale = np.max(np.abs(b["value"][first:]))
    assert np.max(np.abs(a["value"][first:] - b["value"][first:])) <= LOGIT_TOL * scale


LC_MODEL = dict(synth.GEMMA3_270M, n_layers=6, vocab=4096, context=8448)


def test_long_context_vs_oracle_golden(ctx, model_dir):
    """Config 3's regime against the oracle: a 6-block model with the Gemma-3-270M block shape
    (global block 5), 8192 positions of uniform ids filling the cache, then 16 more teacher-forced
    steps whose greedy results are compared, so the global block attends over up to 8208
    positions (16 chunks of up to 513) and the local blocks over their 512-slot ring. The oracle's
    vectors are in tests/golden/long_context_6blk.npz (tests/golden/make_long_context.py: the oracle
    needs minutes for 8208 serial steps). Both decode paths: greedy ids identical, their logits
    within the tolerance; the last step's logits and hidden state within the tolerances."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "long_context_6blk.npz"))
    path = os.path.join(str(model_dir), "lc6.gguf")
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, seed=7, **LC_MODEL)
    n_check = gold["index"].size
    toks = synth.uniform_ids(8, 8192 + n_check, 2, LC_MODEL["vocab"])
    scale = np.max(np.abs(gold["last_logits"]))
    g = vrt.Gemma3(ctx, path)
    try:
        assert g.persistent_available()
        for persistent in (True, False):
            g.set_persistent(persistent)
            print(f"[g3] long context, 8208 forced steps, persistent={persistent}", flush=True)
            got = g.forced(toks, 8192)
            assert np.array_equal(got["index"][8192:], gold["index"]), f"persistent={persistent}"
            assert np.max(np.abs(got["value"][8192:] - gold["value"])) <= LOGIT_TOL * scale
        g.set_persistent(True)
        g.forced(toks[:-1], toks.size)                      # positions 0..8206, no LM head
        (idx, _), hid = g.decode(int(toks[-1]), toks.size - 1, top_k=8, hidden=True)
        assert idx == int(gold["index"][-1])
        assert _rel(g.logits(), gold["last_logits"]) <= LOGIT_TOL
        assert _rel(hid, gold["last_hidden"]) <= HIDDEN_TOL
    finally:
        g.close()


def _nan_model(model_dir, name, tensor, idx=0):
    """The tiny model with one NaN written into an F32 norm tensor."""
    import gguf
    base = os.path.join(str(model_dir), "tiny_for_nan.gguf")
    if not os.path.exists(base):
        synth.write_gemma3_gguf(base, seed=11, **synth.TINY)
    f = gguf.GgufFile.open(base)
    w = f.read_f32(tensor)
    f.close()
    w[idx] = np.nan
    path = os.path.join(str(model_dir), name)
    return synth.edit_gguf(base, path, f32={tensor: w})


@pytest.mark.parametrize("tensor,message", [
    ("blk.2.post_ffw_norm.weight", "Non-finite value after Gemma 3 block 2"),
    ("blk.1.attn_q_norm.weight", "Gemma 3 attention softmax failed"),
])
def test_device_detected_errors(ctx, model_dir, tensor, message):
    """A NaN in a norm weight: the oracle and every device path (persistent kernel, multi-kernel
    step, batched prefill) fail with the reference's message (src/gemma3.cpp:1857-1863 for a
    non-finite hidden state, :1609-1696 for the softmax denominator) and reset the KV cache
    (:1878-1881), after which position 0 is next and position 1 is refused."""
    path = _nan_model(model_dir, tensor.replace(".", "_") + ".gguf", tensor)
    m = oracle.Model(path)
    with pytest.raises(RuntimeError, match=message):
        for pos, t in enumerate([17, 33, 5]):
            m.decode(t, pos)
    m.close()
    g = vrt.Gemma3(ctx, path)
    try:
        for persistent in (True, False):
            print(f"[g3] NaN in {tensor}, persistent={persistent}", flush=True)
            g.set_persistent(persistent)
            g.reset()
            with pytest.raises(vrt.VrtError, match=message):
                for pos, t in enumerate([17, 33, 5]):
                    g.decode(t, pos, top_k=1)
            with pytest.raises(vrt.VrtError, match="contiguous"):
                g.decode(17, 1, top_k=1)
            with pytest.raises(vrt.VrtError, match=message):
                g.generate(np.array([17, 33, 5], np.uint32), 4)
        print(f"[g3] NaN in {tensor}, prefill", flush=True)
        with pytest.raises(vrt.VrtError, match=message):
            g.prefill(np.array([17, 33, 5, 8], np.uint32), top_k=1)
        with pytest.raises(vrt.VrtError, match="contiguous"):
            g.decode(17, 1, top_k=1)
    finally:
        g.close()
