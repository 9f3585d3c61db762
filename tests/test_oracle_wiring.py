"""Pins of the oracle's block wiring (src/gemma3.cpp:1511-1864, :1301-1307) by invariants that
follow from the architecture rather than from the oracle's own formulas, and a demonstration
that plausible misreadings of the reference fail them.

Invariants (synthetic 6-block model: d 128, 2 query heads x 64, FFN 256, vocab 1000, window 8,
block 5 global):

* Power-of-two scale absorption (eps = 0). RMSNorm(2^k x) == RMSNorm(x) bit for bit when eps is
  0 (the double sum of squares, the quotient by n, the float square root and its reciprocal all
  move by exact powers of two). So doubling every Q8_0 scale of attn_q (absorbed by QK-norm),
  attn_k (QK-norm), attn_v and attn_output (the post-attention norm), ffn_up and ffn_down (the
  post-FFW norm; gelu(g) * 2u == 2 (gelu(g) * u)) leaves hidden state and logits bit-identical,
  while doubling ffn_gate (inside GELU) changes them.
* Window 1. With sliding_window 1 a local block sees only the current position, so an earlier
  token reaches later positions only through a global block ((l + 1) % 6 == 0): changing
  token 0 changes positions >= 1 of a 6-block model and none of a 5-block model.
* rope.freq_base reaches only global blocks: changing it changes a 6-block model's outputs and
  leaves a 5-block model's bit-identical.
* Branch norms. With ffn_gate zero the FFN adds exactly 0, so ffn_norm and post_ffw_norm
  cannot matter while attn_norm and post_attention_norm do; with attn_v zero the attention adds
  exactly 0, so attn_norm, the QK-norm weights and post_attention_norm cannot matter while
  ffn_norm and post_ffw_norm do.
* Zero projections. Every block projection zero: each block is the identity, and the hidden
  state is RMSNorm(embedding(t) * sqrt(d)) * w_out (float64 check).
* Attention sub-path (src/gemma3.cpp:1557-1696), from the oracle's per-block intermediates
  (or_g3_set_taps) against float64 restatements of the published operations: the query the
  attention reads is per-head RMSNorm (Zhang & Sennrich 2019) of the q projection times the
  q-norm weight, then RoPE (Su et al. 2021, the NeoX half-split pairing (i, i + hd/2)) with
  inverse frequencies base^(-2i/hd) at the block's base; the newest cached key is the k
  projection through the same two steps with the k-norm weight; the newest cached value is the v
  projection bit for bit (no norm on v); per head, q.k of the current position after RoPE equals
  the dot product before it (true only when q and k turn by one table); earlier cache rows are
  earlier steps' newest rows, oldest first, min(p + 1, window) of them in local blocks and p + 1
  in global ones; the attention output is softmax(q K^T / sqrt(hd)) V (Vaswani et al. 2017).

The mutants are compiled from patched copies of oracle/vrt_oracle.c in a temporary directory;
each must fail at least one invariant, the unpatched oracle must pass them all.
"""
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import gguf
import oracle
import synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SRC = os.path.join(REPO, "oracle")

NL = synth.TINY["n_layers"]
TOKS = [17, 402, 9, 733, 58, 260, 911, 4, 77, 123]   # 10 positions: the 8-slot windows evict
SEED = 41
Q8_ABSORBED = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_down")


def _model(d, name, **kw):
    p = os.path.join(d, name + ".gguf")
    if not os.path.exists(p):
        args = dict(synth.TINY)
        args.update(kw)
        synth.write_gemma3_gguf(p, seed=args.pop("seed", SEED), **args)
    return p


def _norm_values(name, n, salt):
    return synth.normal_f32(synth.tensor_seed(SEED + salt, name), n, 0.1, 1.0)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("wiring"))
    m = {}
    base0 = _model(d, "eps0", eps=0.0)
    m["eps0"] = base0
    for t in Q8_ABSORBED + ("ffn_gate",):
        m["x2_" + t] = synth.edit_gguf(base0, os.path.join(d, f"x2_{t}.gguf"),
                                       q8_scale_exp={f"blk.{l}.{t}.weight": 1 for l in range(NL)})
    m["x2_all"] = synth.edit_gguf(base0, os.path.join(d, "x2_all.gguf"),
                                  q8_scale_exp={f"blk.{l}.{t}.weight": 1 for l in range(NL) for t in Q8_ABSORBED})
    for nl in (5, 6):
        m[f"w1_{nl}"] = _model(d, f"w1_{nl}", n_layers=nl, window=1)
        m[f"rope_a_{nl}"] = _model(d, f"rope_a_{nl}", n_layers=nl, rope_global=1.0e6)
        m[f"rope_b_{nl}"] = _model(d, f"rope_b_{nl}", n_layers=nl, rope_global=5.0e4)
    base = _model(d, "base")
    m["base"] = base
    hd, dm = synth.TINY["head_dim"], synth.TINY["d_model"]
    sizes = {"attn_norm": dm, "attn_q_norm": hd, "attn_k_norm": hd, "post_attention_norm": dm,
             "ffn_norm": dm, "post_ffw_norm": dm}
    for branch, zero in (("ffn_off", "ffn_gate"), ("attn_off", "attn_v")):
        z = synth.edit_gguf(base, os.path.join(d, branch + ".gguf"),
                            q8_zero=[f"blk.{l}.{zero}.weight" for l in range(NL)])
        m[branch] = z
        for i, (t, n) in enumerate(sizes.items()):
            m[f"{branch}_{t}"] = synth.edit_gguf(
                z, os.path.join(d, f"{branch}_{t}.gguf"),
                f32={f"blk.{l}.{t}.weight": _norm_values(f"blk.{l}.{t}.weight", n, 100 + i) for l in range(NL)})
    m["zero_proj"] = _model(d, "zero_proj", weight_std=0.0, embd_std=0.02)
    return m


# ---- runners --------------------------------------------------------------------------------

def oracle_runner(lib_path=None):
    """(path, tokens) -> [(hidden, logits)] per position, or None if the decode raised. The
    runner's lib_path attribute names the oracle library it loads (None: the built one)."""
    def run(path, toks):
        m = oracle.Model(path, lib_path=lib_path)
        try:
            out = []
            for i, t in enumerate(toks):
                r = m.decode(int(t), i, want_logits=True, logits=True)
                out.append((r["hidden"], r["logits"]))
            return out
        except RuntimeError:
            return None
        finally:
            m.close()
    run.lib_path = lib_path
    return run


def _same_pos(a, b):
    return all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a, b))


def _same(a, b):
    return a is not None and b is not None and all(_same_pos(x, y) for x, y in zip(a, b))


# ---- invariants (each returns a list of failure descriptions) --------------------------------

def inv_scale_absorption(run, m):
    bad = []
    ref = run(m["eps0"], TOKS)
    if ref is None:
        return ["base model failed to decode"]
    for t in Q8_ABSORBED + ("all",):
        if not _same(run(m["x2_" + t], TOKS), ref):
            bad.append(f"2 x {t} scales changed the outputs")
    if _same(run(m["x2_ffn_gate"], TOKS), ref):
        bad.append("2 x ffn_gate scales left the outputs unchanged")
    return bad


def inv_window1_flow(run, m):
    bad = []
    alt = [900] + TOKS[1:]
    for nl, flows in ((5, False), (6, True)):
        a, b = run(m[f"w1_{nl}"], TOKS), run(m[f"w1_{nl}"], alt)
        if a is None or b is None:
            bad.append(f"{nl} blocks: decode failed")
            continue
        later_same = all(_same_pos(a[i], b[i]) for i in range(1, len(TOKS)))
        if later_same == flows:
            bad.append(f"{nl} blocks, window 1: token 0 {'did not reach' if flows else 'reached'} later positions")
    return bad


def inv_rope_base_global_only(run, m):
    bad = []
    for nl, reaches in ((5, False), (6, True)):
        a, b = run(m[f"rope_a_{nl}"], TOKS), run(m[f"rope_b_{nl}"], TOKS)
        if a is None or b is None:
            bad.append(f"{nl} blocks: decode failed")
        elif _same(a, b) == reaches:
            bad.append(f"{nl} blocks: rope.freq_base {'had no effect' if reaches else 'changed the outputs'}")
    return bad


def inv_branch_norms(run, m):
    bad = []
    cases = (("ffn_off", ("ffn_norm", "post_ffw_norm"), ("attn_norm", "post_attention_norm")),
             ("attn_off", ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm"),
              ("ffn_norm", "post_ffw_norm")))
    for branch, inert, live in cases:
        ref = run(m[branch], TOKS)
        if ref is None:
            bad.append(f"{branch}: decode failed")
            continue
        for t in inert:
            if not _same(run(m[f"{branch}_{t}"], TOKS), ref):
                bad.append(f"{branch}: {t} changed the outputs")
        for t in live:
            if _same(run(m[f"{branch}_{t}"], TOKS), ref):
                bad.append(f"{branch}: {t} had no effect")
    return bad


def inv_zero_projection(run, m):
    path = m["zero_proj"]
    out = run(path, TOKS[:4])
    if out is None:
        return ["zero-projection model failed to decode"]
    f = gguf.GgufFile.open(path)
    try:
        dm = synth.TINY["d_model"]
        w_out = f.read_f32("output_norm.weight").astype(np.float64)
        deq = synth.dequantize_q8_0(f.tensor_bytes("token_embd.weight")).reshape(-1, dm).astype(np.float64)
    finally:
        f.close()
    bad = []
    for (hid, _), tok in zip(out, TOKS[:4]):
        h = deq[tok] * np.float64(np.sqrt(np.float32(dm), dtype=np.float32))
        ref = h / np.sqrt(np.mean(h ** 2) + 1e-6) * w_out
        if np.max(np.abs(hid - ref)) > 1e-6 * np.max(np.abs(ref)):
            bad.append(f"token {tok}: hidden state is not the normed embedding")
    return bad


LOCAL_ROPE_BASE = 1.0e4   # src/gemma3.cpp:271-274: local blocks always turn at base 10000


def _rms64(x, w, eps):
    """Per-row RMSNorm in float64: x / sqrt(mean(x^2) + eps) * w."""
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w.astype(np.float64)


def _rope64(x, pos, base):
    """RoPE of rows x [.., hd] at position pos in float64: pair (i, i + hd/2) turned by
    pos * base^(-2i/hd)."""
    hd = x.shape[-1]
    half = hd // 2
    ang = pos * np.power(np.float64(base), -2.0 * np.arange(half, dtype=np.float64) / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def _sdpa64(q, keys, values, scale):
    """Scaled dot-product attention in float64 for heads q [H, hd] over keys/values [T, hd]."""
    s = (q.astype(np.float64) @ keys.astype(np.float64).T) * scale
    e = np.exp(s - s.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)) @ values.astype(np.float64)


def inv_attention_subpath(run, m):
    path = m["base"]
    f = gguf.GgufFile.open(path)
    try:
        nl = synth.TINY["n_layers"]
        qn = [f.read_f32(f"blk.{l}.attn_q_norm.weight") for l in range(nl)]
        kn = [f.read_f32(f"blk.{l}.attn_k_norm.weight") for l in range(nl)]
    finally:
        f.close()
    md = oracle.Model(path, lib_path=run.lib_path)
    try:
        info = md.info
        H, hd, eps, win = info.head_count, info.head_dim, float(info.rms_epsilon), info.sliding_window
        bases = [info.global_rope_base if (l + 1) % 6 == 0 else LOCAL_ROPE_BASE for l in range(nl)]
        steps, bad = [], []
        for p, tok in enumerate(TOKS):
            try:
                r = md.decode_taps(tok, p, hist_cap=len(TOKS))
            except RuntimeError as e:
                return [f"position {p}: decode failed ({e})"]
            steps.append(r)
            for l in range(nl):
                where = f"position {p} block {l}"
                glob = (l + 1) % 6 == 0
                hist = int(r["history"][l])
                if hist != (p + 1 if glob else min(p + 1, win)):
                    bad.append(f"{where}: {hist} cached rows")
                    continue
                qn64 = _rms64(r["q_proj"][l].reshape(H, hd), qn[l], eps)
                kn64 = _rms64(r["k_proj"][l], kn[l], eps)
                q_want = _rope64(qn64, p, bases[l])
                k_want = _rope64(kn64, p, bases[l])
                q_att = r["q_att"][l].reshape(H, hd).astype(np.float64)
                keys, values = r["keys"][l, :hist], r["values"][l, :hist]
                if np.max(np.abs(q_att - q_want)) > 2e-5 * np.max(np.abs(q_want)):
                    bad.append(f"{where}: query is not QK-norm then RoPE of the q projection")
                if np.max(np.abs(keys[-1] - k_want)) > 2e-5 * np.max(np.abs(k_want)):
                    bad.append(f"{where}: newest key is not QK-norm then RoPE of the k projection")
                if not np.array_equal(values[-1].view(np.uint32), r["v_proj"][l].view(np.uint32)):
                    bad.append(f"{where}: newest value is not the v projection")
                d_rot = q_att @ keys[-1].astype(np.float64)
                d_raw = qn64 @ kn64
                if np.max(np.abs(d_rot - d_raw)) > 2e-5 * np.max(np.abs(qn64)) * np.max(np.abs(kn64)) * hd ** 0.5:
                    bad.append(f"{where}: q.k at the current position changed under RoPE")
                for t in range(hist - 1):
                    e = steps[p - (hist - 1) + t]
                    eh = int(e["history"][l])
                    if not (np.array_equal(keys[t], e["keys"][l, eh - 1]) and
                            np.array_equal(values[t], e["values"][l, eh - 1])):
                        bad.append(f"{where}: cache row {t} is not position {p - (hist - 1) + t}'s entry")
                        break
                att_want = _sdpa64(q_att, keys, values, 1.0 / np.sqrt(hd))
                if np.max(np.abs(r["att"][l].reshape(H, hd) - att_want)) > 1e-5 * np.max(np.abs(values)):
                    bad.append(f"{where}: attention output is not softmax(q K^T / sqrt(hd)) V")
            if bad:
                return bad
        return bad
    finally:
        md.close()


# Invariants over a decoder's outputs only (hidden state and logits per position): they also run
# through the HIP executor (test_gpu_wiring.py). The attention sub-path invariant reads the
# oracle's intermediates and applies to the oracle.
OUTPUT_INVARIANTS = (inv_scale_absorption, inv_window1_flow, inv_rope_base_global_only, inv_branch_norms,
                     inv_zero_projection)
INVARIANTS = OUTPUT_INVARIANTS + (inv_attention_subpath,)


@pytest.mark.parametrize("inv", INVARIANTS, ids=lambda f: f.__name__)
def test_oracle_satisfies_invariant(models, inv):
    assert inv(oracle_runner(), models) == []


# ---- mutants ------------------------------------------------------------------------------------

# name -> [(text in vrt_oracle.c, replacement, expected occurrences)]
MUTANTS = {
    "post_attn_norm_dropped": [("        or_rms_norm_inplace(o, L->post_attn_norm, d, eps);\n", "", 1)],
    "post_ffw_norm_dropped": [("        or_rms_norm_inplace(f, L->post_ffw_norm, d, eps);\n", "", 1)],
    "global_blocks_on_local_rope": [("L->global ? gc : lc", "lc", 2), ("L->global ? gs : ls", "ls", 2)],
    "global_block_index": [("((l + 1u) % 6u) == 0u", "(l % 6u) == 0u", 1)],
    "ffn_norm_is_attn_norm": [("or_rms_norm_into(hidden, L->ffn_norm, xn, d, eps);",
                               "or_rms_norm_into(hidden, L->attn_norm, xn, d, eps);", 1)],
    "gate_up_swapped": [("or_gelu_mul(gate, up, F);", "or_gelu_mul(up, gate, F);", 1),
                        ("L->down, gate, f, F, d, lanes", "L->down, up, f, F, d, lanes", 1)],
    "q_norm_dropped": [("        or_rms_norm_heads(q, L->q_norm, H, hd, eps);\n", "", 1)],
    "k_norm_dropped": [("        or_rms_norm_heads(k, L->k_norm, 1, hd, eps);\n", "", 1)],
    "attn_residual_dropped": [("for (uint32_t i = 0; i < d; ++i) o[i] += hidden[i];", "", 1)],
    "window_on_global_blocks": [("L->cap = (!L->global && m->info.sliding_window)", "L->cap = (m->info.sliding_window)", 1)],
    "embedding_unscaled": [("hidden[i] *= m->emb_scale;", "hidden[i] *= 1.0f;", 1)],
    "attention_scale_one": [("m->attn_scale = 1.0f / sqrtf((float)m->info.head_dim);", "m->attn_scale = 1.0f;", 1)],
    "qk_norm_on_v": [("        or_rms_norm_heads(k, L->k_norm, 1, hd, eps);\n",
                      "        or_rms_norm_heads(k, L->k_norm, 1, hd, eps);\n"
                      "        or_rms_norm_heads(v, L->k_norm, 1, hd, eps);\n", 1)],
    "k_on_local_rope_in_global_blocks": [("or_apply_rope(k, 1, hd, L->global ? gc : lc, L->global ? gs : ls);",
                                          "or_apply_rope(k, 1, hd, lc, ls);", 1)],
}


def _build_mutant(root, name, edits):
    d = os.path.join(root, name)
    os.makedirs(d, exist_ok=True)
    src = open(os.path.join(ORACLE_SRC, "vrt_oracle.c")).read()
    for old, new, count in edits:
        assert src.count(old) == count, f"{name}: '{old}' occurs {src.count(old)} times, expected {count}"
        src = src.replace(old, new)
    with open(os.path.join(d, "vrt_oracle.c"), "w") as fp:
        fp.write(src)
    shutil.copy(os.path.join(ORACLE_SRC, "vrt_oracle.h"), d)
    so = os.path.join(d, "liboracle.so")
    subprocess.run(["gcc", "-O2", "-std=gnu11", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                    "-shared", "-o", so, os.path.join(d, "vrt_oracle.c"), "-lm"], check=True)
    return so


@pytest.fixture(scope="module")
def mutant_libs(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("mutants"))
    with ThreadPoolExecutor(max_workers=4) as ex:
        futs = {n: ex.submit(_build_mutant, root, n, e) for n, e in MUTANTS.items()}
        return {n: f.result() for n, f in futs.items()}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_mutant_fails_an_invariant(models, mutant_libs, name):
    run = oracle_runner(mutant_libs[name])
    failures = []
    for inv in INVARIANTS:
        failures += inv(run, models)
        if failures:
            break
    assert failures, f"mutant {name} passes every wiring invariant"
