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
    """(path, tokens) -> [(hidden, logits)] per position, or None if the decode raised."""
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


INVARIANTS = (inv_scale_absorption, inv_window1_flow, inv_rope_base_global_only, inv_branch_norms,
              inv_zero_projection)


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
