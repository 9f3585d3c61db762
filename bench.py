#!/usr/bin/env python3
"""Decode throughput of the Gemma-3-270M-shape Q8_0 batch-1 token loop on one MI355X.

Workload: random-init Gemma-3-270M-architecture model (18 blocks, d 640, 4 query heads and
1 KV head of 256, FFN 2048, vocab 262144 tied Q8_0 LM head, window 512), an 8-token prompt
of uniform ids in [2, 262144) from seed 0, then greedy decode with an fp32 KV cache. One
"step" is one decode_token (all 18 blocks + LM head + argmax) producing one token. The
prompt is prefilled first (untimed); --steps decode steps at positions 8, 9, ... are timed
with hipEvents on the library's stream. Inputs are resident in HBM before timing.

The whole decode loop is one persistent kernel: a cooperative launch with one workgroup per CU
that runs every block, the LM head and argmax for each of the launch's steps. At this shape every
position runs on k_team (four teams of workgroups, each running one phase type of every block):
its on-chip variant while a head's history fits in a workgroup (136 positions with fp32 KV: 64
in registers and 72 in LDS), its chunked variant after that. With the default 8-token prompt and
up to 128 steps the timed region is exactly one k_team launch, so the roofline's launch duration
is the event-timed region itself; longer runs time two launches together.

Algorithmic bytes per step at position p: every Q8_0 weight byte, the fp32 norm weights, one
embedding row, plus the fp32 KV rows attention reads (min(p+1, window) positions for local
blocks, p+1 for global ones), each counted once.

The line also carries the long-context legs (an 8192-token prompt, then 256 timed steps) with
fp32, fp16 and bf16 KV entries, the 512- and 8192-token prefills, batched decode at 1-64
sequences, the standalone kernels and the oracle's CPU rate; --no-* switches each one off and
--only runs a single leg.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
for sub in ("vortex-rt_amd", "oracle"):
    sys.path.insert(0, os.path.join(REPO, sub))

HBM_PEAK_GBPS = 8000.0
METRIC = "decode tokens/s + achieved HBM GB/s (% of roofline), Gemma3-270M-shape Q8_0, 1 GPU"


def step_bytes(cfg, pos: int, kv_bytes: int = 4) -> int:
    d, H, hd, F, V, L = (cfg.embedding_length, cfg.head_count, cfg.head_dim, cfg.feed_forward_length,
                         cfg.vocab_size, cfg.block_count)
    q8 = lambda rows, k: rows * (k // 32) * 34
    layer = q8(H * hd, d) + 2 * q8(hd, d) + q8(d, H * hd) + 2 * q8(F, d) + q8(d, F)
    norms = (L * (4 * d + 2 * hd) + d) * 4
    total = L * layer + q8(V, d) + norms + (d // 32) * 34
    for l in range(L):
        glob = (l + 1) % 6 == 0
        slots = cfg.context_length if (glob or cfg.sliding_window == 0) else cfg.sliding_window
        total += min(pos + 1, slots) * hd * kv_bytes * 2
    return total


# rocprofv3 PMC summaries of the timed dispatch per persistent kernel
TRAFFIC_SUMMARY = {"k_team": os.path.join("profiles", "decode_team_gemma3_270m_pmc.json"),
                   "k_decode": os.path.join("profiles", "decode_gemma3_270m_pmc.json")}


def load_traffic(steps: int, kernel: str):
    """HBM bytes per launch of `steps` steps of `kernel` and where the figure comes from: the
    committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE per decode step, calibrated against
    a copy of known size), scaled to `steps`. This run does not measure it."""
    rel = TRAFFIC_SUMMARY.get(kernel)
    if rel is None:
        return None, None
    p = os.path.join(REPO, rel)
    try:
        with open(p) as fp:
            summary = json.load(fp)
        per_step = summary["hbm_bytes_per_step"]
    except (OSError, ValueError, KeyError):
        return None, None
    src = (f"{rel}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of {kernel}, calibrated, "
           f"{per_step / 1e6:.1f} MB per step, scaled to {steps} steps (not measured by this run)")
    if "command" in summary:
        src += f"; command: {summary['command']}"
    return int(per_step * steps), src


def phase_split(g, prompt, cfg, steps: int = 24):
    """Per-phase time of one decode step from the kernel's own clock marks (s_memrealtime, 100 MHz),
    median over blocks 1..L-1. The traced step is position len(prompt), the first of its launch.

    Team kernel (positions below its limit): a phase ends when the last workgroup of its team has
    published; each phase is timed from the previous phase's end (so it includes its hand-off):
    A q|k|v, B attention + O, D norms + gate/up + GELU, E down. All-workgroup kernel: phases A..E
    as that kernel runs them, each phase's end being the latest workgroup's end timestamp."""
    g.set_trace(True)
    g.start(prompt, steps + 1)
    g.step(len(prompt))
    g.step(steps)            # the traced step is the first of this launch
    tr = g.read_trace().astype(np.int64)
    g.collect()
    g.set_trace(False)
    L = cfg.block_count
    nwg, slots = tr.shape
    out = {}
    if slots == 2 * L + 3 + 8:   # team kernel: workgroup w in team (w % 8) // 2
        team = (np.arange(nwg) % 8) // 2
        pub = np.array([[tr[team == t, L + l].max() for l in range(L)] for t in range(4)]) / 100.0   # us
        ends = [pub[t, l] for l in range(L) for t in range(4)]          # A0 B0 D0 E0 A1 ...
        for t, p in enumerate("ABDE"):
            out[p] = float(np.median([ends[4 * l + t] - ends[4 * l + t - 1] for l in range(1, L)]))
        out["lm_head"] = float(tr[:, 2 * L + 2].max() / 100.0 - pub[3, L - 1])
        out["step"] = float((tr[:, 2 * L + 2].max() - tr[:, 2 * L][tr[:, 2 * L] > 0].min()) / 100.0)
        out["kernel"] = "k_team"
        return {k: (round(v, 2) if isinstance(v, float) else v) for k, v in out.items()}
    mx = tr[:, : 5 * L + 3].max(axis=0) * 10.0 / 1000.0        # us
    for k, p in enumerate("ABCDE"):
        out[p] = float(np.median([mx[1 + 5 * l + k] - mx[5 * l + k] for l in range(1, L)]))
    out["lm_head"] = float(mx[5 * L + 2] - mx[5 * L + 1])
    out["step"] = float(mx[5 * L + 2] - mx[0])
    out["kernel"] = "k_decode"
    return {k: (round(v, 2) if isinstance(v, float) else v) for k, v in out.items()}


def long_context(ctx, g, cfg, n_prompt: int = 8192, steps: int = 256, kv: str = "f32"):
    """The long-context workload: an n_prompt-token prompt of uniform ids (seed 1) prefilled
    untimed, then `steps` greedy decode steps timed with events (positions n_prompt..). kv is
    the KV cache's entry type: "f32", or "f16" / "bf16" (2 bytes per element)."""
    if kv != "f32":
        g.set_kv_format(kv)
        try:
            return long_context(ctx, g, cfg, n_prompt, steps)
        finally:
            g.set_kv_format("f32")
    prompt = synth_ids(1, n_prompt, cfg.vocab_size)
    g.start(prompt, steps + 1)
    g.step(n_prompt)
    ctx.sync()
    ev0, ev1 = ctx.event(), ctx.event()
    ctx.record(ev0)
    g.step(steps)
    ctx.record(ev1)
    ms = ctx.elapsed_ms(ev0, ev1)
    ctx.sync()
    toks = g.collect()
    if toks.size < steps + 1:
        raise SystemExit(f"[bench] long context: EOS after {toks.size} generated tokens; the timed steps did not all run")
    kvb = 4 if g.kv_format() == "f32" else 2
    total = sum(step_bytes(cfg, n_prompt + i, kvb) for i in range(steps))
    gbps = total / (ms / 1e3) / 1e9
    return {"workload": f"{n_prompt}-token prompt (untimed prefill), {steps} timed greedy decode steps at positions "
                        f"{n_prompt}..{n_prompt + steps - 1}",
            "tokens_per_s": round(steps / (ms / 1e3), 2), "ms_per_step": round(ms / steps, 5),
            "bytes_per_step_mean": int(total / steps), "hbm_gbps": round(gbps, 1),
            "roofline_frac": round(gbps / HBM_PEAK_GBPS, 4)}


def prefill_flops(cfg, T: int) -> int:
    """Algorithmic FLOPs of a T-token prefill: every projection as a GEMM over T rows, causal
    attention (QK and PV over the keys each position sees), and the last row's LM head."""
    d, H, hd, F, V, L = (cfg.embedding_length, cfg.head_count, cfg.head_dim, cfg.feed_forward_length,
                         cfg.vocab_size, cfg.block_count)
    params = (H * hd + 2 * hd) * d + d * H * hd + 2 * F * d + d * F
    total = 2 * T * params * L + 2 * V * d
    for l in range(L):
        glob = (l + 1) % 6 == 0
        w = T if (glob or cfg.sliding_window == 0) else cfg.sliding_window
        keys = sum(min(t + 1, w) for t in range(T))
        total += 2 * 2 * H * hd * keys
    return total


MFMA_F16_PEAK_TFLOPS = 2500.0
PREFILL_SEGMENT = 2048   # positions per batched prefill pass (longer prompts run as segments)


def prefill_bench(ctx, g, cfg, T: int = 512, reps: int = 5):
    """The batched prefill workload: T uniform prompt ids (seed 4) in one vrt_g3_prefill call,
    timed with events over `reps` calls after a warm-up call."""
    prompt = synth_ids(4, T, cfg.vocab_size)
    g.prefill(prompt, top_k=1)
    ctx.sync()
    ev0, ev1 = ctx.event(), ctx.event()
    ctx.record(ev0)
    for _ in range(reps):
        g.prefill(prompt, top_k=1)
    ctx.record(ev1)
    ctx.sync()
    ms = ctx.elapsed_ms(ev0, ev1) / reps
    flops = prefill_flops(cfg, T)
    tflops = flops / (ms / 1e3) / 1e12
    seg = f", in segments of {PREFILL_SEGMENT}" if T > PREFILL_SEGMENT else ""
    return {"workload": f"{T}-token prompt, one batched prefill{seg} (MFMA Q8_0 GEMMs, causal attention, last-row LM head)",
            "tokens_per_s": round(T / (ms / 1e3), 1), "ms": round(ms, 4), "gflop": round(flops / 1e9, 2),
            "tflops": round(tflops, 2), "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
            "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "note": "projection GEMMs issue two f16 MFMAs per product (activation hi + lo parts); utilisation "
                    "counts the algorithmic FLOPs only"}


def q8_bytes(rows: int, k: int) -> int:
    return rows * (k // 32) * 34


def kernel_legs(ctx, iters: int = 200):
    """The standalone entry points on their workloads: one Q8_0 matvec at 2048 x 640 and at
    640 x 2048 (W ~ N(0, 0.02), seed 0, x ~ N(0, 1)), and the decoder-layer projection block
    (fused Q/K/V triplet 1024 + 256 + 256 rows x 640; fused FFN 2048 x 640 gate/up with the GELU
    product, 640 x 2048 down). Each is launched `iters` times back to back between two events on
    the library's stream; bytes are the weights plus fp32 inputs and outputs, once per call."""
    import synth
    import vrt
    out = {}

    def timed(fn, nbytes):
        fn()
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(iters):
            fn()
        ctx.record(e1)
        ms = ctx.elapsed_ms(e0, e1)
        us = ms * 1e3 / iters
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"us_per_call": round(us, 3), "bytes": nbytes, "gbps": round(gbps, 1),
                "roofline_frac": round(gbps / HBM_PEAK_GBPS, 4)}

    for rows, k in ((2048, 640), (640, 2048)):
        w = synth.q8_matrix(0, f"bench.w{rows}x{k}", rows, k)
        wd = ctx.upload(w)
        xd = ctx.upload(synth.normal_f32(1, k))
        yd = ctx.alloc(rows * 4)
        out[f"matvec_{rows}x{k}"] = timed(lambda: vrt.q8_matvec(ctx, wd, 0, xd, yd, k, rows),
                                          q8_bytes(rows, k) + 4 * (k + rows))
    d, qw, hd, F = 640, 1024, 256, 2048
    mats = [synth.q8_matrix(0, f"bench.{n}", r, c) for n, r, c in
            (("q", qw, d), ("k", hd, d), ("v", hd, d), ("gate", F, d), ("up", F, d), ("down", d, F))]
    offs = np.cumsum([0] + [m.size for m in mats])
    wd = ctx.upload(np.concatenate(mats))
    xd = ctx.upload(synth.normal_f32(2, d))
    yq = ctx.alloc((qw + 2 * hd) * 4)
    ws = ctx.alloc(2 * F * 4)
    yf = ctx.alloc(d * 4)
    out["qkv_triplet_640"] = timed(lambda: vrt.q8_matvec_multi(ctx, wd, offs[:3], (qw, hd, hd), d, xd, yq),
                                   q8_bytes(qw + 2 * hd, d) + 4 * (d + qw + 2 * hd))
    out["ffn_640_2048"] = timed(lambda: vrt.q8_ffn(ctx, wd, int(offs[3]), int(offs[4]), int(offs[5]), d, F, d, xd, ws, yf),
                                2 * q8_bytes(F, d) + q8_bytes(d, F) + 4 * (2 * d))
    out["note"] = (f"{iters} back-to-back calls between two events (launch gaps included); the FFN is two "
                   "launches (gate/up with the GELU product, then down)")
    return out


def synth_ids(seed: int, n: int, vocab: int):
    import synth
    return synth.uniform_ids(seed, n, 2, vocab)


def multikernel_leg(ctx, g, prompt, steps: int = 64):
    """The multi-kernel decode path (a hipGraph per step: five kernels per block, the attention
    merge and the LM head with its final reduction), timed over `steps` steps after the prompt."""
    g.set_persistent(False)
    g.set_graph(True)
    try:
        g.start(prompt, steps + 5)
        g.step(prompt.size + 4)
        ctx.sync()
        ev0, ev1 = ctx.event(), ctx.event()
        ctx.record(ev0)
        g.step(steps)
        ctx.record(ev1)
        ms = ctx.elapsed_ms(ev0, ev1)
        ctx.sync()
        if g.collect().size < steps + 5:
            raise SystemExit("[bench] EOS inside the multi-kernel timed steps; no throughput is reported")
    finally:
        g.set_persistent(True)
    return {"workload": f"{prompt.size}-token prompt + 4 steps, then {steps} timed decode steps (hipGraph per step)",
            "us_per_step": round(ms * 1e3 / steps, 1), "tokens_per_s": round(steps / (ms / 1e3), 1)}


def batched_leg(ctx, g, cfg, sizes=(1, 8, 32, 64), n_prompt: int = 8, steps: int = 16):
    """Batched greedy decode (vrt_g3_batch_step): B sequences with their own 8-token prompts advance
    together, one position per step; after the prompts, `steps` timed steps in which every
    sequence feeds back its greedy token. Each step includes its host round trip (upload of the
    step's rows, results back), as a serving loop would see it."""
    import vrt
    out = {"workload": f"B independent sequences: {n_prompt}-token prompts fed one per step, then {steps} timed "
                       f"steps of B greedy tokens (positions {n_prompt}..{n_prompt + steps - 1})", "batches": {}}
    for B in sizes:
        b = vrt.Gemma3Batch(g, B, n_prompt + steps + 8)
        try:
            prompts = [synth_ids(1000 + i, n_prompt, cfg.vocab_size) for i in range(B)]
            seqs = list(range(B))
            idx = None
            for k in range(n_prompt):
                idx, _ = b.step(seqs, [int(p[k]) for p in prompts])
            t0 = time.perf_counter()
            for _ in range(steps):
                idx, _ = b.step(seqs, [int(t) for t in idx])
            dt = time.perf_counter() - t0
        finally:
            b.close()
        out["batches"][str(B)] = {"ms_per_step": round(dt * 1e3 / steps, 3),
                                  "tokens_per_s": round(B * steps / dt, 1)}
    return out


def copy_calibration(nbytes: int = 1 << 30):
    """A plain device copy of known size for scaling the PMC counters (FETCH_SIZE / WRITE_SIZE
    of this dispatch against nbytes read and nbytes written)."""
    import torch
    a = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes}))


def cpu_baseline(path, prompt, target_s: float = 12.0):
    """The oracle (scalar C, OpenMP over matvec rows) timed on this host: prompt steps without
    the LM head, then greedy decode steps (each with the LM head) until ~target_s of work."""
    import oracle
    m = oracle.Model(path)
    pos = 0
    for i, t in enumerate(prompt):
        r = m.decode(int(t), pos, want_logits=(i == len(prompt) - 1))
        pos += 1
    tok = r["index"]
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        r = m.decode(int(tok), pos, want_logits=True)
        times.append(time.perf_counter() - t0)
        tok = r["index"]
        pos += 1
        if time.perf_counter() - t_all > target_s or len(times) >= 64:
            break
    m.close()
    n = len(times)
    return {"value": n / sum(times), "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": f"{n} greedy decode steps at positions {len(prompt)}..{len(prompt) + n - 1} of the same "
                      f"model and prompt (oracle/vrt_oracle.c, {oracle.num_threads()} OpenMP threads); "
                      f"the reference's Lavapipe path is not available on this host"}


def roofline_kernel(g, cfg, first: int, steps: int) -> str:
    """The persistent launch(es) that run the timed steps at positions first .. first + steps - 1
    (steps below g.team_positions() run on the team kernel, VRT_G3_OPT_QUERY_TEAM_POSITIONS)."""
    per = f"{cfg.block_count} blocks + tied LM head + argmax per step"
    last = first + steps - 1
    limit = g.team_positions() if g.team_available() and g.team_enabled() else 0
    chunked = min(g.team_chunked_from(), limit) if limit else 0
    if last < limit and (last < chunked or first >= chunked):
        return f"k_team (phase-team persistent kernel: {per}, {steps} steps per launch)"
    if last < limit:
        return (f"k_team for positions {first}..{chunked - 1}, then its chunked-history variant for "
                f"{chunked}..{last}: {per}")
    if first < limit:
        return (f"k_team for positions {first}..{limit - 1}, then k_decode (all-workgroup persistent "
                f"kernel) for {limit}..{last}: {per}")
    return f"k_decode (all-workgroup persistent kernel: {per}, {steps} steps per launch)"


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-phases", action="store_true", help="skip the traced per-phase split")
    ap.add_argument("--no-long", action="store_true", help="skip the 8192-token long-context measurement")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the 512- and 8192-token batched prefill measurements")
    ap.add_argument("--no-kernels", action="store_true",
                    help="skip the standalone matvec / QKV / FFN measurements (single-matvec and layer-block workloads)")
    ap.add_argument("--multikernel", action="store_true",
                    help="also time the multi-kernel (hipGraph) decode path")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched-decode (B sequences) measurement")
    ap.add_argument("--no-team", action="store_true",
                    help="decode on the all-workgroup persistent kernel k_decode (the team kernel switched off)")
    ap.add_argument("--only", choices=("prefill", "prefill_8192", "batched", "kernels", "long_context"),
                    help="run only this leg and print it (for profiling one leg at a time; all but "
                         "long_context make no cooperative launch)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (the PMC calibration dispatch) and exit")
    ap.add_argument("--model", default=os.environ.get("VRT_BENCH_MODEL", "/tmp/vrt_bench/gemma3_270m_q8_seed0.gguf"))
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py: this framework runs on one GPU; --gpus {args.gpus} is not supported "
              "(the batch-1 token loop is single-GPU)", file=sys.stderr)
        sys.exit(2)

    import synth
    import vrt

    if not os.path.exists(args.model):
        os.makedirs(os.path.dirname(args.model), exist_ok=True)
        t0 = time.time()
        synth.write_gemma3_gguf(args.model, seed=0, **synth.GEMMA3_270M)
        print(f"[bench] wrote {args.model} in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    ctx = vrt.Context("")
    g = vrt.Gemma3(ctx, args.model)
    cfg = g.config
    if args.no_team:
        g.set_team(False)
    if args.only:
        legs = {"prefill": lambda: prefill_bench(ctx, g, cfg),
                "prefill_8192": lambda: prefill_bench(ctx, g, cfg, T=8192, reps=3),
                "batched": lambda: batched_leg(ctx, g, cfg),
                "kernels": lambda: kernel_legs(ctx),
                "long_context": lambda: long_context(ctx, g, cfg)}
        res = legs[args.only]()
        g.close()
        ctx.close()
        print(json.dumps({"only": args.only, args.only: res}))
        return
    if not g.persistent_available():
        raise SystemExit("[bench] the persistent decode kernel is unavailable for this shape/device")
    prompt = synth.uniform_ids(0, 8, 2, cfg.vocab_size)
    n_prompt = prompt.size
    print(f"[bench] device {ctx.info.name.decode()} ({ctx.info.arch.decode()}, {ctx.info.compute_units} CUs)",
          file=sys.stderr, flush=True)

    # warm-up: a full generation of `warmup` decode steps (graph capture happens here)
    warm = g.generate(prompt, args.warmup + 1)

    # timed: prefill untimed, then exactly `steps` decode steps between two events
    g.start(prompt, args.steps + 1)
    g.step(n_prompt)
    ctx.sync()
    ev0, ev1 = ctx.event(), ctx.event()
    ctx.sync()
    ctx.record(ev0)
    g.step(args.steps)
    ctx.record(ev1)
    ms = ctx.elapsed_ms(ev0, ev1)
    ctx.sync()
    toks = g.collect()
    if toks.size < args.steps + 1:
        # the kernel stopped at EOS: fewer than --steps steps ran inside the timed region
        raise SystemExit(f"[bench] EOS after {toks.size} generated tokens: only {max(toks.size - 1, 0)} of the "
                         f"{args.steps} timed decode steps ran; no throughput is reported")
    k = min(warm.size, toks.size)
    if not np.array_equal(warm[:k], toks[:k]):
        raise SystemExit("[bench] nondeterministic greedy tokens between warm-up and timed run")

    ms_per_step = ms / args.steps
    tok_s = args.steps / (ms / 1e3)
    total_bytes = sum(step_bytes(cfg, n_prompt + i) for i in range(args.steps))
    gbps = total_bytes / (ms / 1e3) / 1e9

    rkernel = roofline_kernel(g, cfg, n_prompt, args.steps)
    single = rkernel.split(" ")[0] if "then" not in rkernel else None
    traffic, traffic_src = load_traffic(args.steps, single) if single else (None, None)
    phases = None if args.no_phases else phase_split(g, prompt, cfg)
    longctx = None if args.no_long else long_context(ctx, g, cfg)
    longctx16 = None if args.no_long else long_context(ctx, g, cfg, kv="f16")
    longctxbf16 = None if args.no_long else long_context(ctx, g, cfg, kv="bf16")
    prefill = None if args.no_prefill else prefill_bench(ctx, g, cfg)
    prefill_long = None if args.no_prefill else prefill_bench(ctx, g, cfg, T=8192, reps=3)
    kernels = None if args.no_kernels else kernel_legs(ctx)
    multikernel = multikernel_leg(ctx, g, prompt) if args.multikernel else None
    batched = None if args.no_batched else batched_leg(ctx, g, cfg)

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights x fp32 activations (int8 dot4 on 3 int8 activation limbs), fp32 KV",
        "data": "synthetic (random-init weights N(0,0.02) quantised to Q8_0, seed 0)",
        "config": {
            "workload": f"Gemma-3-270M-shape Q8_0 batch-1 greedy decode: {n_prompt}-token prompt (untimed prefill), "
                        f"{args.steps} timed decode steps at positions {n_prompt}..{n_prompt + args.steps - 1}",
            "layers": cfg.block_count, "d_model": cfg.embedding_length, "heads": cfg.head_count,
            "kv_heads": cfg.head_count_kv, "head_dim": cfg.head_dim, "ffn": cfg.feed_forward_length,
            "vocab": cfg.vocab_size, "sliding_window": cfg.sliding_window, "batch": 1,
            "parallelism": "single GPU",
        },
        "hbm_gbps": round(gbps, 1),
        "bytes_per_step_mean": int(total_bytes / args.steps),
        "roofline": {
            "kernel": rkernel,
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "mean_launch_us": round(ms * 1e3, 1),
            "algorithmic_bytes_per_launch": total_bytes,
        },
        "phase_us_per_step": phases,
        "long_context": longctx,
        "long_context_kv_f16": longctx16,
        "long_context_kv_bf16": longctxbf16,
        "prefill": prefill,
        "prefill_8192": prefill_long,
        "kernels": kernels,
        "multikernel": multikernel,
        "batched": batched,
        "cpu_baseline": None,
    }
    g.close()
    ctx.close()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.model, prompt)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
