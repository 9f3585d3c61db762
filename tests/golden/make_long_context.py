"""Writes tests/golden/long_context_6blk.npz: the oracle's greedy continuation of a long prompt
on a 6-block model with the Gemma-3-270M block shape (d 640, 4 x 256 query heads, FFN 2048,
window 512; block 5 global), vocabulary 4096, seed 7. The prompt is 8192 uniform ids (seed 8);
16 greedy tokens follow, so the global block attends over up to 8208 positions and the local
ones over their 512-position window. The oracle takes minutes for this (8208 serial steps), so
the GPU test compares against these committed vectors instead of re-running it.

Stored: tokens[16] (greedy ids), values[16] (their logits), last_logits[4096] and
last_hidden[640] at the last generated step (position 8206, fed the 15th greedy token).

Run from the repository root: python tests/golden/make_long_context.py
"""
import os
import sys
import tempfile
import time

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(REPO, "vortex-rt_amd"), os.path.join(REPO, "oracle")]
import oracle  # noqa: E402
import synth  # noqa: E402

MODEL = dict(synth.GEMMA3_270M, n_layers=6, vocab=4096, context=8448)
MODEL_SEED = 7
PROMPT_SEED, N_PROMPT, N_NEW = 8, 8192, 16
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "long_context_6blk.npz")


def main():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "lc6.gguf")
        synth.write_gemma3_gguf(path, seed=MODEL_SEED, **MODEL)
        prompt = synth.uniform_ids(PROMPT_SEED, N_PROMPT, 2, MODEL["vocab"])
        m = oracle.Model(path)
        t0 = time.time()
        pos = 0
        for i, t in enumerate(prompt):
            r = m.decode(int(t), pos, want_logits=(i == N_PROMPT - 1))
            pos += 1
            if pos % 1024 == 0:
                print(f"[golden] {pos} positions, {time.time() - t0:.0f} s", flush=True)
        toks, vals = [r["index"]], [r["value"]]
        for j in range(1, N_NEW):
            last = j == N_NEW - 1
            r = m.decode(toks[-1], pos, want_logits=True, logits=last)
            pos += 1
            toks.append(r["index"])
            vals.append(r["value"])
        m.close()
        np.savez(OUT, tokens=np.array(toks, np.uint32), values=np.array(vals, np.float32),
                 last_logits=r["logits"].astype(np.float32), last_hidden=r["hidden"].astype(np.float32),
                 last_position=np.uint32(pos - 1))
        print(f"[golden] wrote {OUT} ({time.time() - t0:.0f} s): tokens {toks}")


if __name__ == "__main__":
    main()
