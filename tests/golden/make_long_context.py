"""Writes tests/golden/long_context_6blk.npz: the oracle on a long history, for the GPU test of
the long-context regime. Model: 6 blocks with the Gemma-3-270M block shape (d 640, 4 x 256 query
heads, FFN 2048, window 512; block 5 global), vocabulary 4096, seed 7. Tokens: 8208 uniform ids
(seed 8) fed one per position; positions 0..8191 fill the cache, and at each of positions
8192..8207 the step's greedy result is recorded, so the global block attends over up to 8208
positions and the local blocks over their 512-slot ring. The oracle needs minutes for the 8208
serial steps, so the GPU test compares against these committed vectors instead of re-running it.

Stored: index[16], value[16] (greedy argmax and its logit at positions 8192..8207),
last_logits[4096] and last_hidden[640] at position 8207.

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
TOKEN_SEED, N_FILL, N_CHECK = 8, 8192, 16
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "long_context_6blk.npz")


def main():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "lc6.gguf")
        synth.write_gemma3_gguf(path, seed=MODEL_SEED, **MODEL)
        toks = synth.uniform_ids(TOKEN_SEED, N_FILL + N_CHECK, 2, MODEL["vocab"])
        m = oracle.Model(path)
        t0 = time.time()
        idx, val = [], []
        for pos, t in enumerate(toks):
            check = pos >= N_FILL
            r = m.decode(int(t), pos, want_logits=check, logits=pos == toks.size - 1)
            if check:
                idx.append(r["index"])
                val.append(r["value"])
            if (pos + 1) % 1024 == 0:
                print(f"[golden] {pos + 1} positions, {time.time() - t0:.0f} s", flush=True)
        m.close()
        np.savez(OUT, index=np.array(idx, np.uint32), value=np.array(val, np.float32),
                 last_logits=r["logits"].astype(np.float32), last_hidden=r["hidden"].astype(np.float32))
        print(f"[golden] wrote {OUT} ({time.time() - t0:.0f} s): greedy ids {idx}")


if __name__ == "__main__":
    main()
