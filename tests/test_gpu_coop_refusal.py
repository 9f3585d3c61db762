"""A second process decoding on a GPU where this process has already made a cooperative launch:
the device refuses the second process's cooperative launch (hipErrorIllegalState on this ROCm
stack), and its executor continues on the multi-kernel path with the same tokens."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import synth
import vrt

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import json, sys
sys.path[:0] = [sys.argv[1] + "/vortex-rt_amd", sys.argv[1] + "/oracle"]
import numpy as np, vrt
ctx = vrt.Context("")
g = vrt.Gemma3(ctx, sys.argv[2])
toks = g.generate(np.array(json.loads(sys.argv[3]), np.uint32), 12)
persistent = vrt.lib().vrt_g3_set_option(g.h, vrt.OPT_QUERY_PERSISTENT, 0) == vrt.VRT_OK
print(json.dumps({"tokens": [int(t) for t in toks], "persistent": persistent}))
g.close(); ctx.close()
"""


def test_second_process_decodes_after_refused_cooperative_launch(ctx, tiny_model):
    prompt = synth.uniform_ids(900, 5, 2, 1000)
    g = vrt.Gemma3(ctx, tiny_model)
    try:
        assert g.persistent_available()
        mine = g.generate(prompt, 12)   # a cooperative launch in this (still live) process
        print("[coop] child process decoding", flush=True)
        r = subprocess.run([sys.executable, "-c", CHILD, REPO, tiny_model, json.dumps([int(t) for t in prompt])],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        out = json.loads(r.stdout.strip().splitlines()[-1])
        print(f"[coop] child persistent path: {out['persistent']}", flush=True)
        np.testing.assert_array_equal(np.array(out["tokens"], np.uint32), mine)
    finally:
        g.close()
