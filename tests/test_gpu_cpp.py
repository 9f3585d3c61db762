"""The vortexrt:: C++ surface (libvortexrt.so over libvrt_hip.so) on the GPU: the C++ test
programs of tests/cpp, which restate the reference's own test mains, and Gemma3Model against
the oracle."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "_build")


def _run(name, *args, timeout=120):
    exe = os.path.join(BIN, name)
    assert os.path.exists(exe), f"{exe} not built (vortex-rt_amd/build.py)"
    print(f"[gpu] {name} {' '.join(map(str, args))}", flush=True)
    r = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"{name} exited {r.returncode}"
    return r.stdout


def test_cpp_q8_matvec():
    assert "q8_matvec_test ok" in _run("q8_matvec_test")


def test_cpp_ffn():
    assert "ffn_test ok" in _run("ffn_test")


def test_cpp_gemma3_model(tiny_model):
    prompt = [2, 17, 301, 5]
    got = json.loads(_run("gemma3_test", tiny_model, 10, *prompt).strip().splitlines()[-1])
    m = oracle.Model(tiny_model)
    ref = m.generate(np.array(prompt, np.uint32), 10)
    assert got["generate"] == ref.tolist()
    m.reset()
    for i, t in enumerate(prompt):
        r = m.decode(t, i, want_logits=i == len(prompt) - 1, logits=i == len(prompt) - 1)
    logits, hidden = r["logits"], r["hidden"]
    scale = np.max(np.abs(logits))
    top = np.argsort(-logits, kind="stable")[:4]
    ids = [t[0] for t in got["top4"]]
    vals = np.array([t[1] for t in got["top4"]])
    assert ids[0] == int(top[0])
    assert np.max(np.abs(vals - logits[ids])) <= 1e-3 * scale
    assert np.max(np.abs(np.array(got["hidden"]) - hidden)) <= 1e-4 * np.max(np.abs(hidden))
    m.reset()
    r0 = m.decode(prompt[0], 0, want_logits=True)
    assert got["single"][0] == r0["index"]
    assert got["errors"] == [1, 1, 1, 1]
    m.close()
