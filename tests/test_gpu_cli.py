"""vortexrt-gemma (the command line of src/gemma_main.cpp on the HIP build) on the GPU: the
report lines the reference's CI greps (.github/workflows/build.yml:81-123), checked against the
oracle: the forward pass of one token (final hidden checksum, top logits) and prompted greedy
generation (prompt ids from the oracle tokenizer, generated ids from the oracle's loop)."""
import os
import re
import subprocess

import numpy as np
import pytest

import gguf
import oracle
from tokenizer import Tokenizer

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(REPO, "vortex-rt_amd", "_build", "vortexrt-gemma")


def _cli(*args, rc=0):
    assert os.path.exists(CLI), f"{CLI} not built (vortex-rt_amd/build.py)"
    print(f"[gpu] vortexrt-gemma {' '.join(map(str, args))}", flush=True)
    r = subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=120)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == rc, r.stderr
    return r.stdout, r.stderr


def _oracle_tokenizer(path):
    f = gguf.GgufFile.open(path)
    arr = lambda k: list(f.metadata[k][1][1])
    tok = Tokenizer(arr("tokenizer.ggml.tokens"), arr("tokenizer.ggml.scores"), arr("tokenizer.ggml.token_type"),
                    bos=f.meta_u64("tokenizer.ggml.bos_token_id"), eos=f.meta_u64("tokenizer.ggml.eos_token_id"),
                    unk=f.meta_u64("tokenizer.ggml.unknown_token_id"))
    f.close()
    return tok


def test_cli_forward_report(tiny_model):
    out, _ = _cli(tiny_model, "--token-id", 2, "--top-k", 8)
    for line in ("Vortex-RT Gemma 3 runtime", "Layers: 6", "Hidden: 128", "Heads: 2 / KV 1", "Sliding window: 8",
                 "Vocab: 1000", "Token: 2", "Top logits:", "Validation: OK"):
        assert line in out, line
    m = oracle.Model(tiny_model)
    r = m.decode(2, 0, want_logits=True, logits=True)
    m.close()
    hidden, logits = r["hidden"], r["logits"]
    checksum = float(np.sum(hidden.astype(np.float64) * np.arange(1, hidden.size + 1)))
    got = float(re.search(r"Final hidden checksum: (\S+)", out).group(1))
    # hidden within 1e-4 of max|hidden| per element bounds the checksum difference
    bound = 1e-4 * float(np.max(np.abs(hidden))) * hidden.size * (hidden.size + 1) / 2
    assert abs(got - checksum) <= bound
    tops = re.findall(r"(\d+): id=(\d+) logit=(\S+) piece=\"", out)
    assert [int(t[0]) for t in tops] == list(range(1, 9))
    ids = [int(t[1]) for t in tops]
    assert ids[0] == int(r["index"])
    vals = np.array([float(t[2]) for t in tops])
    assert np.max(np.abs(vals - logits[ids])) <= 1e-3 * np.max(np.abs(logits))
    assert np.all(np.diff(vals) <= 0)


def test_cli_prompted_generation(tiny_model):
    prompt = "t300 t417  t999 x"
    out, _ = _cli(tiny_model, "--prompt", prompt, "--generate", 6)
    tok = _oracle_tokenizer(tiny_model)
    want_prompt = tok.tokenize(prompt, True)
    got_prompt = [int(x) for x in re.search(r"Prompt token ids:((?: \d+)*)\n", out).group(1).split()]
    assert got_prompt == want_prompt
    m = oracle.Model(tiny_model)
    want = m.generate(np.array(want_prompt, np.uint32), 6).tolist()
    m.close()
    got = [int(x) for x in re.search(r"Generated token ids:((?: \d+)*)\n", out).group(1).split()]
    assert got == want
    text = b"".join(tok.decode_piece(t) for t in want if t != tok.eos).decode("utf-8", "replace")
    body = re.search(r"TEXT_BEGIN\n(.*)\nTEXT_END\n", out, re.S).group(1)
    assert body == text
    assert "Validation: OK" in out


def test_cli_generation_from_bos_and_errors(tiny_model, tmp_path):
    out, _ = _cli(tiny_model, "--generate", 3)
    assert "Prompt token ids: 2\n" in out and "TEXT_BEGIN" in out and "Validation: OK" in out
    _, err = _cli(tiny_model, "--generate", 129, rc=1)
    assert "capped at 128" in err
    _, err = _cli(str(tmp_path / "missing.gguf"), rc=1)
    assert err.startswith("vortexrt-gemma: ")
    _, err = _cli(tiny_model, "--q8-lanes", 12, rc=1)
    assert "--q8-lanes" in err


@pytest.mark.parametrize("lanes,fusion", [(64, "off"), (32, "off"), (16, "off"), (8, "off"), (8, "on")])
def test_cli_lane_fusion_loop(tiny_model, lanes, fusion):
    """The reference CI's lane x fusion loop (.github/workflows/build.yml:105-123): every lane
    width with projection fusion off, then 8 lanes with it on. The report states the policy that
    ran, and the generated ids are the oracle's."""
    out, _ = _cli(tiny_model, "--q8-lanes", lanes, "--projection-fusion", fusion, "--generate", 4)
    assert "Validation: OK" in out
    on = fusion == "on"
    assert f"Narrow Q8 kernel: {lanes} lanes" in out        # 4 blocks per row: every width is instantiated
    assert f"Projection fusion: {'enabled' if on else 'disabled'}" in out
    assert f"Fused FFN: {'enabled' if on else 'disabled'}" in out
    m = oracle.Model(tiny_model)
    want = m.generate(np.array([2], np.uint32), 4).tolist()
    m.close()
    got = [int(x) for x in re.search(r"Generated token ids:((?: \d+)*)\n", out).group(1).split()]
    assert got == want
