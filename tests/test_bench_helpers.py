"""bench.py's measurement helpers on the CPU: the algorithmic bytes of a decode step, the name of
the kernel the roofline is quoted on, and the HBM traffic taken from the committed PMC summaries.

The byte count is checked against the Gemma-3-270M shape's tensor sizes, summed here from
the tensor list (rows x K / 32 Q8_0 blocks of 34 bytes; fp32 norm weights), not from
bench.py's formula.
"""
import importlib.util
import json
import os
from types import SimpleNamespace

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


CFG_270M = SimpleNamespace(embedding_length=640, head_count=4, head_dim=256, feed_forward_length=2048,
                           vocab_size=262144, block_count=18, context_length=32768, sliding_window=512)


def _bytes_270m(pos, kv_bytes):
    q8 = lambda rows, k: rows * (k // 32) * 34
    per_block = {
        "attn_q": q8(1024, 640), "attn_k": q8(256, 640), "attn_v": q8(256, 640),
        "attn_output": q8(640, 1024), "ffn_gate": q8(2048, 640), "ffn_up": q8(2048, 640),
        "ffn_down": q8(640, 2048),
    }
    assert sum(per_block.values()) == 5_918_720
    lm = q8(262144, 640)
    assert lm == 178_257_920
    # attn_norm, attn_q_norm, attn_k_norm, post_attention_norm, ffn_norm, post_ffw_norm per
    # block, then output_norm
    norm_floats = 18 * (640 + 256 + 256 + 640 + 640 + 640) + 640
    assert norm_floats * 4 == 223_744
    emb_row = 680
    # blocks 6, 12 and 18 are global (every history position); the other 15 keep 512
    kv_rows = 15 * min(pos + 1, 512) + 3 * (pos + 1)
    return 18 * 5_918_720 + lm + norm_floats * 4 + emb_row + kv_rows * 256 * kv_bytes * 2


@pytest.mark.parametrize("pos", [0, 8, 27, 511, 512, 4000, 8192])
@pytest.mark.parametrize("kv_bytes", [4, 2])
def test_step_bytes_270m(bench, pos, kv_bytes):
    assert bench.step_bytes(CFG_270M, pos, kv_bytes) == _bytes_270m(pos, kv_bytes)


class _FakeExecutor:
    def __init__(self, available=True, enabled=True, limit=32768, chunked=136):
        self._a, self._e, self._l, self._c = available, enabled, limit, chunked

    def team_available(self):
        return self._a

    def team_enabled(self):
        return self._e

    def team_positions(self):
        return self._l if self._a else 0

    def team_chunked_from(self):
        return self._c


def test_roofline_kernel_names(bench):
    g = _FakeExecutor()
    assert bench.roofline_kernel(g, CFG_270M, 8, 20).startswith("k_team (")
    assert bench.roofline_kernel(g, CFG_270M, 8, 128).startswith("k_team (")       # positions 8..135
    assert bench.roofline_kernel(g, CFG_270M, 8192, 256).startswith("k_team (")    # chunked variant only
    mixed = bench.roofline_kernel(g, CFG_270M, 100, 100)                           # 100..199
    assert mixed.startswith("k_team for positions 100..135, then its chunked-history variant for 136..199")
    # the team kernel switched off (bench.py --no-team) or not built for the shape
    assert bench.roofline_kernel(_FakeExecutor(enabled=False), CFG_270M, 8, 20).startswith("k_decode (")
    assert bench.roofline_kernel(_FakeExecutor(available=False), CFG_270M, 8, 20).startswith("k_decode (")
    # a team kernel limited below the context hands later positions to k_decode
    lim = bench.roofline_kernel(_FakeExecutor(limit=136, chunked=136), CFG_270M, 100, 100)
    assert lim.startswith("k_team for positions 100..135, then k_decode")


@pytest.mark.parametrize("kernel", ["k_team", "k_decode"])
def test_load_traffic_reads_committed_summary(bench, kernel):
    rel = bench.TRAFFIC_SUMMARY[kernel]
    with open(os.path.join(REPO, rel)) as fp:
        summary = json.load(fp)
    assert summary["kernel"] == kernel
    # the summary's bytes are its calibrated counters: FETCH x fetch_scale + WRITE x write_scale
    steps = summary["steps_per_launch"]
    fetch = summary["fetch_kib_per_launch_raw"] * 1024 * summary["fetch_scale"] / steps
    write = summary["write_kib_per_launch_raw"] * 1024 * summary["write_scale"] / steps
    assert abs(fetch + write - summary["hbm_bytes_per_step"]) <= 1e-4 * summary["hbm_bytes_per_step"]
    assert summary["algorithmic_bytes_per_step"] == int(sum(_bytes_270m(8 + i, 4) for i in range(20)) / 20)
    traffic, src = bench.load_traffic(20, kernel)
    assert traffic == int(summary["hbm_bytes_per_step"] * 20)
    assert rel in src
    assert bench.load_traffic(20, "k_other") == (None, None)
