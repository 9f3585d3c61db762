"""The block-wiring invariants of test_oracle_wiring.py (power-of-two scale absorption with
eps = 0, information flow through global blocks only at window 1, rope.freq_base reaching only
global blocks, branch norms that cannot matter, the zero-projection closed form) run through the
HIP executor itself, on the persistent decode kernel and on the multi-kernel step. They hold bit
for bit on the device as on the CPU: every scaling involved is by an exact power of two, and the
device's activation limbs and fp32 sums scale exactly with it."""
import numpy as np
import pytest

import vrt
from test_oracle_wiring import OUTPUT_INVARIANTS, models  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def gpu_runner(ctx, persistent):
    def run(path, toks):
        g = vrt.Gemma3(ctx, path)
        try:
            if persistent and not g.persistent_available():
                raise AssertionError("persistent decode kernel unavailable for the wiring model")
            g.set_persistent(persistent)
            out = []
            for i, t in enumerate(toks):
                _, hid = g.decode(int(t), i, top_k=8, hidden=True)
                out.append((hid, g.logits()))
            return out
        except vrt.VrtError:
            return None
        finally:
            g.close()
    return run


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "multikernel"])
@pytest.mark.parametrize("inv", OUTPUT_INVARIANTS, ids=lambda f: f.__name__)
def test_hip_path_satisfies_invariant(ctx, models, inv, persistent):  # noqa: F811
    print(f"[wiring] {inv.__name__} persistent={persistent}", flush=True)
    assert inv(gpu_runner(ctx, persistent), models) == []
