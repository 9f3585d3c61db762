"""Shared pytest setup: import paths, the `gpu` marker, GPU context and synthetic models."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("vortex-rt_amd", "oracle"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvrt_hip.so)")


@pytest.fixture(scope="session")
def ctx():
    import vrt
    c = vrt.Context("")
    print(f"[gpu] device {c.info.name.decode()} {c.info.arch.decode()} CUs={c.info.compute_units}", flush=True)
    yield c
    c.close()


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


def _tiny(model_dir, name, **kw):
    import synth
    path = os.path.join(str(model_dir), name)
    if not os.path.exists(path):
        synth.write_gemma3_gguf(path, **kw)
    return path


@pytest.fixture(scope="session")
def tiny_model(model_dir):
    """6 blocks (one global), d=128, 2 heads x 64, ffn 256, vocab 1000, window 8."""
    import synth
    return _tiny(model_dir, "tiny.gguf", seed=11, **synth.TINY)


@pytest.fixture(scope="session")
def tiny_model_nowindow(model_dir):
    import synth
    kw = dict(synth.TINY)
    return _tiny(model_dir, "tiny_nowin.gguf", seed=12, with_window=False, **kw)


@pytest.fixture(scope="session")
def full_model(model_dir):
    """Gemma-3-270M shape: 18 blocks, d 640, 4 heads x 256, FFN 2048, vocab 262144, seed 0."""
    import synth
    path = os.path.join(str(model_dir), "gemma3_270m_seed0.gguf")
    if not os.path.exists(path):
        print("[g3] writing Gemma-3-270M-shape model", flush=True)
        synth.write_gemma3_gguf(path, seed=0, **synth.GEMMA3_270M)
    return path
