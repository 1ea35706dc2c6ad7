import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "llm-inference-engine_amd"
for p in (str(ROOT), str(PKG / "python")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def golden():
    from safetensors.numpy import load_file
    return load_file(str(ROOT / "tests" / "golden" / "hf_attention.safetensors"))


@pytest.fixture(scope="session")
def ehip_mod():
    import ehip
    ehip.lib()
    return ehip


@pytest.fixture(scope="session")
def gctx(ehip_mod):
    """One HIP context for the whole GPU session (fails loudly without a GPU:
    there is no CPU fallback behind the GPU tests)."""
    ctx = ehip_mod.Context(0)
    yield ctx
    ctx.close()


@pytest.fixture
def tctx(ehip_mod, monkeypatch):
    """A context reads the EHIP_* tuning switches once, when it is created.
    tctx(NAME=value, ...) sets switches (undone after the test) and returns a
    new context that carries them; every context made is closed at teardown."""
    made = []

    def make(**env):
        for k, v in env.items():
            monkeypatch.setenv(k, str(v))
        ctx = ehip_mod.Context(0)
        made.append(ctx)
        return ctx

    yield make
    for ctx in made:
        ctx.close()
