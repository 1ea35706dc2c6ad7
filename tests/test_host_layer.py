"""Runs the C++ host-layer tests (tests/cpp/host_tests.cpp).

The CPU half covers the block pool, block tables, prefix forks, the
scheduler and step assembly on host-memory slabs; the GPU half drives the
same layer over HBM slabs through the C ABI (per-layer append protocol,
gather, single-sequence decode, a mixed bf16 step over several layers) and
checks it against the CPU oracle. The binary is built by
__graft_entry__.build().
"""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "_build" / "host_tests"


def _run(mode):
    assert BIN.exists(), f"{BIN} is not built (run __graft_entry__.build())"
    r = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    print(r.stderr[-4000:])
    assert r.returncode == 0, f"host_tests {mode} failed:\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
    assert "0 failed" in r.stdout


def test_host_layer_cpu():
    _run("--cpu")


@pytest.mark.gpu
def test_host_layer_gpu():
    _run("--gpu")


@pytest.mark.parametrize("value,want", [(None, "unset"), ("", "unset"), ("hip", "hip"),
                                        ("avx2", "cpu"), ("scalar", "cpu"), ("neon", "cpu")])
def test_process_device_choice_from_environment(value, want):
    """ENGINE_FORCE_ISA as a fresh process reads it: a CPU ISA name pins the
    CPU kernels, "hip" the GPU path, nothing leaves it to the pool."""
    import os
    env = {k: v for k, v in os.environ.items() if k != "ENGINE_FORCE_ISA"}
    if value is not None:
        env["ENGINE_FORCE_ISA"] = value
    r = subprocess.run([str(BIN), "--forced"], capture_output=True, text=True, timeout=30, env=env)
    assert r.returncode == 0 and r.stdout.strip() == want, (r.returncode, r.stdout, r.stderr)


def test_unknown_forced_isa_is_fatal():
    import os
    env = dict(os.environ, ENGINE_FORCE_ISA="cuda")
    r = subprocess.run([str(BIN), "--forced"], capture_output=True, text=True, timeout=30, env=env)
    assert r.returncode == -6 and "names no kernel set" in r.stderr
