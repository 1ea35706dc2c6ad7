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
