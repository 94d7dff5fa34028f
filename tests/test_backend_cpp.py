"""The C++ Backend adapter (include/halo_mi355x_backend.hpp) through its own C++ test program,
tests/cpp/backend_pair.cpp: gemv on GGUF and SLAB buffers against the CPU oracle (bitwise /
within the bound), batch invariance, gate_up_swiglu, and the reference's error mapping."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "backend_pair")


def _need_binary():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: build it with __graft_entry__.build()")


def test_binary_links_library_and_oracle():
    """Loads without a GPU: every symbol the adapter and the test use resolves."""
    _need_binary()
    r = subprocess.run([BIN, "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "backend_pair" in r.stdout


@pytest.mark.gpu
def test_backend_adapter_on_the_gpu():
    _need_binary()
    print("[case] backend_pair (C++ adapter)", flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    sys.stdout.write(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
