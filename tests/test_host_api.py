"""The C++ host API (include/thrml_hip.hpp) through its test program
tests/native/build/host_api_test (built by __graft_entry__.build()).  The CPU
test runs the cases that make no GPU call (RngKey::split against the oracle,
lattice and colouring known answers); the GPU test runs every case: the
reference's energy cases, a lattice sweep and hinton_init bit-identical to the
oracle, estimate_moments with a clamped block, categorical sweeps (q = 4 and q = 300
through the two-byte accessors), a discrete
factor program's sweep and energies, dense energies, the reference's error
strings, and a caller's observer run through sample_with_observation."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "native", os.environ.get("THRML_NATIVE_BUILD", "build"), "host_api_test")


def _run(*args, timeout=120):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    return r.stdout


def test_host_api_cpu_cases():
    out = _run("--cpu-only")
    assert "3 of 3 cases passed" in out


@pytest.mark.gpu
def test_host_api_all_cases():
    out = _run()
    assert "12 of 12 cases passed" in out
