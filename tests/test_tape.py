"""The C++ device tape (talos-xii_amd/host/tape.hpp): the reference's own autograd tests and
oracle-compared graphs, run by tests/cpp/test_tape (built by __graft_entry__.build())."""
import os
import subprocess

import pytest

import talos_hip as th

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "test_tape")


def _run():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build()")
    return subprocess.run([BIN], capture_output=True, text=True, timeout=110)


@pytest.mark.gpu
def test_tape_reference_tests_on_gpu():
    r = _run()
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert " 0 failed" in r.stdout


def test_tape_without_gpu_fails_cleanly():
    # no GPU: the first device allocation raises the library's message instead of crashing
    if th.device_count() > 0:
        pytest.skip("a GPU is present")
    r = _run()
    assert r.returncode == 1
    assert "no usable GPU" in r.stdout
