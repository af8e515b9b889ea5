"""Runs the C++-API test program (tests/cpp/*.cpp, built into lib/ctd_tests by
emberlm_amd/build.py) on the GPU: tiny models built through include/ctd/ as the
reference's own tests build them (training vs inference logits, overfitting a
fixed batch with and without checkpointing / offload, KV-cache equivalences)."""
import os
import subprocess

import pytest

from emberlm_amd import trainer as TR

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(TR.LIB_PATH), "ctd_tests")


def test_cpp_api_tests():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(EXE), "build first: python -m emberlm_amd.build"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


def test_cpp_ce_masked_past_int32_offsets():
    """ops::cross_entropy_masked and its backward over N = 14200 rows of
    V = 151936 logits (2.16e9 elements): the loss and the dlogits of rows on
    both sides of 2^31 against the oracle (the reference's int32 row * V
    offsets wrap there, src/ops/loss.cu:263-264, 322-323)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(EXE), "build first: python -m emberlm_amd.build"
    r = subprocess.run([EXE, "--large"], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
