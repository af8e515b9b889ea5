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
