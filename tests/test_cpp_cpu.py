"""The C++-API test program's host-only tests (lib/ctd_tests --cpu): the
safetensors reader and writer on host tensors — the writer's exact header bytes
for a hand-written example, the round trip, SafetensorsReader::read, and each
class of malformed file.  The GPU run of the same program adds the device
variants (tests/test_gpu_cpp.py)."""
import os
import subprocess

from emberlm_amd import trainer as TR

EXE = os.path.join(os.path.dirname(TR.LIB_PATH), "ctd_tests")


def test_cpp_host_tests():
    assert os.path.exists(EXE), "build first: python -m emberlm_amd.build"
    r = subprocess.run([EXE, "--cpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
