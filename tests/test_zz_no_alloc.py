"""The allocation-free RMSNorm backward (ember_rmsnorm_bwd_noalloc), called
through the C ABI, against the workspace entry point ember_rmsnorm_bwd on the
same inputs: dx and dw bitwise equal, over two calls in a row of which the
second is smaller, so the second reads a scratch array that still holds the
first call's partials.  Sizes: the Qwen3-1.7B block norm (32768 rows x 2048,
4 MiB of partials), then QK-Norm-width rows (x 128), then a ragged H that
takes the scalar kernel."""
import numpy as np
import pytest

from emberlm_amd import capi
from tests.helpers import call, dev, empty, p

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _both(rows, H, seed, with_rstd=True, with_dx=True):
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, H)).astype(np.float32)
    dy = r.standard_normal((rows, H)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    X, DY, W = dev(x), dev(dy), dev(w)
    RS = None
    if with_rstd:
        Y, RS = empty((rows, H)), empty((rows,))
        call("ember_rmsnorm_fwd", p(X), p(W), p(Y), p(RS), rows, H, 1e-6, None)
    ws_n = int(capi.lib().ember_rmsnorm_bwd_workspace_bytes(rows, H))
    assert 0 < ws_n <= 16 << 20
    WS = empty((ws_n // 4,))
    DX1 = empty((rows, H)) if with_dx else None
    DX2 = empty((rows, H)) if with_dx else None
    DW1, DW2 = empty((H,)), empty((H,))
    DW2.fill_(float("nan"))
    call("ember_rmsnorm_bwd", p(DY), p(X), p(W), p(RS), p(DX1), p(DW1), rows, H, 1e-6, p(WS),
         ws_n, None)
    call("ember_rmsnorm_bwd_noalloc", p(DY), p(X), p(W), p(RS), p(DX2), p(DW2), rows, H, 1e-6,
         None)
    torch.cuda.synchronize()
    assert torch.equal(DW1, DW2), (rows, H)
    if with_dx:
        assert torch.equal(DX1, DX2), (rows, H)


def test_noalloc_equals_workspace_entry_over_calls():
    _both(32768, 2048, seed=1)                  # 512 partial rows x 2048
    _both(4096, 128, seed=2)                    # smaller: 512 partial rows x 128
    _both(300, 70, seed=3, with_rstd=False)     # scalar kernel, rstd recomputed
    _both(257, 2048, seed=4, with_dx=False)     # dw only


def test_noalloc_rejects_beyond_scratch():
    # H = 8192 at 32768 rows needs 1024 x 8192 floats = 32 MiB of partials; the
    # buffers are full size, and the call returns before any launch.
    lib = capi.lib()
    rows, H = 32768, 8192
    assert lib.ember_rmsnorm_bwd_workspace_bytes(rows, H) > 16 << 20
    X, DY, W, D = empty((rows, H)), empty((rows, H)), empty((H,)), empty((H,))
    rc = lib.ember_rmsnorm_bwd_noalloc(p(DY), p(X), p(W), None, None, p(D), rows, H, 1e-6, None)
    assert rc == -5 and b"fixed scratch" in lib.ember_status_string(rc)
