"""GPU parity of every kernel behind include/ember_hip.h against the CPU oracle.

Called through the C ABI (ctypes); torch only provides device buffers.  Sizes
are the configs' real per-op shapes where the oracle finishes in seconds, plus
ragged/odd shapes that take the scalar paths; bitwise run-to-run determinism
is checked for every kernel that the checkpointed recompute relies on.
Tolerance: |a-b| <= 1e-4|b| + 1e-4 max|b| and relative L2 <= 1e-4 (fp32 vs the
fp64 oracle); AdamW 1e-5.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O
from emberlm_amd import capi
from tests.helpers import assert_close, call, dev, empty, fma_f32, host, p

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

I64 = C.c_int64


def rng(s=0):
    return np.random.default_rng(s)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()


# ------------------------------------------------------------------ GEMM
def gemm(a, b, ta, tb, alpha=1.0, beta=0.0, c=None):
    A, B = dev(a), dev(b)
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    Cm = dev(c) if c is not None else empty((M, N))
    call("ember_gemm_f32", int(ta), int(tb), M, N, K, alpha, p(A), a.shape[1], 0, p(B),
         b.shape[1], 0, beta, p(Cm), N, 0, 1, None)
    return host(Cm)


@pytest.mark.parametrize("M,N,K,ta,tb", [
    (256, 576, 576, 0, 1),    # c1 q/o projection (Linear, NT)
    (256, 192, 576, 0, 1),    # c1 k/v projection
    (256, 1536, 576, 0, 1),   # c1 gate/up
    (256, 576, 1536, 0, 0),   # c1 down dX (NN)
    (1536, 576, 256, 1, 0),   # c1 dW (TN, K = tokens)
    (37, 53, 29, 0, 0), (37, 53, 29, 0, 1), (37, 53, 29, 1, 0), (37, 53, 29, 1, 1),
    (130, 129, 18, 1, 1), (1, 1, 1, 0, 0),
])
def test_gemm_vs_oracle(M, N, K, ta, tb):
    r = rng(M + N + K)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    assert_close(gemm(a, b, ta, tb), O.matmul(a, b, ta, tb), name="gemm")


def test_gemm_alpha_beta_and_kat():
    # tests/test_matmul.cpp:48-67 known answer
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.arange(1, 13, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(gemm(a, b, 0, 0), [[38, 44, 50, 56], [83, 98, 113, 128]])
    r = rng(3)
    a = r.standard_normal((70, 40)).astype(np.float32)
    b = r.standard_normal((40, 90)).astype(np.float32)
    c = r.standard_normal((70, 90)).astype(np.float32)
    got = gemm(a, b, 0, 0, alpha=0.5, beta=1.0, c=c)
    assert_close(got, 0.5 * O.matmul(a, b) + c, name="alpha/beta")


@pytest.mark.parametrize("K", [40, 48])
def test_gemm_batched(K):
    r = rng(4)
    a = r.standard_normal((3, 64, K)).astype(np.float32)
    b = r.standard_normal((3, 72, K)).astype(np.float32)
    A, B = dev(a), dev(b)
    Cm = empty((3, 64, 72))
    call("ember_gemm_f32", 0, 1, 64, 72, K, 1.0, p(A), K, 64 * K, p(B), K, 72 * K, 0.0, p(Cm),
         72, 64 * 72, 3, None)
    assert_close(host(Cm), O.bmm(a, b, False, True), name="bmm")


def test_gemm_full_size_vs_torch_and_deterministic():
    # c5 gate projection shape, checked against torch's fp32 GEMM on the GPU.
    M, N, K = 32768, 6144, 2048
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(M, K, device="cuda", generator=g)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    out = empty((M, N))
    call("ember_gemm_f32", 0, 1, M, N, K, 1.0, p(x), K, 0, p(w), K, 0, 0.0, p(out), N, 0, 1, None)
    ref = x @ w.t()
    torch.cuda.synchronize()
    rel = ((out - ref).norm() / ref.norm()).item()
    assert rel < 1e-5, (rel, int((~torch.isfinite(out)).sum()), int((~torch.isfinite(ref)).sum()),
                        int((~torch.isfinite(x)).sum()), int((~torch.isfinite(w)).sum()))
    out2 = empty((M, N))
    call("ember_gemm_f32", 0, 1, M, N, K, 1.0, p(x), K, 0, p(w), K, 0, 0.0, p(out2), N, 0, 1, None)
    assert torch.equal(out, out2)


def gemm_ws(a, b, ta, tb, alpha=1.0, beta=0.0, c=None, ws_bytes=None):
    """ember_gemm_f32_ws with the workspace it asks for (or ws_bytes)."""
    A, B = dev(a), dev(b)
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    need = capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1)
    nb = need if ws_bytes is None else ws_bytes
    ws = torch.empty(max(nb // 4, 1), device="cuda")
    Cm = dev(c) if c is not None else empty((M, N))
    call("ember_gemm_f32_ws", int(ta), int(tb), M, N, K, alpha, p(A), a.shape[1], 0, p(B),
         b.shape[1], 0, beta, p(Cm), N, 0, 1, p(ws) if nb else None, nb, None)
    return host(Cm), need


@pytest.mark.parametrize("ta,tb,K", [(1, 0, 5003), (0, 0, 5003), (0, 1, 5003), (1, 1, 5003),
                                     (1, 0, 5008), (0, 1, 5008)]
                         + [(ta, tb, K) for K in (1000, 2048) for ta in (0, 1) for tb in (0, 1)])
def test_gemm_split_k_vs_oracle(ta, tb, K):
    # Few output tiles: the K-split path with partials (K % 16 == 0 takes the
    # LDS-DMA kernel, a ragged K the register-staged one), 16 splits of a long K
    # and 3 or 8 of a short one.
    M, N = 132, 200
    r = rng(11 + 2 * ta + tb)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c = r.standard_normal((M, N)).astype(np.float32)
    got, need = gemm_ws(a, b, ta, tb, alpha=0.5, beta=0.25, c=c)
    assert need >= 2 * M * N * 4  # the split path really ran
    ref = 0.5 * O.matmul(a, b, ta, tb) + 0.25 * c
    assert_close(got, ref, name="split-K")
    again, _ = gemm_ws(a, b, ta, tb, alpha=0.5, beta=0.25, c=c)
    assert np.array_equal(got, again)  # fixed-order reduction
    # no workspace: the one-pass kernel, same product
    one, _ = gemm_ws(a, b, ta, tb, alpha=0.5, beta=0.25, c=c, ws_bytes=0)
    assert_close(one, ref, name="unsplit")


@pytest.mark.parametrize("ta,tb,M,N,K", [
    (1, 0, 2048, 2048, 32768),   # c5 q/o weight gradient: 8 splits on 256x128 tiles
    (1, 0, 6144, 2048, 32768),   # gate/up: 4 splits
    (0, 0, 4096, 2048, 8192),    # NN (the LM head's dh form): 4 splits
])
def test_gemm_split_k_on_256_tiles_vs_torch(ta, tb, M, N, K):
    """The K split on 256x128 tiles against an fp64 product on the GPU, and
    bitwise the same on a second call (fixed-order reduce)."""
    g = torch.Generator(device="cuda").manual_seed(M + K)
    a = torch.randn((K, M) if ta else (M, K), device="cuda", generator=g)
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g)
    wsb = int(capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1))
    assert wsb >= 4 * M * N * 4   # the split path
    ws = empty((wsb // 4,))
    out, out2 = empty((M, N)), empty((M, N))
    for o in (out, out2):
        call("ember_gemm_f32_ws", ta, tb, M, N, K, 1.0, p(a), a.shape[1], 0, p(b), b.shape[1], 0,
             0.0, p(o), N, 0, 1, p(ws), wsb, None)
    ad, bd = a.double(), b.double()
    ref = ((ad.t() if ta else ad) @ (bd.t() if tb else bd)).float()
    rel = ((out - ref).norm() / ref.norm()).item()
    assert rel < 1e-5, rel
    assert torch.equal(out, out2)


@pytest.mark.parametrize("ta,tb", [(1, 0), (1, 1)])
def test_gemm_m_contiguous_a_on_256_tiles_ragged_rows(ta, tb):
    """An M-contiguous A on the unsplit 256x128 kernel (its tile rows sit
    permuted in the MFMA registers and are mapped back in the store), with a
    last row tile holding 4 rows: every row of C against an fp64 product, the
    rows past M (a guard band after C) left alone."""
    M, N, K = 8196, 4096, 512          # 33 x 32 tiles of 256 x 128: the unsplit big-tile plan
    g = torch.Generator(device="cuda").manual_seed(11 + tb)
    a = torch.randn(K, M, device="cuda", generator=g)
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g)
    buf = torch.full((M + 8, N), 7.0, device="cuda")
    call("ember_gemm_f32_ws", ta, tb, M, N, K, 1.0, p(a), M, 0, p(b), b.shape[1], 0, 0.0,
         p(buf), N, 0, 1, None, 0, None)
    ad, bd = a.double(), b.double()
    ref = (ad.t() @ (bd.t() if tb else bd)).float()
    rel = ((buf[:M] - ref).norm() / ref.norm()).item()
    assert rel < 1e-5, rel
    row_rel = ((buf[:M] - ref).norm(dim=1) / ref.norm(dim=1)).max().item()
    assert row_rel < 1e-5, row_rel     # no row lost or swapped
    assert torch.equal(buf[M:], torch.full((8, N), 7.0, device="cuda"))


def test_gemm_dyn_rows_split_on_256_tiles_vs_torch():
    """The device-sized GEMM (rows of C wanted up to a count) on the 256x128
    K split: rows below the count match an fp64 product, whole row tiles past
    it are left alone."""
    M, N, K, count = 4096, 2048, 8192, 1000
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randn(M, K, device="cuda", generator=g)
    b = torch.randn(K, N, device="cuda", generator=g)
    wsb = int(capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1))
    ws = empty((wsb // 4,))
    out = torch.full((M, N), 7.0, device="cuda")
    cnt = dev(np.array([count], np.int64))
    call("ember_gemm_f32_dyn", 0, 0, M, N, K, 1.0, p(a), K, p(b), N, 0.0, p(out), N, p(cnt), 0,
         0, p(ws), wsb, None)
    ref = (a[:count].double() @ b.double()).float()
    rel = ((out[:count] - ref).norm() / ref.norm()).item()
    assert rel < 1e-5, rel
    assert bool((out[1024:] == 7.0).all())   # tiles of 256 rows past the count


def test_gemm_split_k_weight_gradient_shape_vs_torch():
    # c5 k/v weight gradient: dW[1024,2048] = dY^T X over 32768 tokens (TN).
    M, N, K = 1024, 2048, 32768
    assert capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1) > 0
    g = torch.Generator(device="cuda").manual_seed(1)
    dy = torch.randn(K, M, device="cuda", generator=g)
    x = torch.randn(K, N, device="cuda", generator=g)
    ws = torch.empty(capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1) // 4, device="cuda")
    out = empty((M, N))
    call("ember_gemm_f32_ws", 1, 0, M, N, K, 1.0, p(dy), M, 0, p(x), N, 0, 0.0, p(out), N, 0, 1,
         p(ws), ws.numel() * 4, None)
    ref = (dy.double().t() @ x.double()).float()
    rel = ((out - ref).norm() / ref.norm()).item()
    assert rel < 1e-5, rel


@pytest.mark.parametrize("ta,tb,M,N,K", [
    (0, 1, 33000, 1000, 40), (0, 0, 33000, 1000, 40), (1, 0, 33000, 1000, 40),
    (1, 1, 33000, 1000, 40),                        # register-staged kernel (K % 16 != 0)
    (0, 1, 33000, 1000, 48), (0, 0, 33000, 1000, 48), (1, 0, 33000, 1000, 48),
    (1, 1, 33000, 1000, 48),                        # LDS-DMA kernel, M, N off the tile grid
    (0, 1, 33001, 999, 48),                         # LDS-DMA, K-contiguous rows clamped
    # one and two 16-k stages: the peeled k loop's DMA-free tail only
    (0, 1, 33000, 1000, 16), (0, 0, 33000, 1000, 32), (1, 0, 33000, 1000, 16),
    (1, 1, 33000, 1000, 32), (0, 1, 500, 300, 16), (1, 0, 500, 300, 32),
    (0, 1, 500, 300, 64),                           # 128x128 tiles, two stages of DMA ahead
])
def test_gemm_large_tile_ragged_vs_oracle(ta, tb, M, N, K):
    # Enough tiles for the 256x128 kernels, with M and N off the tile grid.
    r = rng(21 + 2 * ta + tb)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    assert_close(gemm(a, b, ta, tb), O.matmul(a, b, ta, tb), name="gemm 256x128")


# -------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("rows,H,eps", [(256, 576, 1e-5), (4096, 128, 1e-6), (999, 64, 1e-5),
                                        (33, 2048, 1e-6), (7, 30, 1e-5), (3, 4, 1e-5)])
def test_rmsnorm_fwd_bwd_vs_oracle(rows, H, eps):
    r = rng(rows + H)
    x = r.standard_normal((rows, H)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    dy = r.standard_normal((rows, H)).astype(np.float32)
    X, W, DY = dev(x), dev(w), dev(dy)
    Y, RS = empty((rows, H)), empty((rows,))
    call("ember_rmsnorm_fwd", p(X), p(W), p(Y), p(RS), rows, H, eps, None)
    assert_close(host(Y), O.rmsnorm_fwd(x, w, eps), name="rms fwd")
    ws_n = int(capi.lib().ember_rmsnorm_bwd_workspace_bytes(rows, H))
    WS = empty((max(ws_n // 4, 1),))
    DX, DW = empty((rows, H)), empty((H,))
    call("ember_rmsnorm_bwd", p(DY), p(X), p(W), p(RS), p(DX), p(DW), rows, H, eps, p(WS), ws_n, None)
    dx_ref, dw_ref = O.rmsnorm_bwd(dy, x, w, eps)
    assert_close(host(DX), dx_ref, name="rms dx")
    assert_close(host(DW), dw_ref, name="rms dw")
    # bitwise determinism, and the recomputed-rstd path gives the same bits as the
    # saved-rstd path (forward and backward accumulate sum(x^2) in the same order)
    DX2, DW2 = empty((rows, H)), empty((H,))
    call("ember_rmsnorm_bwd", p(DY), p(X), p(W), p(RS), p(DX2), p(DW2), rows, H, eps, p(WS), ws_n, None)
    assert torch.equal(DW, DW2) and torch.equal(DX, DX2)
    call("ember_rmsnorm_bwd", p(DY), p(X), p(W), None, p(DX2), p(DW2), rows, H, eps, p(WS), ws_n, None)
    assert torch.equal(DW, DW2) and torch.equal(DX, DX2)
    Y2 = empty((rows, H))
    call("ember_rmsnorm_fwd", p(X), p(W), p(Y2), None, rows, H, eps, None)
    assert torch.equal(Y, Y2)


def test_rmsnorm_full_size_c5():
    rows, H = 32768, 2048
    x = torch.randn(rows, H, device="cuda")
    w = torch.rand(H, device="cuda") + 0.5
    y = empty((rows, H))
    call("ember_rmsnorm_fwd", p(x), p(w), p(y), None, rows, H, 1e-6, None)
    ref = x * torch.rsqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6).float() * w
    torch.cuda.synchronize()
    assert ((y - ref).abs().max() / ref.abs().max()).item() < 1e-5


@pytest.mark.parametrize("rows,H", [(300, 2048), (1000, 128), (77, 576), (50, 130)])
def test_rmsnorm_bwd_accumulate_bitwise(rows, H):
    """dx += the input gradient: bitwise ember_rmsnorm_bwd followed by one add
    per element (the float4 paths at 2048, 128 and 576, the scalar one at 130)."""
    r = rng(rows + H)
    x = r.standard_normal((rows, H)).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(H)).astype(np.float32)
    dy = r.standard_normal((rows, H)).astype(np.float32)
    d0 = r.standard_normal((rows, H)).astype(np.float32)
    X, W, DY, D0 = dev(x), dev(w), dev(dy), dev(d0)
    ws_n = int(capi.lib().ember_rmsnorm_bwd_workspace_bytes(rows, H))
    WS = empty((max(ws_n // 4, 1),))
    DX, DW, DW2 = empty((rows, H)), empty((H,)), empty((H,))
    call("ember_rmsnorm_bwd", p(DY), p(X), p(W), None, p(DX), p(DW), rows, H, 1e-6, p(WS), ws_n,
         None)
    ACC = D0.clone()
    call("ember_rmsnorm_bwd_accumulate", p(DY), p(X), p(W), None, p(ACC), p(DW2), rows, H, 1e-6,
         p(WS), ws_n, None)
    assert torch.equal(ACC, D0 + DX) and torch.equal(DW2, DW)


# ----------------------------------------------------------------- RoPE
def freqs(D, theta, factor=0.0):
    out = (C.c_float * (D // 2))()
    capi.check(capi.lib().ember_rope_freqs_host(out, D, theta, factor, 1.0, 4.0, 8192))
    return out


@pytest.mark.parametrize("B,T,H,D,theta,factor,pos0,sign", [
    (1, 256, 9, 64, 1e5, 0.0, 0, 1.0),       # c1 Q
    (2, 300, 2, 128, 1e6, 0.0, 0, -1.0),     # c3/c5 head_dim, transpose (backward)
    (1, 2048, 2, 64, 5e5, 32.0, 0, 1.0),     # c4 llama3 scaling, full T
    (1, 4096, 1, 128, 1e6, 0.0, 0, 1.0),     # c5 full T (large angles)
    (1, 5, 3, 8, 1e4, 0.0, 7, 1.0),          # position offset (test_rope.cpp:57-72)
])
def test_rope_vs_oracle(B, T, H, D, theta, factor, pos0, sign):
    r = rng(T + D)
    x = r.standard_normal((B, T, H, D)).astype(np.float32)
    X, Y = dev(x), empty((B, T, H, D))
    call("ember_rope", p(X), p(Y), B, T, H, D, pos0, freqs(D, theta, factor), sign, None)
    ref = O.rope(x, theta, pos0=pos0, sign=sign, factor=factor)
    assert_close(host(Y), ref, name="rope")
    # in place (apply_rope_inplace) gives the same bits
    call("ember_rope", p(X), p(X), B, T, H, D, pos0, freqs(D, theta, factor), sign, None)
    assert torch.equal(X, Y)


def test_rope_roundtrip_identity():
    x = torch.randn(2, 64, 4, 128, device="cuda")
    y, z = torch.empty_like(x), torch.empty_like(x)
    fr = freqs(128, 1e6)
    call("ember_rope", p(x), p(y), 2, 64, 4, 128, 0, fr, 1.0, None)
    call("ember_rope", p(y), p(z), 2, 64, 4, 128, 0, fr, -1.0, None)
    torch.cuda.synchronize()
    assert (z - x).abs().max().item() < 1e-5


@pytest.mark.parametrize("B,T,H,D,theta,factor,pos0", [
    (2, 64, 16, 128, 1e6, 0.0, 0),      # Qwen3 q heads
    (1, 37, 8, 128, 1e6, 0.0, 5),       # k heads, ragged row count, offset positions
    (2, 50, 3, 64, 5e5, 32.0, 0),       # D = 64 with llama3 frequencies
    (1, 4096, 2, 128, 1e6, 0.0, 0),     # full T: large angles
])
def test_qknorm_rope_bitwise_equals_norm_then_rope(B, T, H, D, theta, factor, pos0):
    """The fused QK-Norm + RoPE kernels against ember_rmsnorm_* and ember_rope
    run one after the other (each pinned against the oracle above): forward
    y and rstd, backward dx and dw, bit for bit."""
    r = rng(B * T * H + D)
    rows, eps = B * T * H, 1e-6
    x = r.standard_normal((B, T, H, D)).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(D)).astype(np.float32)
    dy = r.standard_normal((B, T, H, D)).astype(np.float32)
    X, W, DY = dev(x), dev(w), dev(dy)
    fr = freqs(D, theta, factor)
    # separate kernels
    Yn, RS, Yr = empty((B, T, H, D)), empty((rows,)), empty((B, T, H, D))
    call("ember_rmsnorm_fwd", p(X), p(W), p(Yn), p(RS), rows, D, eps, None)
    call("ember_rope", p(Yn), p(Yr), B, T, H, D, pos0, fr, 1.0, None)
    G, DX, DW = empty((B, T, H, D)), empty((B, T, H, D)), empty((D,))
    ws_n = int(capi.lib().ember_rmsnorm_bwd_workspace_bytes(rows, D))
    WS = empty((max(ws_n // 4, 1),))
    call("ember_rope", p(DY), p(G), B, T, H, D, pos0, fr, -1.0, None)
    call("ember_rmsnorm_bwd", p(G), p(X), p(W), p(RS), p(DX), p(DW), rows, D, eps, p(WS), ws_n,
         None)
    # fused
    Y, RS2, DX2, DW2 = empty((B, T, H, D)), empty((rows,)), empty((B, T, H, D)), empty((D,))
    call("ember_qknorm_rope_fwd", p(X), p(W), p(Y), p(RS2), rows, H, T, D, eps, pos0, fr, None)
    call("ember_qknorm_rope_bwd", p(DY), p(X), p(W), p(RS2), p(DX2), p(DW2), rows, H, T, D, eps,
         pos0, fr, p(WS), ws_n, None)
    assert torch.equal(Y, Yr) and torch.equal(RS2, RS)
    assert torch.equal(DX2, DX) and torch.equal(DW2, DW)
    # dx alone, no rstd (recomputed), as the separate kernels do it
    DX3 = empty((B, T, H, D))
    call("ember_qknorm_rope_bwd", p(DY), p(X), p(W), None, p(DX3), None, rows, H, T, D, eps,
         pos0, fr, None, 0, None)
    call("ember_rmsnorm_bwd", p(G), p(X), p(W), None, p(DX), None, rows, D, eps, None, 0, None)
    assert torch.equal(DX3, DX)


def test_qknorm_rope_rejects_other_head_dims():
    X = empty((4, 96))
    fr = freqs(96, 1e6)
    with pytest.raises(capi.EmberError):
        capi.call("ember_qknorm_rope_fwd", p(X), p(X[0]), p(X), None, 4, 2, 2, 96, 1e-6, 0, fr,
                  None)


# ----------------------------------------------------------- elementwise
def test_elementwise_vs_oracle():
    r = rng(5)
    n = 1536 * 256 + 3  # odd tail
    a = (r.standard_normal(n) * 3).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    g = r.standard_normal(n).astype(np.float32)
    A, Bt, G = dev(a), dev(b), dev(g)
    Y = empty((n,))
    call("ember_add", p(A), p(Bt), p(Y), n, None)
    assert np.array_equal(host(Y), a + b)
    call("ember_mul", p(A), p(Bt), p(Y), n, None)
    assert np.array_equal(host(Y), a * b)
    call("ember_sub", p(A), p(Bt), p(Y), n, None)
    assert np.array_equal(host(Y), a - b)
    call("ember_scale", p(A), 0.125, p(Y), n, None)
    assert np.array_equal(host(Y), a * np.float32(0.125))
    call("ember_silu", p(A), p(Y), n, None)
    assert_close(host(Y), O.silu(a), name="silu")
    call("ember_silu_bwd", p(A), p(G), p(Y), n, None)
    assert_close(host(Y), O.silu_bwd(a, g), name="silu bwd")
    call("ember_swiglu_fwd", p(A), p(Bt), p(Y), n, None)
    assert_close(host(Y), O.silu(a) * b, name="swiglu fwd")
    DG, DU = empty((n,)), empty((n,))
    call("ember_swiglu_bwd", p(A), p(Bt), p(G), p(DG), p(DU), n, None)
    assert_close(host(DG), O.silu_bwd(a, g * b), name="swiglu dg")
    assert_close(host(DU), g * O.silu(a), name="swiglu du")
    # in place (dg over g, du over u, as the MLP's backward runs it): the same
    # bits as into separate buffers, on the vector path and the scalar one
    for off in (0, 1):
        m = n - off
        A2, B2 = dev(a), dev(b)
        pa = C.c_void_p(A2.data_ptr() + 4 * off)
        pb = C.c_void_p(B2.data_ptr() + 4 * off)
        pg = C.c_void_p(G.data_ptr() + 4 * off)
        DG2, DU2 = empty((m,)), empty((m,))
        call("ember_swiglu_bwd", pa, pb, pg, p(DG2), p(DU2), m, None)
        call("ember_swiglu_bwd", pa, pb, pg, pa, pb, m, None)
        assert torch.equal(A2[off:], DG2) and torch.equal(B2[off:], DU2), off
        # forward over the gate (nn::MLP's no-grad activation)
        A3, H3 = dev(a), empty((m,))
        pa3 = C.c_void_p(A3.data_ptr() + 4 * off)
        call("ember_swiglu_fwd", pa3, pb, p(H3), m, None)
        call("ember_swiglu_fwd", pa3, pb, pa3, m, None)
        assert torch.equal(A3[off:], H3), off
    Z = dev(b)
    call("ember_accumulate", p(Z), p(A), n, None)
    assert np.array_equal(host(Z), b + a)
    # misaligned (scalar) path
    call("ember_add", C.c_void_p(A.data_ptr() + 4), C.c_void_p(Bt.data_ptr() + 4), p(Y), n - 1, None)
    assert np.array_equal(host(Y)[: n - 1], a[1:] + b[1:])


# ------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("N,V", [(64, 49152), (8, 151936), (33, 1001), (5, 7)])
def test_ce_masked_vs_oracle(N, V):
    r = rng(N + V)
    logits = (r.standard_normal((N, V)) * 2).astype(np.float32)
    tgt = r.integers(0, V, N).astype(np.int64)
    mask = (r.random(N) > 0.4).astype(np.float32)
    mask[0] = 1.0
    L, T_, M = dev(logits), dev(tgt), dev(mask)
    lse, loss, ms = empty((N,)), empty((1,)), empty((1,))
    ws = empty((N,))
    call("ember_ce_masked_fwd", p(L), p(T_), p(M), N, V, p(lse), p(loss), p(ms), p(ws), N * 4, None)
    ref_loss, ref_lse, ref_ms = O.ce_masked_fwd(logits, tgt, mask)
    assert abs(host(loss)[0] - ref_loss) <= 1e-5 * abs(ref_loss)
    assert host(ms)[0] == ref_ms
    live = mask > 0
    assert_close(host(lse)[live], ref_lse[live], name="lse")
    dl = dev(np.array([0.7], np.float32))
    D_ = empty((N, V))
    call("ember_ce_masked_bwd", p(L), p(T_), p(M), p(lse), p(dl), p(ms), N, V, p(D_), None)
    ref_d = O.ce_masked_bwd(logits, tgt, mask, dy=0.7)
    assert_close(host(D_), ref_d, name="dlogits")
    assert (host(D_)[~live] == 0).all()
    # in place over the logits gives the same bits
    call("ember_ce_masked_bwd", p(L), p(T_), p(M), p(lse), p(dl), p(ms), N, V, p(L), None)
    assert torch.equal(L, D_)


def test_ce_zero_mask_loss_is_zero():
    N, V = 4, 16
    L = torch.randn(N, V, device="cuda")
    T_ = torch.zeros(N, dtype=torch.int64, device="cuda")
    M = torch.zeros(N, device="cuda")
    lse, loss, ms, ws = empty((N,)), empty((1,)), empty((1,)), empty((N,))
    call("ember_ce_masked_fwd", p(L), p(T_), p(M), N, V, p(lse), p(loss), p(ms), p(ws), N * 4, None)
    assert host(loss)[0] == 0.0 and host(ms)[0] == 0.0


# ------------------------------------------ LM head over the active rows
def _mask_rows(mask):
    """idx, count of ember_mask_rows on the device (count as a device tensor)."""
    N = mask.shape[0]
    M = dev(mask)
    idx = torch.full((max(N, 1),), -7, dtype=torch.int64, device="cuda")
    cnt = torch.full((1,), -7, dtype=torch.int64, device="cuda")
    call("ember_mask_rows", p(M), N, p(idx), p(cnt), None)
    return idx, cnt


@pytest.mark.parametrize("N", [0, 1, 1000, 32768, 100003])
def test_mask_rows_lists_nonzero_rows(N):
    r = rng(N)
    mask = np.where(r.random(N) < 0.45, 0.0, r.standard_normal(N)).astype(np.float32)
    if N > 10:
        mask[3], mask[5], mask[7] = np.nan, -0.0, -2.0   # NaN counts, -0 does not
    idx, cnt = _mask_rows(mask)
    want = np.nonzero(mask != 0)[0]
    assert host(cnt)[0] == len(want)
    assert np.array_equal(host(idx)[: len(want)], want)
    if N > 10:
        assert 3 in want and 5 not in want and 7 in want


@pytest.mark.parametrize("H", [72, 30])   # float4 and scalar rows
def test_rows_gather_scatter(H):
    N, R = 3000, 1024
    r = rng(H)
    mask = (r.random(N) < 0.5).astype(np.float32)
    src = r.standard_normal((N, H)).astype(np.float32)
    idx, cnt = _mask_rows(mask)
    act = np.nonzero(mask)[0]
    S_ = dev(src)
    for base in (0, 512, 1400, len(act), len(act) + 5):
        n = min(max(len(act) - base, 0), R)
        D_ = torch.full((R, H), 5.0, device="cuda")
        call("ember_rows_gather", p(S_), H, H, p(idx), p(cnt), base, R, p(D_), None)
        d = host(D_)
        fill = min(R, -(-n // 256) * 256)
        assert np.array_equal(d[:n], src[act[base:base + n]])
        assert (d[n:fill] == 0).all() and (d[fill:] == 5.0).all()
        O_ = torch.full((N, H), 9.0, device="cuda")
        call("ember_rows_scatter", p(D_), H, p(idx), p(cnt), base, R, p(O_), H, None)
        o = host(O_)
        rows = act[base:base + n]
        assert np.array_equal(o[rows], src[rows])
        rest = np.ones(N, bool)
        rest[rows] = False
        assert (o[rest] == 9.0).all()


@pytest.mark.parametrize("V", [4096, 1001])
def test_ce_rows_idx_equal_all_rows_bitwise(V):
    # The active-rows CE over gathered logits rows gives the all-rows kernels'
    # lse, row loss and dlogits bits for those rows.
    N, R, base = 300, 128, 64
    r = rng(V)
    logits = (r.standard_normal((N, V)) * 2).astype(np.float32)
    tgt = r.integers(0, V, N).astype(np.int64)
    mask = (r.random(N) > 0.4).astype(np.float32)
    L, T_, M = dev(logits), dev(tgt), dev(mask)
    lse_f, rl_f = empty((N,)), empty((N,))
    call("ember_ce_masked_rows", p(L), p(T_), p(M), N, V, p(lse_f), p(rl_f), None)
    ms = dev(np.array([mask.sum()], np.float32))
    dl = dev(np.array([0.7], np.float32))
    D_ = empty((N, V))
    call("ember_ce_masked_bwd", p(L), p(T_), p(M), p(lse_f), p(dl), p(ms), N, V, p(D_), None)
    idx, cnt = _mask_rows(mask)
    act = np.nonzero(mask)[0]
    n = min(len(act) - base, R)
    Lc = empty((R, V))
    call("ember_rows_gather", p(L), V, V, p(idx), p(cnt), base, R, p(Lc), None)
    lse_c, rl = empty((R,)), torch.zeros(N, device="cuda")
    call("ember_ce_masked_rows_idx", p(Lc), p(T_), p(M), p(idx), p(cnt), base, R, V, p(lse_c),
         p(rl), None)
    rows = act[base:base + n]
    assert np.array_equal(host(lse_c)[:n], host(lse_f)[rows])
    rl_h = host(rl)
    assert np.array_equal(rl_h[rows], host(rl_f)[rows])
    others = np.ones(N, bool)
    others[rows] = False
    assert (rl_h[others] == 0).all()
    call("ember_ce_masked_bwd_idx", p(Lc), p(T_), p(M), p(lse_c), p(idx), p(cnt), base, R, V,
         p(dl), p(ms), p(Lc), None)
    assert np.array_equal(host(Lc)[:n], host(D_)[rows])


def _gemm_dyn(a, b, ta, tb, count, base, dim, beta=0.0, c=None, alpha=1.0):
    A, B = dev(a), dev(b)
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    Cm = dev(c) if c is not None else torch.full((M, N), 7.0, device="cuda")
    wsb = int(capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1)) if dim == 0 else 0
    ws = empty((max(wsb // 4, 1),))
    cnt = dev(np.array([count], np.int64))
    call("ember_gemm_f32_dyn", int(ta), int(tb), M, N, K, alpha, p(A), a.shape[1], p(B),
         b.shape[1], beta, p(Cm), N, p(cnt), base, dim, p(ws), wsb, None)
    return host(Cm)


@pytest.mark.parametrize("ta,tb,M,N,K,count,base", [
    (0, 1, 4096, 1200, 64, 4096, 0),      # every row
    (0, 1, 4096, 1200, 64, 1000, 0),
    (0, 1, 4096, 1200, 64, 1300, 300),     # count - base = 1000
    (0, 1, 4096, 1200, 64, 0, 0),          # nothing: C untouched
    (0, 1, 4096, 1200, 64, 99999, 10),     # clamped to M
    (0, 1, 8192, 4096, 32, 5000, 0),       # 256x128 tiles
    (0, 0, 512, 256, 8192, 300, 0),        # NN with a K split: partials + reduce
    (0, 0, 512, 256, 8192, 0, 0),
])
def test_gemm_dyn_rows_vs_oracle(ta, tb, M, N, K, count, base):
    r = rng(M + N + K + count)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    got = _gemm_dyn(a, b, ta, tb, count, base, 0)
    v = min(max(count - base, 0), M)
    if v:
        assert_close(got[:v], O.matmul(a[:v], b, ta, tb), name="gemm dyn rows")
    past = -(-v // 256) * 256
    assert (got[past:] == 7.0).all()   # whole row tiles past v are skipped


@pytest.mark.parametrize("H,V,count", [(1024, 2048, 300), (1024, 2048, 17), (512, 4096, 33)])
def test_gemm_dyn_rows_split_k_writes_the_last_16_row_group(H, V, count):
    # The LM head's logits GEMM (NT, rows sized on the device) on a grid of few
    # tiles, which splits K: rows [count, round16(count)) come from zero-filled
    # rows of h and must be stored as zeros (the dW product that follows reads
    # K rounded up to 16), whatever the output buffer held before.
    M = -(-count // 16) * 16 + 16
    assert capi.lib().ember_gemm_f32_workspace_bytes(M, V, H, 1) > 0   # K is split
    r = rng(H + V + count)
    hc = r.standard_normal((M, H)).astype(np.float32)
    hc[count:] = 0.0                                  # the gather's zero rows
    w = r.standard_normal((V, H)).astype(np.float32)
    a, b = dev(hc), dev(w)
    out = torch.full((M, V), float("nan"), device="cuda")
    wsb = int(capi.lib().ember_gemm_f32_workspace_bytes(M, V, H, 1))
    ws = empty((wsb // 4,))
    cnt = dev(np.array([count], np.int64))
    call("ember_gemm_f32_dyn", 0, 1, M, V, H, 1.0, p(a), H, p(b), H, 0.0, p(out), V, p(cnt), 0,
         0, p(ws), wsb, None)
    got = host(out)
    r16 = -(-count // 16) * 16
    assert_close(got[:count], O.matmul(hc[:count], w, False, True), name="logits rows")
    assert (got[count:r16] == 0.0).all(), "rows of the last 16-row group must be zeros"


@pytest.mark.parametrize("M,N,K,count,beta", [
    (1024, 512, 4096, 4096, 0.0), (1024, 512, 4096, 1000, 0.0), (1024, 512, 4096, 17, 0.0),
    (1024, 512, 4096, 1000, 1.0), (1024, 512, 4096, 0, 1.0), (1024, 512, 4096, 0, 0.0),
    (33000, 1024, 64, 40, 0.0),            # 256x128 tiles
])
def test_gemm_dyn_k_vs_oracle(M, N, K, count, beta):
    # TN (dW form): rows [v, round16(v)) of both operands are zero, rows past
    # that hold values the product must not read.
    r = rng(M + K + count)
    a = r.standard_normal((K, M)).astype(np.float32)
    b = r.standard_normal((K, N)).astype(np.float32)
    v = min(count, K)
    k16 = -(-v // 16) * 16
    a[v:k16] = 0
    b[v:k16] = 0
    c = r.standard_normal((M, N)).astype(np.float32)
    got = _gemm_dyn(a, b, 1, 0, count, 0, 1, beta=beta, c=c)
    ref = beta * c.astype(np.float64)
    if v:
        ref = ref + O.matmul(a[:v], b[:v], True, False)
    if v == 0 and beta == 1.0:
        assert np.array_equal(got, c)
    else:
        assert_close(got, ref, name="gemm dyn k")


def test_gemm_dyn_rejects_shapes_off_the_dma_path():
    A = empty((64, 40))
    cnt = dev(np.array([10], np.int64))
    Cm = empty((64, 64))
    with pytest.raises(capi.EmberError):   # K = 40 is not whole 16-k stages
        capi.call("ember_gemm_f32_dyn", 0, 1, 64, 64, 40, 1.0, p(A), 40, p(A), 40, 0.0, p(Cm),
                  64, p(cnt), 0, 0, None, 0, None)
    with pytest.raises(capi.EmberError):   # dim must be 0 or 1
        capi.call("ember_gemm_f32_dyn", 0, 1, 64, 64, 32, 1.0, p(A), 40, p(A), 40, 0.0, p(Cm),
                  64, p(cnt), 0, 2, None, 0, None)


# ------------------------------------------------- product + residual add
def _gemm_ws(A, B, ta, tb, M, N, K, lda, ldb):
    wsb = int(capi.lib().ember_gemm_f32_workspace_bytes(M, N, K, 1))
    ws = empty((max(wsb // 4, 1),))
    Cm = empty((M, N))
    call("ember_gemm_f32_ws", int(ta), int(tb), M, N, K, 1.0, p(A), lda, 0, p(B), ldb, 0, 0.0,
         p(Cm), N, 0, 1, p(ws), wsb, None)
    return Cm, ws, wsb


@pytest.mark.parametrize("ta,tb,M,N,K", [
    (0, 1, 4096, 2048, 512),    # Linear forward shape: 256x128 DMA tiles
    (0, 1, 300, 200, 64),       # 128x128 DMA tiles, ragged edges
    (0, 0, 1000, 300, 48),      # NN
    (1, 0, 256, 128, 8192),     # TN with a K split: the reduce adds D
    (1, 1, 200, 150, 70),       # K not whole 16-k stages: register-staged kernel
    (0, 1, 5, 1000, 256),       # M <= 8: skinny kernel
    (0, 1, 100, 64, 0),         # K = 0: C = D
])
def test_gemm_add_bitwise_equals_product_then_add(ta, tb, M, N, K):
    """ember_gemm_f32_add = the same product stored, then one IEEE add per
    element (torch's add here), bit for bit; D separate and D = C."""
    r = rng(M + 3 * N + 7 * K)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    d = r.standard_normal((M, N)).astype(np.float32)
    A, B, Dd = dev(a), dev(b), dev(d)
    lda, ldb = a.shape[1], b.shape[1]
    prod, ws, wsb = _gemm_ws(A, B, ta, tb, M, N, K, lda, ldb)
    want = host(prod + Dd)
    Cm = empty((M, N))
    call("ember_gemm_f32_add", int(ta), int(tb), M, N, K, 1.0, p(A), lda, p(B), ldb, p(Dd), N,
         p(Cm), N, p(ws), wsb, None)
    assert np.array_equal(host(Cm), want)
    C2 = Dd.clone()                 # D aliased to C: the beta = 1 form
    call("ember_gemm_f32_add", int(ta), int(tb), M, N, K, 1.0, p(A), lda, p(B), ldb, p(C2), N,
         p(C2), N, p(ws), wsb, None)
    assert np.array_equal(host(C2), want)
    if K:
        assert_close(host(Cm), O.matmul(a, b, ta, tb) + d, name="gemm add")


@pytest.mark.parametrize("ta,tb,big", [(0, 1, "a"), (1, 0, "a"), (0, 0, "b"), (1, 1, "b")])
def test_gemm_global_address_dma_bitwise_equals_buffer_dma(ta, tb, big):
    """The DMA kernels copy operands into LDS through a buffer resource with
    32-bit offsets unless some offset of the product reaches 2^31 bytes; then
    with 64-bit global addresses.  A leading dimension large enough to force
    the second form (a few strided rows of a 0.3-2.1 GB buffer) gives the same
    bits as the compact operands, which take the first."""
    M, N, K = 20, 20, 32
    r = rng(11 + 2 * ta + tb)
    a = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    want = gemm(a, b, ta, tb)
    x = a if big == "a" else b
    rows, cols = x.shape
    kc = (big == "a" and not ta) or (big == "b" and tb)
    ld = (1 << 22) if kc else (1 << 24)   # 128 * ld or K * ld floats: 2^31 bytes
    X = torch.zeros((rows - 1) * ld + cols, device="cuda")
    for i in range(rows):
        X[i * ld: i * ld + cols].copy_(torch.from_numpy(x[i]))
    Y = dev(b if big == "a" else a)
    A, lda = (X, ld) if big == "a" else (Y, a.shape[1])
    B, ldb = (X, ld) if big == "b" else (Y, b.shape[1])
    Cm = empty((M, N))
    call("ember_gemm_f32", int(ta), int(tb), M, N, K, 1.0, p(A), lda, 0, p(B), ldb, 0, 0.0,
         p(Cm), N, 0, 1, None)
    assert np.array_equal(host(Cm), want)
    del X
    torch.cuda.empty_cache()


def test_gemm_add_rejects_overlap_and_short_rows():
    A = empty((64, 32))
    buf = empty((65, 64))
    D, Cm = buf[1:], buf[:64]       # D starts one row into C
    with pytest.raises(capi.EmberError):
        capi.call("ember_gemm_f32_add", 0, 1, 64, 64, 32, 1.0, p(A), 32, p(A), 32, p(D), 64,
                  p(Cm), 64, None, 0, None)
    C2 = empty((64, 64))
    with pytest.raises(capi.EmberError):   # ldd < N
        capi.call("ember_gemm_f32_add", 0, 1, 64, 64, 32, 1.0, p(A), 32, p(A), 32, p(C2), 32,
                  p(C2), 64, None, 0, None)
    with pytest.raises(capi.EmberError):   # D = C with another row stride
        capi.call("ember_gemm_f32_add", 0, 1, 32, 32, 32, 1.0, p(A), 32, p(A), 32, p(C2), 64,
                  p(C2), 32, None, 0, None)


# ------------------------------------------------------------ embedding
def test_embedding_kat_and_bwd():
    V, H = 7, 5
    w = np.array([[v * 10 + h for h in range(H)] for v in range(V)], np.float32)
    ids = np.array([3, 0, 6, 3], np.int64)
    W, I = dev(w), dev(ids)
    out = empty((4, H))
    call("ember_embedding_fwd", p(I), p(W), p(out), 4, H, V, None)
    assert np.array_equal(host(out), w[ids])
    r = rng(6)
    n, V, H = 4096, 49152, 576
    ids = r.integers(0, 300, n).astype(np.int64)  # many repeats
    dy = r.standard_normal((n, H)).astype(np.float32)
    I, DY = dev(ids), dev(dy)
    DW = empty((V, H))
    call("ember_embedding_bwd", p(I), p(DY), p(DW), n, H, V, 0, None, 0, None)
    got = host(DW)
    assert_close(got[:300], O.embedding_bwd(ids, dy, V)[:300], name="emb dw")
    assert (got[300:] == 0).all()
    DW2 = empty((V, H))
    call("ember_embedding_bwd", p(I), p(DY), p(DW2), n, H, V, 0, None, 0, None)
    assert torch.equal(DW, DW2)
    call("ember_embedding_bwd", p(I), p(DY), p(DW2), n, H, V, 1, None, 0, None)  # accumulate
    assert_close(host(DW2)[:300], 2 * O.embedding_bwd(ids, dy, V)[:300], name="emb accumulate")


def test_embedding_fwd_rows_of_four_columns():
    # The float4 gather (H % 4 == 0), ids outside [0, V) giving zero rows.
    r = rng(23)
    V, H, n = 1000, 2048, 777
    w = r.standard_normal((V, H)).astype(np.float32)
    ids = r.integers(-2, V + 2, n).astype(np.int64)
    out = empty((n, H))
    I, W = dev(ids), dev(w)
    call("ember_embedding_fwd", p(I), p(W), p(out), n, H, V, None)
    valid = (ids >= 0) & (ids < V)
    want = np.where(valid[:, None], w[np.clip(ids, 0, V - 1)], 0.0).astype(np.float32)
    assert np.array_equal(host(out), want)


def _emb_bwd(ids, dy, V, accumulate=0, dw=None, sorted_path=True):
    n, H = dy.shape
    lib = capi.lib()
    wsb = lib.ember_embedding_bwd_workspace_bytes(n, H, V) if sorted_path else 0
    assert (wsb > 0) == sorted_path
    WS = empty((max(wsb // 4, 1),))
    DW = dev(dw) if dw is not None else empty((V, H))
    I, DY = dev(ids), dev(dy)  # held until the call has run (p() keeps only the address)
    call("ember_embedding_bwd", p(I), p(DY), p(DW), n, H, V, accumulate,
         p(WS) if wsb else None, wsb, None)
    torch.cuda.synchronize()
    return DW


@pytest.mark.parametrize("case", ["repeats", "one_id", "mostly_one", "long_runs", "invalid",
                                  "odd_width"])
def test_embedding_bwd_sorted_vs_oracle(case):
    # The sorted-window form: random ids with repeats, a batch of one repeated id
    # (every window continues the same run), 90% one id, runs longer than a
    # window, ids outside [0, V) (skipped), and a row width not a multiple of 4
    # (one column per thread).  Deterministic over repeat calls and equal to
    # the oracle's sums; accumulate adds onto dw.
    r = rng(21)
    V, H = 5000, {"one_id": 2048, "mostly_one": 2048, "odd_width": 30}.get(case, 96)
    n = 32768 if case in ("one_id", "mostly_one") else 3000
    if case in ("repeats", "odd_width"):
        ids = r.integers(0, 300, n)
    elif case == "one_id":
        ids = np.full(n, 17)
    elif case == "mostly_one":
        ids = np.where(r.random(n) < 0.9, 4999, r.integers(0, V, n))
    elif case == "long_runs":
        ids = np.repeat(r.integers(0, V, 20), 150)[:n]
    else:
        ids = r.integers(-3, V + 3, n)
    ids = ids.astype(np.int64)
    dy = r.standard_normal((n, H)).astype(np.float32)
    valid = (ids >= 0) & (ids < V)
    ref = O.embedding_bwd(np.where(valid, ids, 0), dy * valid[:, None], V)
    DW = _emb_bwd(ids, dy, V)
    got = host(DW)
    hit = np.unique(ids[valid])
    assert_close(got[hit], ref[hit], name=f"emb {case}")
    miss = np.setdiff1d(np.arange(V), hit)
    assert (got[miss] == 0).all()
    assert torch.equal(DW, _emb_bwd(ids, dy, V))
    base = r.standard_normal((V, H)).astype(np.float32)
    acc = host(_emb_bwd(ids, dy, V, accumulate=1, dw=base))
    assert_close(acc[hit], base[hit] + ref[hit], name=f"emb {case} accumulate")
    assert np.array_equal(acc[miss], base[miss])
    if case == "repeats":  # the scan form (no workspace) agrees within tolerance
        assert_close(host(_emb_bwd(ids, dy, V, sorted_path=False))[hit], ref[hit], name="scan")


# ---------------------------------------------------------------- AdamW
def test_adamw_vs_oracle():
    r = rng(7)
    n = 100003
    pp, g = r.standard_normal(n).astype(np.float32), r.standard_normal(n).astype(np.float32)
    m, v = (0.1 * r.standard_normal(n)).astype(np.float32), r.random(n).astype(np.float32) * 0.01
    P, G, Mt, Vt = dev(pp), dev(g), dev(m), dev(v)
    lr, b1, b2, eps, wd = 1e-4, 0.9, 0.95, 1e-8, 0.1
    bc1, bc2 = np.float32(1 - 0.9 ** 3), np.float32(1 - 0.95 ** 3)
    call("ember_adamw", p(P), p(G), p(Mt), p(Vt), n, lr, b1, b2, eps, wd, float(bc1), float(bc2), None)
    rp, rm, rv = O.adamw(pp, g, m, v, np.float32(lr), np.float32(b1), np.float32(b2), np.float32(eps),
                         np.float32(wd), bc1, bc2)
    # Per element: rtol 1e-5 plus an absolute floor of 1e-6 * max|ref| for entries that
    # cancel to ~0 (m = b1*m + (1-b1)*g); the reference's own KAT uses 1e-5 absolute
    # on p ~ 1 (tests/test_autograd.cpp:560).
    for got, ref, name in [(P, rp, "p"), (Mt, rm, "m"), (Vt, rv, "v")]:
        err = np.abs(host(got) - ref)
        bound = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max()
        i = int(np.argmax(err - bound))
        assert (err <= bound).all(), (name, i, float(host(got)[i]), float(ref[i]), float(err[i]))


@pytest.mark.parametrize("max_blocks,offset", [(256, 0), (7, 0), (256, 3), (1, 1)])
def test_adamw_bounded_equals_adamw_bitwise(max_blocks, offset):
    # The offloaded optimizer's low-register, bounded-grid update must round
    # exactly like ember_adamw (float4 path), also off a 16-byte boundary.
    r = rng(8)
    n = 70001
    pp, g = r.standard_normal(n + 4).astype(np.float32), r.standard_normal(n + 4).astype(np.float32)
    m, v = (0.1 * r.standard_normal(n + 4)).astype(np.float32), r.random(n + 4).astype(np.float32)
    args = (1e-3, 0.9, 0.95, 1e-8, 0.1, 0.271, 0.1426)
    A = [dev(x) for x in (pp, g, m, v)]
    B = [dev(x) for x in (pp, g, m, v)]
    call("ember_adamw", *[p(t) for t in A], n + 4, *args, None)
    off = 4 * offset
    call("ember_adamw_bounded", *[C.c_void_p(t.data_ptr() + off) for t in B], n, *args,
         max_blocks, None)
    for a, b, name in zip(A, B, ("p", "g", "m", "v")):
        ha, hb = host(a), host(b)
        assert np.array_equal(ha[offset:offset + n], hb[offset:offset + n]), name
        # nothing outside [offset, offset + n) was touched
        assert np.array_equal(hb[:offset], (pp, g, m, v)[("p", "g", "m", "v").index(name)][:offset])
        assert np.array_equal(hb[offset + n:], (pp, g, m, v)[("p", "g", "m", "v").index(name)][offset + n:])


def test_scale_multi_equals_per_tensor_scale():
    # The batched in-place scale of the gradient clip: every tensor (float4
    # and scalar paths, one a float off a 16-byte boundary, one empty) equals
    # ember_scale on it alone, bit for bit.
    r = rng(17)
    arrs = [r.standard_normal(n).astype(np.float32) for n in (4, 9, 1000003, 1, 50_001, 0, 1025)]
    alpha = 0.37
    ts = [dev(a) if a.size else empty((1,)) for a in arrs]
    want = []
    for a in arrs:
        if not a.size:
            want.append(a)
            continue
        t = dev(a)
        call("ember_scale", p(t), alpha, p(t), a.size, None)
        want.append(host(t))
    off = [0, 0, 0, 0, 4, 0, 0]   # the 50001-element one starts a float in
    ptrs = (C.c_void_p * len(ts))(*[t.data_ptr() + o for t, o in zip(ts, off)])
    sizes = (C.c_int64 * len(ts))(*[a.size - (1 if o else 0) for a, o in zip(arrs, off)])
    lib = capi.lib()
    wsb = lib.ember_scale_multi_workspace_bytes(len(ts))
    ws = empty((wsb // 4,))
    call("ember_scale_multi", ptrs, sizes, len(ts), alpha, p(ws), wsb, None)
    for i, (a, t) in enumerate(zip(arrs, ts)):
        if not a.size:
            continue
        got = host(t)
        if off[i]:
            ref = a.copy()
            sub = dev(a[1:])
            call("ember_scale", p(sub), alpha, p(sub), a.size - 1, None)
            ref[1:] = host(sub)
            assert np.array_equal(got, ref), i
        else:
            assert np.array_equal(got, want[i]), i


def test_sumsq_multi():
    r = rng(8)
    arrs = [r.standard_normal(s).astype(np.float32) for s in (4, 9, 16, 1000003, 1)]
    ts = [dev(a) for a in arrs]
    ptrs = (C.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    sizes = (C.c_int64 * len(ts))(*[a.size for a in arrs])
    lib = capi.lib()
    wsb = lib.ember_sumsq_workspace_bytes(len(ts))
    ws, out = empty((wsb // 4,)), empty((1,))
    call("ember_sumsq_multi", ptrs, sizes, len(ts), p(out), p(ws), wsb, None)
    ref = sum(float((a.astype(np.float64) ** 2).sum()) for a in arrs)
    assert abs(host(out)[0] - ref) <= 1e-5 * ref
    # ClipGradNorm KAT: three all-ones grads of 4, 9, 16 elements -> sqrt(29)
    ones = [dev(np.ones(s, np.float32)) for s in (4, 9, 16)]
    ptrs = (C.c_void_p * 3)(*[t.data_ptr() for t in ones])
    sizes = (C.c_int64 * 3)(4, 9, 16)
    call("ember_sumsq_multi", ptrs, sizes, 3, p(out), p(ws), wsb, None)
    assert abs(math.sqrt(host(out)[0]) - math.sqrt(29)) < 1e-5
    # The float4 path over the most workgroups a tensor gets (50M + 1 elements:
    # a ragged tail), and a view one float off a 16-byte boundary (the scalar
    # path); a second call must give the same bits.
    big = r.standard_normal(50_000_001).astype(np.float32)
    base = r.standard_normal(1001).astype(np.float32)
    tb, tbase = dev(big), dev(base)
    ptrs = (C.c_void_p * 2)(tb.data_ptr(), tbase.data_ptr() + 4)
    sizes = (C.c_int64 * 2)(big.size, 1000)
    wsb = lib.ember_sumsq_workspace_bytes(2)
    ws = empty((wsb // 4,))
    call("ember_sumsq_multi", ptrs, sizes, 2, p(out), p(ws), wsb, None)
    first = host(out)[0]
    ref = float((big.astype(np.float64) ** 2).sum() + (base[1:].astype(np.float64) ** 2).sum())
    assert abs(first - ref) <= 1e-5 * ref
    call("ember_sumsq_multi", ptrs, sizes, 2, p(out), p(ws), wsb, None)
    assert host(out)[0] == first


def test_sgd_exact():
    # fma(-lr, g, p): one float32 rounding (float4 path and a ragged tail on
    # the scalar one); gradients of 0 leave p unchanged.
    r = rng(12)
    for n, off in ((1_000_003, 0), (1001, 1)):
        p0 = r.standard_normal(n + off).astype(np.float32)
        g = r.standard_normal(n + off).astype(np.float32)
        g[:7] = 0.0
        P, G = dev(p0), dev(g)
        call("ember_sgd", C.c_void_p(P.data_ptr() + 4 * off), C.c_void_p(G.data_ptr() + 4 * off), n,
             0.01, None)
        lr = np.float32(0.01)
        want = p0.copy()
        want[off:] = fma_f32(np.full(n, -lr, np.float32), g[off:], p0[off:])
        assert np.array_equal(host(P), want)


# ------------------------------------------------------------ attention
@pytest.mark.parametrize("B,T,H,Hk,D", [
    (1, 256, 9, 3, 64),     # c1 block attention (SmolLM2 shape)
    (1, 200, 4, 2, 128),    # ragged T, Qwen3 head_dim
    (2, 130, 2, 2, 64),     # MHA, two batches, ragged
    (1, 1, 2, 1, 128),      # single token
])
def test_attention_fwd_bwd_vs_oracle(B, T, H, Hk, D):
    r = rng(B * T + H + D)
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    do = r.standard_normal((B, T, H, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    Q, K, Vv, DO = dev(q), dev(k), dev(v), dev(do)
    Ot, L = empty((B, T, H, D)), empty((B, H, T))
    call("ember_attn_fwd", p(Q), p(K), p(Vv), p(Ot), p(L), B, T, H, Hk, D, scale, None)
    o_ref, lse_ref = O.attention_fwd(q, k, v, scale)
    assert_close(host(Ot), o_ref, name="attn o")
    assert_close(host(L), lse_ref, name="attn lse")
    lib = capi.lib()
    wsb = lib.ember_attn_bwd_workspace_bytes(B, T, H)
    WS = empty((wsb // 4,))
    DQ, DK, DV = empty((B, T, H, D)), empty((B, T, Hk, D)), empty((B, T, Hk, D))
    call("ember_attn_bwd", p(Q), p(K), p(Vv), p(Ot), p(L), p(DO), p(DQ), p(DK), p(DV), B, T, H, Hk,
         D, scale, p(WS), wsb, None)
    dq_ref, dk_ref, dv_ref = O.attention_bwd(q, k, v, do, scale)
    # at T = 1 dq and dk are exactly 0 in exact arithmetic (softmax of one score);
    # fp32 leaves rounding residue of order 1e-7, hence the absolute floor
    assert_close(host(DQ), dq_ref, name="dq", atol=1e-5)
    assert_close(host(DK), dk_ref, name="dk", atol=1e-5)
    assert_close(host(DV), dv_ref, name="dv")
    # bitwise run-to-run determinism (forward and backward)
    O2, L2 = empty((B, T, H, D)), empty((B, H, T))
    call("ember_attn_fwd", p(Q), p(K), p(Vv), p(O2), p(L2), B, T, H, Hk, D, scale, None)
    DQ2, DK2, DV2 = empty((B, T, H, D)), empty((B, T, Hk, D)), empty((B, T, Hk, D))
    call("ember_attn_bwd", p(Q), p(K), p(Vv), p(Ot), p(L), p(DO), p(DQ2), p(DK2), p(DV2), B, T, H,
         Hk, D, scale, p(WS), wsb, None)
    assert torch.equal(Ot, O2) and torch.equal(L, L2)
    assert torch.equal(DQ, DQ2) and torch.equal(DK, DK2) and torch.equal(DV, DV2)


def _attn_hip(Q, K, Vv, DO, B, T, H, Hk, D, scale, wsb=None):
    """Forward and backward through the C ABI on device tensors (the backward
    with `wsb` bytes of workspace, by default all it can use)."""
    Ot, L = empty((B, T, H, D)), empty((B, H, T))
    call("ember_attn_fwd", p(Q), p(K), p(Vv), p(Ot), p(L), B, T, H, Hk, D, scale, None)
    if wsb is None:
        wsb = capi.lib().ember_attn_bwd_workspace_bytes(B, T, H)
    WS = empty(((wsb + 3) // 4,))
    DQ, DK, DV = empty((B, T, H, D)), empty((B, T, Hk, D)), empty((B, T, Hk, D))
    call("ember_attn_bwd", p(Q), p(K), p(Vv), p(Ot), p(L), p(DO), p(DQ), p(DK), p(DV), B, T, H, Hk,
         D, scale, p(WS), wsb, None)
    return Ot, L, DQ, DK, DV


def _ds_row_floats(T):
    # dS strips of one (batch, head): 64 key rows x (T32 - 64 kb) queries
    T32 = (T + 31) // 32 * 32
    return sum(64 * (T32 - 64 * kb) for kb in range((T + 63) // 64))


@pytest.mark.parametrize("B,T,H,Hk,D", [
    (2, 300, 8, 2, 64),     # 4 KV rows, ragged T (T32 = 320)
    (4, 130, 8, 1, 128),    # 4 KV rows of group 8, D 128
    (1, 200, 32, 8, 64),    # 8 KV rows of group 4 (the c4 head layout)
    (2, 96, 32, 8, 64),     # 16 KV rows: chunks of 8 keep the XCD regrouping
    (1, 700, 4, 2, 128),    # three 256-query dQ tiles: a workgroup takes 2 and 0, one 1 alone
])
def test_attention_bwd_workspace_paths(B, T, H, Hk, D):
    # The backward keeps dS in the workspace when it fits, in chunks of KV rows
    # when only part fits, and recomputes it with the minimum workspace.  dK
    # and dV come from the same arithmetic on every path (bitwise equal); dQ
    # is bitwise equal across chunkings and within tolerance of the oracle on
    # both dQ kernels.
    r = rng(B * 1000 + T + H)
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    do = r.standard_normal((B, T, H, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    lib = capi.lib()
    lo = lib.ember_attn_bwd_workspace_bytes_min(B, T, H)
    hi = lib.ember_attn_bwd_workspace_bytes(B, T, H)
    kv_row = (H // Hk) * _ds_row_floats(T) * 4
    table = (B * H * 8 + 255) // 256 * 256
    assert lo == (B * T * H * 4 + 255) // 256 * 256 + table and hi == lo + B * Hk * kv_row
    assert lib.ember_attn_bwd_ds_row_bytes(T, H, Hk) == kv_row
    Q, K, Vv, DO = dev(q), dev(k), dev(v), dev(do)
    runs = {}
    for name, wsb in [("full", hi), ("one", lo + kv_row), ("three", lo + 3 * kv_row + 100),
                      ("eight", lo + 8 * kv_row), ("min", lo)]:
        _, _, DQ, DK, DV = _attn_hip(Q, K, Vv, DO, B, T, H, Hk, D, scale, wsb)
        runs[name] = (host(DQ), host(DK), host(DV))
    dq_ref, dk_ref, dv_ref = O.attention_bwd(q, k, v, do, scale)
    for name, (dq, dk, dv) in runs.items():
        assert np.array_equal(dk, runs["full"][1]) and np.array_equal(dv, runs["full"][2]), name
        if name != "min":
            assert np.array_equal(dq, runs["full"][0]), name
    for name in ("full", "min"):
        dq, dk, dv = runs[name]
        assert_close(dq, dq_ref, name=f"{name} dq")
        assert_close(dk, dk_ref, name=f"{name} dk")
        assert_close(dv, dv_ref, name=f"{name} dv")


def _bwd_chunk(rows, kv_rows):
    """KV rows per chunk of the attention backward with room for `rows`: the
    chunks as equal as the room allows, multiples of 8 where it holds 8."""
    if rows >= kv_rows:
        return kv_rows
    if rows >= 8:
        rows -= rows % 8
    nch = -(-kv_rows // rows)
    even = -(-kv_rows // nch)
    if rows >= 8:
        even = -(-even // 8) * 8
    return min(even, rows)


@pytest.mark.parametrize("B,T,H,Hk,D,split", [
    (2, 96, 32, 8, 64, [3, 5.5, 0, 8]),   # 16 KV rows over four buffers (one empty)
    (2, 96, 32, 8, 64, [5, 6]),           # 11 rows: chunks cut to 8
    (2, 96, 32, 8, 64, [1, 1, 1]),        # 3 rows: chunks of 3 (the last of 1)
    (2, 96, 32, 8, 64, [3, 2]),           # 5 rows: four equal chunks of 4
    (3, 64, 32, 8, 64, [9, 9]),           # 24 KV rows, 18 fit: chunks of 16 and 8
    (1, 200, 32, 8, 64, [2, 2, 2, 2]),    # all 8 rows, group 4
    (4, 130, 8, 1, 128, [0.5, 2.9]),      # D 128: a buffer too small for a row
])
def test_attention_bwd_scattered_equals_contiguous(B, T, H, Hk, D, split):
    # dS in separate buffers (ember_attn_bwd_scattered) gives dQ, dK and dV
    # bitwise equal to one contiguous workspace with the same rows per chunk,
    # and writes nothing outside the whole rows of each buffer.
    r = rng(B * 77 + T + len(split))
    q, k, v, do = (r.standard_normal(s).astype(np.float32)
                   for s in ((B, T, H, D), (B, T, Hk, D), (B, T, Hk, D), (B, T, H, D)))
    scale = 1.0 / math.sqrt(D)
    lib = capi.lib()
    lo = lib.ember_attn_bwd_workspace_bytes_min(B, T, H)
    row = lib.ember_attn_bwd_ds_row_bytes(T, H, Hk)
    kv_rows = B * Hk
    sizes = [int(f * row) // 256 * 256 if f != int(f) else int(f) * row for f in split]
    rows = sum(s // row for s in sizes)
    chunk = _bwd_chunk(rows, kv_rows)
    Q, K, Vv, DO = dev(q), dev(k), dev(v), dev(do)
    Ot, L, DQc, DKc, DVc = _attn_hip(Q, K, Vv, DO, B, T, H, Hk, D, scale, lo + chunk * row)
    # the buffers: one device allocation, each buffer followed by a guard band
    guard = 4096
    offs, o = [], 0
    for s in sizes:
        offs.append(o)
        o += (s + guard + 255) // 256 * 256
    POOL = torch.full(((o + 3) // 4,), 7.25, device="cuda")
    base = POOL.data_ptr()
    ptrs = (C.c_void_p * len(sizes))(*[base + off if s else None for off, s in zip(offs, sizes)])
    szs = (C.c_size_t * len(sizes))(*sizes)
    WS = empty(((lo + 3) // 4,))
    DQ, DK, DV = empty((B, T, H, D)), empty((B, T, Hk, D)), empty((B, T, Hk, D))
    call("ember_attn_bwd_scattered", p(Q), p(K), p(Vv), p(Ot), p(L), p(DO), p(DQ), p(DK), p(DV),
         B, T, H, Hk, D, scale, p(WS), lo, ptrs, szs, len(sizes), None)
    assert torch.equal(DQ, DQc) and torch.equal(DK, DKc) and torch.equal(DV, DVc)
    pool = host(POOL).view(np.uint8)
    fill = np.frombuffer(np.float32(7.25).tobytes(), np.uint8)
    left = chunk  # row slots are taken in buffer order
    for off, s in zip(offs, sizes):
        used = min(s // row, left)
        left -= used
        tail = pool[off + used * row: off + s + guard]
        assert np.array_equal(tail.reshape(-1, 4), np.broadcast_to(fill, (tail.size // 4, 4)))


def _keep_scores_run(Q, K, Vv, DO, B, T, H, Hk, D, scale, sizes, fill=7.25, guard=4096):
    """ember_attn_fwd_scores then ember_attn_bwd_from_scores over buffers of
    `sizes` bytes carved from one pool, each followed by a guard band."""
    lib = capi.lib()
    offs, o = [], 0
    for s in sizes:
        offs.append(o)
        o += (s + guard + 255) // 256 * 256
    POOL = torch.full(((o + 3) // 4,), fill, device="cuda")
    base = POOL.data_ptr()
    ptrs = (C.c_void_p * len(sizes))(*[base + off if s else None for off, s in zip(offs, sizes)])
    szs = (C.c_size_t * len(sizes))(*sizes)
    tws = lib.ember_attn_scores_workspace_bytes(B, H)
    TW = empty(((tws + 3) // 4,))
    Ot, L = empty((B, T, H, D)), empty((B, H, T))
    call("ember_attn_fwd_scores", p(Q), p(K), p(Vv), p(Ot), p(L), B, T, H, Hk, D, scale, ptrs, szs,
         len(sizes), p(TW), tws, None)
    lo = lib.ember_attn_bwd_workspace_bytes_min(B, T, H)
    WS = empty(((lo + 3) // 4,))
    DQ, DK, DV = empty((B, T, H, D)), empty((B, T, Hk, D)), empty((B, T, Hk, D))
    call("ember_attn_bwd_from_scores", p(Q), p(K), p(Vv), p(Ot), p(L), p(DO), p(DQ), p(DK), p(DV),
         B, T, H, Hk, D, scale, p(WS), lo, ptrs, szs, len(sizes), None)
    return Ot, L, DQ, DK, DV, POOL, offs


@pytest.mark.parametrize("B,T,H,Hk,D,split", [
    (1, 256, 9, 3, 64, [3]),              # c1's heads, one buffer holding every row
    (2, 300, 8, 2, 64, [1, 2.5, 0, 1]),   # ragged T (T32 = 320), rows over several buffers
    (4, 130, 8, 1, 128, [4]),             # group 8, D 128
    (1, 200, 32, 8, 64, [8]),             # group 4 (the c4 head layout)
    (2, 96, 32, 8, 64, [5, 6, 5]),        # 16 KV rows: the XCD regrouping
    (8, 256, 16, 8, 128, [64]),           # the c5 launch layout at T = 256
])
def test_attention_keep_scores(B, T, H, Hk, D, split):
    # The forward that keeps its scores gives o and lse bitwise equal to the
    # plain forward; the backward from them agrees with the oracle to the same
    # tolerance as the recompute path, and with that path to fp32 rounding
    # (S is the forward's rounding of the same products); runs repeat bit for
    # bit; nothing is written past each buffer's whole rows.
    r = rng(B * 131 + T + H)
    q, k, v, do = (r.standard_normal(s).astype(np.float32)
                   for s in ((B, T, H, D), (B, T, Hk, D), (B, T, Hk, D), (B, T, H, D)))
    scale = 1.0 / math.sqrt(D)
    lib = capi.lib()
    row = lib.ember_attn_bwd_ds_row_bytes(T, H, Hk)
    sizes = [int(f * row) // 256 * 256 if f != int(f) else int(f) * row for f in split]
    assert sum(s // row for s in sizes) >= B * Hk
    Q, K, Vv, DO = dev(q), dev(k), dev(v), dev(do)
    Oc, Lc, DQc, DKc, DVc = _attn_hip(Q, K, Vv, DO, B, T, H, Hk, D, scale)
    Ot, L, DQ, DK, DV, POOL, offs = _keep_scores_run(Q, K, Vv, DO, B, T, H, Hk, D, scale, sizes)
    assert torch.equal(Ot, Oc) and torch.equal(L, Lc)
    dq_ref, dk_ref, dv_ref = O.attention_bwd(q, k, v, do, scale)
    assert_close(host(DQ), dq_ref, name="dq (kept scores)")
    assert_close(host(DK), dk_ref, name="dk (kept scores)")
    assert_close(host(DV), dv_ref, name="dv (kept scores)")
    for got, want in ((DQ, DQc), (DK, DKc), (DV, DVc)):
        rel = ((got - want).norm() / want.norm()).item()
        assert rel < 2e-6, rel
    again = _keep_scores_run(Q, K, Vv, DO, B, T, H, Hk, D, scale, sizes)
    for a, b in zip((Ot, L, DQ, DK, DV), again[:5]):
        assert torch.equal(a, b)
    pool = host(POOL).view(np.uint8)
    fill = np.frombuffer(np.float32(7.25).tobytes(), np.uint8)
    left = B * Hk  # row slots are taken in buffer order
    for off, s in zip(offs, sizes):
        used = min(s // row, left)
        left -= used
        tail = pool[off + used * row: off + s + 4096]
        assert np.array_equal(tail.reshape(-1, 4), np.broadcast_to(fill, (tail.size // 4, 4)))


def test_attention_keep_scores_needs_every_row():
    # Buffers that hold fewer KV rows than B*Hk are refused before any launch.
    B, T, H, Hk, D = 2, 128, 8, 2, 64
    lib = capi.lib()
    row = lib.ember_attn_bwd_ds_row_bytes(T, H, Hk)
    Q, K, Vv = dev(np.zeros((B, T, H, D), np.float32)), dev(np.zeros((B, T, Hk, D), np.float32)), \
        dev(np.zeros((B, T, Hk, D), np.float32))
    S = empty(((3 * row) // 4,))
    ptrs = (C.c_void_p * 1)(S.data_ptr())
    szs = (C.c_size_t * 1)(3 * row)
    tws = lib.ember_attn_scores_workspace_bytes(B, H)
    TW = empty(((tws + 3) // 4,))
    Ot, L = empty((B, T, H, D)), empty((B, H, T))
    rc = lib.ember_attn_fwd_scores(p(Q), p(K), p(Vv), p(Ot), p(L), B, T, H, Hk, D, 0.125, ptrs, szs,
                                   1, p(TW), tws, None)
    assert rc == -2, rc  # EMBER_EWORKSPACE
    lo = lib.ember_attn_bwd_workspace_bytes_min(B, T, H)
    WS = empty(((lo + 3) // 4,))
    rc = lib.ember_attn_bwd_from_scores(p(Q), p(K), p(Vv), p(Ot), p(L), p(Q), p(Q), p(K), p(Vv), B,
                                        T, H, Hk, D, 0.125, p(WS), lo, ptrs, szs, 1, None)
    assert rc == -2, rc


# The launch layouts of the BASELINE configs: c3 Qwen3-0.6B (64 (batch, head)
# rows, group 2, D 128), c4 LLaMA-3.2-1B (128 rows, group 4, D 64), c5
# Qwen3-1.7B (128 rows, group 2, D 128).  Row counts that are multiples of 8
# above 8 take the XCD regrouping of the work items, and group 4 takes the
# dK/dV kernel's loop over four query heads per KV head.
REAL_LAYOUTS = [("c3", 4, 1024, 16, 8, 128), ("c4", 4, 2048, 32, 8, 64),
                ("c5", 8, 4096, 16, 8, 128)]


@pytest.mark.parametrize("name,B,T,H,Hk,D", REAL_LAYOUTS)
def test_attention_real_layouts_vs_oracle(name, B, T, H, Hk, D):
    # Every (batch, head) row of the real launch, at T = 256 so the oracle
    # finishes in seconds.
    T = 256
    r = rng({"c3": 31, "c4": 41, "c5": 51}[name])
    q = r.standard_normal((B, T, H, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hk, D)).astype(np.float32)
    do = r.standard_normal((B, T, H, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    Ot, L, DQ, DK, DV = _attn_hip(dev(q), dev(k), dev(v), dev(do), B, T, H, Hk, D, scale)
    o_ref, lse_ref = O.attention_fwd(q, k, v, scale)
    assert_close(host(Ot), o_ref, name=f"{name} o")
    assert_close(host(L), lse_ref, name=f"{name} lse")
    dq_ref, dk_ref, dv_ref = O.attention_bwd(q, k, v, do, scale)
    assert_close(host(DQ), dq_ref, name=f"{name} dq")
    assert_close(host(DK), dk_ref, name=f"{name} dk")
    assert_close(host(DV), dv_ref, name=f"{name} dv")


@pytest.mark.parametrize("name,B,T,H,Hk,D", REAL_LAYOUTS)
def test_attention_real_layouts_full_T_vs_torch(name, B, T, H, Hk, D):
    # The full launch at the config's own B, T and heads against fp32 torch
    # autograd of softmax(Q K^T * scale + causal mask) V on the GPU, one
    # (batch, KV head) group of query heads at a time.
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(B, T, H, D, device="cuda", generator=g)
    k = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    v = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    do = torch.randn(B, T, H, D, device="cuda", generator=g)
    scale = 1.0 / math.sqrt(D)
    Ot, L, DQ, DK, DV = _attn_hip(q, k, v, do, B, T, H, Hk, D, scale)
    # the recompute path (minimum workspace) at the same full size
    _, _, DQm, DKm, DVm = _attn_hip(q, k, v, do, B, T, H, Hk, D, scale,
                                    capi.lib().ember_attn_bwd_workspace_bytes_min(B, T, H))
    assert torch.equal(DK, DKm) and torch.equal(DV, DVm)
    G = H // Hk
    causal = torch.triu(torch.ones(T, T, dtype=torch.bool, device="cuda"), 1)
    refs = {n: torch.empty_like(t) for n, t in (("o", Ot), ("dq", DQ), ("dk", DK), ("dv", DV))}
    ref_lse = torch.empty_like(L)
    for b in range(B):
        for j in range(Hk):
            heads = slice(j * G, (j + 1) * G)
            qg = q[b, :, heads].permute(1, 0, 2).contiguous().requires_grad_(True)  # [G,T,D]
            kj = k[b, :, j].contiguous().requires_grad_(True)
            vj = v[b, :, j].contiguous().requires_grad_(True)
            s = torch.matmul(qg, kj.t().contiguous()) * scale          # [G,T,T]
            s = s.masked_fill(causal, -math.inf)
            og = torch.matmul(torch.softmax(s, -1), vj)
            og.backward(do[b, :, heads].permute(1, 0, 2).contiguous())
            refs["o"][b, :, heads] = og.detach().permute(1, 0, 2)
            refs["dq"][b, :, heads] = qg.grad.permute(1, 0, 2)
            refs["dk"][b, :, j] = kj.grad
            refs["dv"][b, :, j] = vj.grad
            ref_lse[b, heads] = torch.logsumexp(s.detach(), -1)
    torch.cuda.synchronize()
    for n, got in (("o", Ot), ("dq", DQ), ("dk", DK), ("dv", DV), ("dq", DQm)):
        rel = ((got - refs[n]).norm() / refs[n].norm()).item()
        assert rel < 1e-5, (name, n, rel)
        err = (got - refs[n]).abs()
        bound = 1e-4 * refs[n].abs() + 1e-4 * refs[n].abs().max()
        assert bool((err <= bound).all()), (name, n, err.max().item())
    assert (L - ref_lse).abs().max().item() < 1e-4


def test_attention_full_T_c5_vs_torch_sdpa():
    # c5 per-head shape at full T=4096: one batch row, one KV group (2 query heads).
    B, T, H, Hk, D = 1, 4096, 2, 1, 128
    g = torch.Generator(device="cuda").manual_seed(1)
    q = torch.randn(B, T, H, D, device="cuda", generator=g)
    k = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    v = torch.randn(B, T, Hk, D, device="cuda", generator=g)
    o, lse = empty((B, T, H, D)), empty((B, H, T))
    call("ember_attn_fwd", p(q), p(k), p(v), p(o), p(lse), B, T, H, Hk, D, 1 / math.sqrt(D), None)
    # fp32 math reference on the GPU, one head at a time ([T,T] fp32 = 64 MB)
    for h in range(H):
        s = (q[0, :, h] @ k[0, :, 0].t().contiguous()) / math.sqrt(D)
        s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool, device="cuda"), 1), -math.inf)
        ref = torch.softmax(s, -1) @ v[0, :, 0]
        torch.cuda.synchronize()
        rel = ((o[0, :, h] - ref).norm() / ref.norm()).item()
        assert rel < 1e-5, rel
        assert ((lse[0, h] - torch.logsumexp(s, -1)).abs().max()).item() < 1e-4


# ----------------------------------------------------- unfused chain ops
def test_reference_chain_ops_vs_oracle():
    r = rng(9)
    rows, N = 64, 300
    x = (r.standard_normal((rows, N)) * 4).astype(np.float32)
    g = r.standard_normal((rows, N)).astype(np.float32)
    X, G, Y, DX = dev(x), dev(g), empty((rows, N)), empty((rows, N))
    call("ember_softmax_fwd", p(X), p(Y), rows, N, None)
    y = host(Y)
    assert_close(y, O.softmax_fwd(x), name="softmax")
    call("ember_softmax_bwd", p(Y), p(G), p(DX), rows, N, None)
    assert_close(host(DX), O.softmax_bwd(y, g), name="softmax bwd")
    s = np.ones((2, 4, 4), np.float32)
    S = dev(s)
    call("ember_causal_mask", p(S), p(S), 8, 4, 4, 0, -3.4028234663852886e38, None)
    assert np.array_equal(host(S), O.causal_mask(s).astype(np.float32))
    kv = r.standard_normal((2, 5, 3, 16)).astype(np.float32)
    KV, Y = dev(kv), empty((2, 5, 6, 16))
    call("ember_repeat_kv", p(KV), p(Y), 10, 3, 2, 16, None)
    assert np.array_equal(host(Y), O.repeat_kv(kv, 2))
    Z = empty((2, 5, 3, 16))
    call("ember_repeat_kv_sum", p(Y), p(Z), 10, 3, 2, 16, None)
    assert np.array_equal(host(Z), 2 * kv)
    t = np.arange(2 * 3 * 4 * 2, dtype=np.float32).reshape(2, 3, 4, 2)
    Tt, Y = dev(t), empty((2, 4, 3, 2))
    shape = (C.c_int64 * 4)(2, 3, 4, 2)
    perm = (C.c_int * 4)(0, 2, 1, 3)
    call("ember_permute", p(Tt), p(Y), 4, shape, perm, None)
    assert np.array_equal(host(Y), t.transpose(0, 2, 1, 3))


def test_fill_normal_statistics_and_reproducible():
    n = 1 << 22
    a, b = empty((n,)), empty((n,))
    call("ember_fill_normal", p(a), n, 0, 0, 0.0, 0.02, None)
    call("ember_fill_normal", p(b), n, 0, 0, 0.0, 0.02, None)
    assert torch.equal(a, b)
    assert abs(a.mean().item()) < 1e-4 and abs(a.std().item() - 0.02) < 1e-4
