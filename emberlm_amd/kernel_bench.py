"""Per-kernel timings at the benchmark workload's shapes (Qwen3-1.7B, B=8,
T=4096: N = 32768 tokens, hidden 2048, MLP 6144, 16/8 heads of 128, vocab
151936), through the C ABI (include/ember_hip.h) on device buffers from torch.

Each entry launches one C-ABI call `reps` times between two HIP events on the
stream the calls run on (the null stream, which torch's events also use) after
warmup launches, and reports the average launch time and the rate of its
algorithmic work: bytes that must cross HBM for the bandwidth-bound kernels
(each input read once, each output written once), flops for attention.

    python -m emberlm_amd.kernel_bench [--only NAME ...] [--reps R]

prints one JSON line per kernel.  `bench.py --kernels` runs the same table.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import sys

HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3

N, HID, INTER, H, HK, D, V, B, T = 32768, 2048, 6144, 16, 8, 128, 151936, 8, 4096


def _time(fn, reps, warmup=3):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def entries():
    """name -> (setup() returning (launch, algorithmic bytes, flops, shape))."""
    import torch

    from emberlm_amd import capi

    lib = capi.lib()
    P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    f32 = torch.float32

    def rand(*shape):
        return torch.randn(*shape, device="cuda", dtype=f32)

    def ck(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: status {rc}")

    def rmsnorm_fwd():
        x, w, y, r = rand(N, HID), rand(HID), rand(N, HID), rand(N)
        return (lambda: ck(lib.ember_rmsnorm_fwd(P(x), P(w), P(y), P(r), N, HID, 1e-6, None), "rms"),
                8.0 * N * HID, 0.0, f"[{N}, {HID}]")

    def rmsnorm_bwd(acc):
        def setup():
            dy, x, w, r, dx, dw = rand(N, HID), rand(N, HID), rand(HID), rand(N), rand(N, HID), rand(HID)
            wsb = lib.ember_rmsnorm_bwd_workspace_bytes(N, HID)
            ws = torch.empty(wsb // 4 + 1, device="cuda")
            fn = lib.ember_rmsnorm_bwd_accumulate if acc else lib.ember_rmsnorm_bwd
            return (lambda: ck(fn(P(dy), P(x), P(w), P(r), P(dx), P(dw), N, HID, 1e-6, P(ws), wsb,
                                  None), "rms bwd"),
                    (16.0 if acc else 12.0) * N * HID, 0.0, f"[{N}, {HID}]")
        return setup

    def qknorm_rope(bwd):
        def setup():
            rows = N * H
            x, w, y, r = rand(rows, D), rand(D), rand(rows, D), rand(rows)
            fr = (C.c_float * (D // 2))()
            ck(lib.ember_rope_freqs_host(fr, D, 1e6, 0.0, 1.0, 4.0, 8192), "freqs")
            if not bwd:
                return (lambda: ck(lib.ember_qknorm_rope_fwd(P(x), P(w), P(y), P(r), rows, H, T, D,
                                                             1e-6, 0, fr, None), "qkn"),
                        8.0 * rows * D, 0.0, f"q [{rows}, {D}]")
            dy, dx, dw = rand(rows, D), rand(rows, D), rand(D)
            wsb = lib.ember_rmsnorm_bwd_workspace_bytes(rows, D)
            ws = torch.empty(wsb // 4 + 1, device="cuda")
            return (lambda: ck(lib.ember_qknorm_rope_bwd(P(dy), P(x), P(w), P(r), P(dx), P(dw), rows,
                                                         H, T, D, 1e-6, 0, fr, P(ws), wsb, None),
                               "qkn bwd"),
                    12.0 * rows * D, 0.0, f"q [{rows}, {D}]")
        return setup

    def swiglu(bwd):
        def setup():
            n = N * INTER
            g, u, h = rand(n), rand(n), rand(n)
            if not bwd:
                return (lambda: ck(lib.ember_swiglu_fwd(P(g), P(u), P(h), n, None), "swiglu"),
                        12.0 * n, 0.0, f"[{N}, {INTER}]")
            dg, du = rand(n), rand(n)
            return (lambda: ck(lib.ember_swiglu_bwd(P(g), P(u), P(h), P(dg), P(du), n, None), "swiglu b"),
                    20.0 * n, 0.0, f"[{N}, {INTER}]")
        return setup

    def embedding(bwd):
        def setup():
            ids = torch.randint(0, V, (N,), device="cuda", dtype=torch.int64)
            w, out = rand(V, HID), rand(N, HID)
            if not bwd:
                return (lambda: ck(lib.ember_embedding_fwd(P(ids), P(w), P(out), N, HID, V, None), "emb"),
                        8.0 * N * HID, 0.0, f"{N} ids x {HID}")
            wsb = lib.ember_embedding_bwd_workspace_bytes(N, HID, V)
            ws = torch.empty(wsb // 4 + 1, device="cuda")
            # accumulate into an existing dW (the tied head's): dy read once, the
            # touched rows of dW read and written once
            distinct = int(torch.unique(ids).numel())
            return (lambda: ck(lib.ember_embedding_bwd(P(ids), P(out), P(w), N, HID, V, 1, P(ws), wsb,
                                                       None), "emb bwd"),
                    4.0 * N * HID + 8.0 * distinct * HID, 0.0,
                    f"{N} ids ({distinct} distinct) x {HID}, V {V}")
        return setup

    def adamw():
        n = 1 << 24
        p_, g, m, v = rand(n), rand(n), rand(n), rand(n).abs()
        return (lambda: ck(lib.ember_adamw(P(p_), P(g), P(m), P(v), n, 1e-4, 0.9, 0.95, 1e-8, 0.1, 0.5,
                                           0.5, None), "adamw"),
                28.0 * n, 0.0, f"{n}")

    def clip(scale):
        def setup():
            # the Qwen3-1.7B parameter list: embedding, 28 x (11 tensors), final norm
            sizes = [V * HID]
            for _ in range(28):
                sizes += [HID, H * D * HID, HK * D * HID, HK * D * HID, HID * H * D, D, D, HID,
                          INTER * HID, INTER * HID, HID * INTER]
            sizes.append(HID)
            ts = [torch.randn(s, device="cuda") for s in sizes]
            cnt = len(ts)
            ptrs = (C.c_void_p * cnt)(*[t.data_ptr() for t in ts])
            szs = (C.c_int64 * cnt)(*sizes)
            out = torch.empty(1, device="cuda")
            total = float(sum(sizes))
            if not scale:
                wsb = lib.ember_sumsq_workspace_bytes(cnt)
                ws = torch.empty(wsb // 4 + 1, device="cuda")
                return (lambda: ck(lib.ember_sumsq_multi(ptrs, szs, cnt, P(out), P(ws), wsb, None),
                                   "sumsq"), 4.0 * total, 0.0, f"{cnt} tensors")
            wsb = lib.ember_scale_multi_workspace_bytes(cnt)
            ws = torch.empty(wsb // 4 + 1, device="cuda")
            return (lambda: ck(lib.ember_scale_multi(ptrs, szs, cnt, 1.0, P(ws), wsb, None), "scale"),
                    8.0 * total, 0.0, f"{cnt} tensors")
        return setup

    def attention(bwd, ds_rows=None):
        def setup():
            q, k, v = rand(B, T, H, D) * 0.5, rand(B, T, HK, D) * 0.5, rand(B, T, HK, D)
            o, lse = torch.empty(B, T, H, D, device="cuda"), torch.empty(B, H, T, device="cuda")
            scale = 1.0 / math.sqrt(D)
            fwd_flops = 4.0 * B * H * D * (T * (T + 1) / 2)
            run_f = lambda: ck(lib.ember_attn_fwd(P(q), P(k), P(v), P(o), P(lse), B, T, H, HK, D,  # noqa: E731
                                                  scale, None), "attn")
            if not bwd:
                return run_f, 0.0, fwd_flops, f"B{B} T{T} H{H}/{HK} D{D}"
            run_f()
            do = rand(B, T, H, D)
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            lo = lib.ember_attn_bwd_workspace_bytes_min(B, T, H)
            rows = B * HK if ds_rows is None else ds_rows  # KV rows of dS kept per chunk
            wsb = lo + rows * lib.ember_attn_bwd_ds_row_bytes(T, H, HK)
            ws = torch.empty(wsb // 4 + 1, device="cuda")
            return (lambda: ck(lib.ember_attn_bwd(P(q), P(k), P(v), P(o), P(lse), P(do), P(dq), P(dk),
                                                  P(dv), B, T, H, HK, D, scale, P(ws), wsb, None),
                               "attn bwd"),
                    0.0, 2.0 * fwd_flops,
                    f"B{B} T{T} H{H}/{HK} D{D}, dS of {rows} KV rows per chunk ({(wsb - lo) / 1e9:.2f} GB)")
        return setup

    return {
        "rmsnorm_fwd": rmsnorm_fwd, "rmsnorm_bwd": rmsnorm_bwd(False),
        "rmsnorm_bwd_accumulate": rmsnorm_bwd(True), "qknorm_rope_fwd": qknorm_rope(False),
        "qknorm_rope_bwd": qknorm_rope(True), "swiglu_fwd": swiglu(False), "swiglu_bwd": swiglu(True),
        "embedding_fwd": embedding(False), "embedding_bwd": embedding(True), "adamw": adamw,
        "clip_sumsq": clip(False), "clip_scale": clip(True), "attn_fwd": attention(False),
        "attn_bwd": attention(True), "attn_bwd_32_rows": attention(True, 32),
        "attn_bwd_no_ds": attention(True, 0),
    }


def run(only=None, reps=10, out=sys.stdout):
    import torch
    rows = []
    for name, setup in entries().items():
        if only and name not in only:
            continue
        launch, nbytes, flops, shape = setup()
        ms = _time(launch, reps)
        row = {"kernel": name, "shape": shape, "avg_ms": round(ms, 4)}
        if nbytes:
            gbps = nbytes / (ms / 1e3) / 1e9
            row.update(bytes=nbytes, gbps=round(gbps, 1), frac_of_hbm_peak=round(gbps / HBM_PEAK_GBPS, 4))
        if flops:
            tf = flops / (ms / 1e3) / 1e12
            row.update(flops=flops, tflops=round(tf, 2), frac_of_fp32_mfma_peak=round(tf / FP32_MFMA_PEAK_TFLOPS, 4))
        print(json.dumps(row), file=out, flush=True)
        rows.append(row)
        del launch
        torch.cuda.empty_cache()
    return rows


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--only", nargs="*", default=None)
    ap.add_argument("--reps", type=int, default=10)
    a = ap.parse_args()
    run(a.only, a.reps)


if __name__ == "__main__":
    main()
