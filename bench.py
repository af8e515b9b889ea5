#!/usr/bin/env python3
"""Headline benchmark: Qwen3-1.7B-shaped fp32 training step with gradient
checkpointing (block recompute) and AdamW m/v offloaded to pinned host memory,
batch 8 x seq 4096 on one MI355X.

One step = forward_train_masked -> backward (each block recomputed) ->
clip_grad_norm_(1.0) -> offloaded AdamW step -> zero_grad, i.e. the reference's
ctd_train step (tools/ctd_train/main.cpp:348-398), run through the C++ layer
(libctd.so) on the gfx950 kernels (libember_hip.so).  Inputs are seeded
synthetic token ids (uniform in [0,V)) with an assistant-prefix loss mask;
weights ~N(0,0.02), norm weights 1.

Prints ONE JSON line: tokens/s (B*T per second), peak HBM, the GEMM roofline
(HIP events around every GEMM launch of the timed steps) and a CPU baseline
(the reference's scalar fp32 CPU test ops on one host core
measured in full, this workload extrapolated from measured slices).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train tokens/s + peak HBM GB, Qwen3-1.7B recompute+offload seq4096, 1 GPU"
FP32_MFMA_PEAK_TFLOPS = 157.3
PCIE_GEN5_X16_GBPS = 63.0
HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    # name: (preset, B, T, masked)
    "qwen3-1.7b": ("qwen3-1.7b", 8, 4096, True),      # configs[4], the metric's config
    "llama3.2-1b": ("llama3.2-1b", 4, 2048, False),   # configs[3]
    "qwen3-0.6b": ("qwen3-0.6b", 4, 1024, True),      # configs[2]
    "smollm2-135m": ("smollm2-135m", 4, 512, True),   # configs[1]
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _ref_block(rng, d, H, Hk, D, I, qk_norm, norm_std):
    """Block weights ~N(0, 0.02) in float32; norm weights 1, or ~N(0, 0.02)
    too when norm_std."""
    import numpy as np
    n = lambda *sh: (0.02 * rng.standard_normal(sh)).astype(np.float32)  # noqa: E731
    norm = (lambda k: n(k)) if norm_std else (lambda k: np.ones(k, np.float32))
    w = {"input_layernorm": norm(d), "post_attention_layernorm": norm(d),
         "q_proj": n(H * D, d), "k_proj": n(Hk * D, d), "v_proj": n(Hk * D, d),
         "o_proj": n(d, H * D), "gate_proj": n(I, d), "up_proj": n(I, d), "down_proj": n(d, I)}
    if qk_norm:
        w["q_norm"], w["k_norm"] = norm(D), norm(D)
    return w


def cpu_baseline(cfg, B, T):
    """The reference's scalar fp32 CPU ops as its unit tests write them
    (oracle/ref_f32.c: mm_cpu, rms_norm_cpu, softmax_cpu, rope_cpu, silu, the
    AdamW closed form; the backward formulas are that file's scalar restatement
    of the reference kernels), built -O2 and run on one host core.

    1. BASELINE config 0 in full, measured: one SmolLM2-135M block at B=1,
       T=256 forward+backward without and with checkpointing, and one AdamW
       step over its 3.54 M weights.
    2. The benchmark workload, extrapolated from measured slices (a full step
       would take days): one block forward + recompute + backward on s tokens
       at full width (scaled by tokens and layers), one attention head forward
       (twice: forward and recompute) + backward at T_s (scaled by (T/T_s)^2,
       heads, batch and layers), the tied LM head + masked CE on r rows x V_s
       vocabulary rows (scaled by tokens and V), and AdamW over 4 M weights
       (scaled by the parameter count)."""
    import numpy as np
    from oracle import ref_f32 as RF

    rng = np.random.default_rng(0)
    t = time.perf_counter

    # 1. config 0 in full
    c1 = RF.BlockCfg(d=576, H=9, Hk=3, Dh=64, I=1536, eps=1e-5, theta=1e5)
    w1 = _ref_block(rng, 576, 9, 3, 64, 1536, False, True)
    x = rng.standard_normal((256, 576)).astype(np.float32)
    dy = rng.standard_normal((256, 576)).astype(np.float32)
    t0 = t()
    RF.block_fwd_bwd(c1, w1, x, dy, checkpoint=False)
    t_off = t() - t0
    t0 = t()
    _, _, g1 = RF.block_fwd_bwd(c1, w1, x, dy, checkpoint=True)
    t_on = t() - t0
    t0 = t()
    for k, p in w1.items():
        RF.adamw(p, g1[k], np.zeros_like(p), np.zeros_like(p), 1e-4, 0.9, 0.95, 1e-8,
                 0.1 if p.ndim == 2 else 0.0, 1)
    t_adam1 = t() - t0

    # 2. the workload's slices
    d, I, H, Hk, D, V, L = (cfg.hidden_size, cfg.intermediate_size, cfg.num_heads,
                            cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size, cfg.num_layers)
    cb = RF.BlockCfg(d=d, H=H, Hk=Hk, Dh=D, I=I, eps=cfg.rms_norm_eps, theta=cfg.rope_theta)
    wb = _ref_block(rng, d, H, Hk, D, I, bool(cfg.qk_norm), False)
    s = 16
    xs = rng.standard_normal((s, d)).astype(np.float32)
    t0 = t()
    RF.block_fwd_bwd(cb, wb, xs, xs, checkpoint=True)
    t_block = t() - t0
    Ts = 512
    q = rng.standard_normal((Ts, D)).astype(np.float32)
    t0 = t()
    RF.attention_head(q, q, q)
    t_afwd = t() - t0
    t0 = t()
    RF.attention_head(q, q, q, q)
    t_afb = t() - t0
    r, Vs = 2, min(V, 16384)
    hs = rng.standard_normal((r, d)).astype(np.float32)
    E = (0.02 * rng.standard_normal((Vs, d))).astype(np.float32)
    t0 = t()
    RF.lm_head_ce(hs, E, rng.integers(0, Vs, r), np.ones(r, np.float32))
    t_head = t() - t0
    na = 1 << 22
    pa = rng.standard_normal(na).astype(np.float32)
    t0 = t()
    RF.adamw(pa, pa, np.zeros_like(pa), np.zeros_like(pa), 1e-4, 0.9, 0.95, 1e-8, 0.1, 1)
    t_adam = t() - t0
    from emberlm_amd import trainer as TR
    P = TR.param_count(cfg)
    N = B * T
    # the block sample's own attention over s tokens is negligible beside its projections
    step_s = (t_block / s * N * L + (t_afwd + t_afb) * (T / Ts) ** 2 * H * B * L
              + t_head / r * N * (V / Vs) + t_adam * P / na)
    sample_s = t_off + t_on + t_adam1 + t_block + t_afwd + t_afb + t_head + t_adam
    ncpu = os.cpu_count()
    return {
        "value": N / step_s,
        "unit": "tokens/s",
        "cores": 1,
        "cores_of": ncpu,
        "kind": "port",
        "sample": (f"the reference's scalar fp32 CPU test ops (mm_cpu, rms_norm_cpu, softmax_cpu, "
                   f"rope_cpu, silu, AdamW closed form) composed into the block, LM head and "
                   f"AdamW, 1 thread of {ncpu}; value extrapolated to this workload's step from "
                   f"a block fwd+recompute+bwd on {s} tokens ({t_block:.2f}s), one attention head "
                   f"fwd x2 + bwd at T={Ts} ({t_afwd + t_afb:.2f}s, scaled by T^2), the LM head + "
                   f"CE on {r} rows x {Vs} vocab rows ({t_head:.2f}s) and AdamW on {na} weights "
                   f"({t_adam:.3f}s): extrapolated step {step_s:.0f}s; sample {sample_s:.1f}s"),
        "config0_measured": {
            "workload": "one SmolLM2-135M block, B1 T256 (BASELINE configs[0])",
            "fwd_bwd_s": round(t_off, 3),
            "fwd_bwd_checkpoint_s": round(t_on, 3),
            "recompute_overhead": round(t_on / t_off - 1.0, 4),
            "adamw_step_s": round(t_adam1, 4),
            "tokens_per_s_checkpoint_plus_adamw": round(256 / (t_on + t_adam1), 2),
        },
        "cpu_model": _cpu_model(),
        "nproc": ncpu,
    }


def profiled_traffic(workload, variant):
    """HBM bytes per launch of the dominant GEMM from the committed rocprofv3 PMC
    summary of this workload (FETCH_SIZE/WRITE_SIZE scaled by a known-size copy), or None."""
    key = {"NT": "gemm_nt", "NN": "gemm_nn", "TN": "gemm_tn"}.get(variant)
    pdir = os.path.join(ROOT, "profiles")
    if not key or not os.path.isdir(pdir):
        return None, None
    for fn in sorted(os.listdir(pdir)):
        if workload in fn and fn.endswith(".md"):
            for line in open(os.path.join(pdir, fn)):
                parts = line.split()
                if len(parts) == 3 and parts[0] == "TRAFFIC_BYTES_PER_LAUNCH" and parts[1] == key:
                    return float(parts[2]), "profiles/" + fn
    return None, None


def pinned_copy_rates(nbytes=1 << 30):
    """The box's own pinned-memory copy rates in GB/s, over `nbytes` each:
    host->device alone, device->host alone, and both at once on two streams
    (per direction) -- the link ceiling the offloaded step is held to."""
    from emberlm_amd import capi
    lib, ck = capi.lib(), capi.check
    hin, hout, din, dout = (C.c_void_p() for _ in range(4))
    streams = [C.c_void_p(), C.c_void_p()]
    evs = [C.c_void_p() for _ in range(3)]
    ck(lib.ember_host_malloc_pinned(C.byref(hin), nbytes), "pinned alloc")
    ck(lib.ember_host_malloc_pinned(C.byref(hout), nbytes), "pinned alloc")
    ck(lib.ember_device_malloc(C.byref(din), nbytes), "device alloc")
    ck(lib.ember_device_malloc(C.byref(dout), nbytes), "device alloc")
    for s in streams:
        ck(lib.ember_stream_create(C.byref(s)), "stream")
    for e in evs:
        ck(lib.ember_event_create(C.byref(e)), "event")
    h2d = (din, hin, 0)
    d2h = (hout, dout, 1)

    def span(jobs):
        # jobs[i] runs on streams[i], all released by one event on streams[0]
        ck(lib.ember_event_record(evs[0], streams[0]), "record")
        for i, (dst, src, kind) in enumerate(jobs):
            ck(lib.ember_stream_wait_event(streams[i], evs[0]), "wait")
            ck(lib.ember_memcpy_async(dst, src, nbytes, kind, streams[i]), "copy")
            ck(lib.ember_event_record(evs[1 + i], streams[i]), "record")
        ms = 0.0
        for i in range(len(jobs)):
            ck(lib.ember_event_synchronize(evs[1 + i]), "sync")
            t = C.c_float()
            ck(lib.ember_event_elapsed_ms(C.byref(t), evs[0], evs[1 + i]), "elapsed")
            ms = max(ms, t.value)
        return nbytes / (ms / 1e3) / 1e9

    try:
        span([h2d, d2h])  # first touch of the pinned pages, not timed
        return {"bytes": nbytes, "h2d": round(span([h2d]), 2), "d2h": round(span([d2h]), 2),
                "duplex_per_direction": round(span([h2d, d2h]), 2)}
    finally:
        for e in evs:
            lib.ember_event_destroy(e)
        for s in streams:
            lib.ember_stream_destroy(s)
        lib.ember_device_free(din)
        lib.ember_device_free(dout)
        lib.ember_host_free_pinned(hin)
        lib.ember_host_free_pinned(hout)


def link_probe():
    """pinned_copy_rates() in a child process: there its two streams are the
    only ones and get hardware queues of their own, whereas in this process
    they would share queues with the trainer's compute and copy streams and
    the two directions would run one after the other."""
    import subprocess
    try:
        out = subprocess.run([sys.executable, os.path.abspath(__file__), "--link-probe"],
                             capture_output=True, text=True, timeout=180, check=True).stdout
        return json.loads(out.strip().splitlines()[-1])
    except (subprocess.SubprocessError, ValueError, IndexError) as e:
        log(f"[bench] link probe failed: {e}")
        return None


def decode_point(tr, cfg, n_params, prompt_len, new_tokens):
    """ctd_generate's loop (greedy, batch 1) on the benchmark's model: a prompt
    of prompt_len seeded ids, then new_tokens tokens through the KV cache.
    HBM bytes per decoded token: every weight once (the tied embedding as the
    LM head) plus the K/V rows attended to."""
    import numpy as np
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, prompt_len)
    tr.generate(prompt[:8], 4)                         # warm the allocator and kernels
    toks, pf_ms, dc_ms = tr.generate(prompt, new_tokens)
    steps = new_tokens - 1
    ms_tok = dc_ms / steps
    avg_len = prompt_len + new_tokens / 2
    kv_bytes = 2.0 * cfg.num_layers * cfg.num_kv_heads * cfg.head_dim * 4 * avg_len
    bytes_tok = 4.0 * n_params + kv_bytes
    gbps = bytes_tok / (ms_tok / 1e3) / 1e9
    log(f"[bench] decode P={prompt_len}: prefill {pf_ms:.1f} ms, {ms_tok:.3f} ms/token "
        f"({1e3 / ms_tok:.1f} tok/s, {gbps:.0f} GB/s)")
    return {"prompt_tokens": prompt_len, "new_tokens": new_tokens, "sampling": "greedy",
            "prefill_ms": round(pf_ms, 2), "prefill_tokens_per_s": round(prompt_len / pf_ms * 1e3, 1),
            "ms_per_token": round(ms_tok, 4), "tokens_per_s": round(1e3 / ms_tok, 2),
            "hbm_bytes_per_token": bytes_tok, "achieved_gbps": round(gbps, 1),
            "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=15)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="qwen3-1.7b", choices=sorted(WORKLOADS))
    ap.add_argument("--no-checkpointing", action="store_true")
    ap.add_argument("--no-offload", action="store_true")
    ap.add_argument("--nockpt-steps", type=int, default=1,
                    help="extra steps without checkpointing for the recompute overhead and "
                         "the no-checkpoint peak HBM (0 = skip)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="launch one ember_scale over 1 GiB (reads 1 GiB, writes 1 GiB) first: "
                         "the known-size copy that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--max-norm", type=float, default=1.0)
    ap.add_argument("--prefetch-chunks", type=int, default=None,
                    help="cap of the optimizer state the backward stages for the offloaded "
                         "step (library default when omitted; 0 turns it off)")
    ap.add_argument("--decode-tokens", type=int, default=64,
                    help="tokens generated per inference measurement (0: skip)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the inference measurement (greedy ctd_generate loop on the "
                         "workload's model): prints one JSON line with the decode points")
    ap.add_argument("--prefetch-layer", type=int, default=None,
                    help="layer whose re-run in the backward starts that prefetch (-1: none; "
                         "default: the library's estimate for the model and batch)")
    ap.add_argument("--attn-ds-bytes", type=int, default=None,
                    help="device bytes the attention backward may keep dS in (0: recompute it; "
                         "default: the library's)")
    ap.add_argument("--attn-keep-scores", action="store_true",
                    help="the checkpointed re-run's attention forward keeps its scores for the "
                         "backward (ops::set_attention_keep_scores): one product fewer per "
                         "layer for 4.36 GB more live memory at Qwen3-1.7B")
    ap.add_argument("--head-chunk-rows", type=int, default=None,
                    help="rows per chunk of the fused LM head + loss (default: the library's)")
    ap.add_argument("--alloc-history", default=None,
                    help="write the device allocator's history of the timed steps to this file "
                         "(replayable on the host: emberlm_amd.trainer.alloc_replay)")
    ap.add_argument("--kernels", action="store_true",
                    help="only the per-kernel table at this workload's shapes "
                         "(emberlm_amd/kernel_bench.py): one JSON line per kernel")
    ap.add_argument("--link-probe", action="store_true",
                    help="only the pinned host<->device copy rates of this box (one JSON line)")
    args = ap.parse_args()

    if args.link_probe:
        print(json.dumps(pinned_copy_rates()))
        return
    if args.kernels:
        from emberlm_amd import kernel_bench
        kernel_bench.run()
        return

    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported "
                          "(multi-GPU data parallelism is a design note only)"}))
        sys.exit(2)

    from emberlm_amd import trainer as TR

    if args.copy_probe:
        from emberlm_amd import capi
        n = (1 << 30) // 4
        buf = C.c_void_p()
        capi.check(capi.lib().ember_device_malloc(C.byref(buf), 2 * n * 4), "malloc")
        src, dst = buf.value, buf.value + n * 4
        capi.check(capi.lib().ember_fill(src, n, 1.0, None), "fill")
        capi.check(capi.lib().ember_scale(src, 1.0, dst, n, None), "copy probe")
        capi.check(capi.lib().ember_device_synchronize(), "sync")
        capi.check(capi.lib().ember_device_free(buf), "free")
        log("[bench] copy probe: ember_scale over 1 GiB done")

    preset, B, T, masked = WORKLOADS[args.workload]
    cfg = TR.preset(preset)
    if args.decode_only:
        n_params = TR.param_count(cfg)
        tr = TR.Trainer(cfg, seed=0, init_std=0.02, norm_value=1.0)
        points = [decode_point(tr, cfg, n_params, P, max(args.decode_tokens, 2))
                  for P in (128, T)]
        tr.close()
        print(json.dumps({"metric": "decode tokens/s (greedy, batch 1)", "model": preset,
                          "params": n_params, "dtype": "f32", "data": "synthetic prompt ids, "
                          "weights ~N(0,0.02)", "decode": points}), flush=True)
        return
    ckpt = not args.no_checkpointing
    offload = not args.no_offload
    n_params = TR.param_count(cfg)
    log(f"[bench] {args.workload}: {n_params / 1e9:.4f} B params, B={B} T={T}, "
        f"checkpointing={ckpt}, offload={offload}")

    if args.attn_ds_bytes is not None:
        TR.set_attn_ds_bytes(args.attn_ds_bytes)
    if args.attn_keep_scores:
        TR.set_attn_keep_scores(True)
    if args.head_chunk_rows is not None:
        TR.set_head_chunk_rows(args.head_chunk_rows)
    # Device memory in use before the first tensor: the HIP runtime's context
    # and code objects (part of peak_hbm_gb, not of the allocator's figures).
    base_used = TR.memory().device_used
    if args.alloc_history:
        TR.alloc_history_start()   # from the first allocation: setup, warmup and timed steps
    t0 = time.time()
    tr = TR.Trainer(cfg, seed=0, init_std=0.02, norm_value=1.0)
    tr.set_checkpointing(ckpt)
    tr.make_optimizer(lr=1e-4, weight_decay=0.1, beta1=0.9, beta2=0.95, eps=1e-8, offload=offload)
    if args.prefetch_chunks is not None:
        tr.set_prefetch_chunks(args.prefetch_chunks)
    if args.prefetch_layer is not None:
        tr.set_prefetch_layer(args.prefetch_layer)
    tr.synthetic_batch(B, T, seed=0, masked=masked)
    log(f"[bench] setup {time.time() - t0:.1f}s")

    for i in range(args.warmup):
        st = tr.train_step(args.max_norm)
        log(f"[bench] warmup {i}: {st.total_ms:.0f} ms loss {st.loss:.4f}")

    TR.reset_peak_memory()
    TR.gemm_profile(True)
    tr.synchronize()
    times = []
    t_wall = time.perf_counter()
    for i in range(args.steps):
        st = tr.train_step(args.max_norm)
        times.append(st)
        log(f"[bench] step {i}: total {st.total_ms:.0f} ms (fwd {st.forward_ms:.0f}, bwd "
            f"{st.backward_ms:.0f}, clip {st.clip_ms:.0f}, opt {st.optimizer_ms:.0f}, "
            f"opt stream {st.optimizer_stream_ms:.0f}) "
            f"loss {st.loss:.4f}")
    tr.synchronize()
    wall = time.perf_counter() - t_wall
    if args.alloc_history:
        TR.alloc_history_stop(args.alloc_history)
    TR.gemm_profile(False)
    prof = TR.gemm_profile()
    mem = TR.memory()
    # m/v of the leading chunks that the last timed step's backward had already
    # staged on the device (AdamW::prefetch): they cross host->device before
    # the step's transfer window, so that window's rate is the device->host one.
    prefetched = tr.offload_stats()[2] if offload else 0.0
    step_dirs = tr.offload_detail() if offload else None

    ms_step = wall / args.steps * 1e3
    tokens = B * T
    value = tokens / (ms_step / 1e3)
    avg = lambda f: sum(getattr(s, f) for s in times) / len(times)  # noqa: E731
    # The offloaded update runs on its own streams behind the next forward;
    # each step reports the previous step's transfer+update span.
    opt_ms = avg("optimizer_stream_ms") if offload else avg("optimizer_ms")
    bytes_dir = 8.0 * n_params if offload else 0.0
    mask_sum = times[-1].mask_sum

    # Dominant GEMM instantiation (largest summed time) for the roofline line.
    kname = {"NT": "gemm_f32_dma<A K-contig, B K-contig> (Linear forward, NT)",
             "NN": "gemm_f32_dma<A K-contig, B N-contig> (dX, NN)",
             "TN": "gemm_f32_dma<A M-contig, B N-contig> (dW, TN)",
             "TT": "gemm_f32_dma<A M-contig, B K-contig> (TT)"}
    attn = {k: prof.pop(k) for k in ("attn_fwd", "attn_bwd")}
    # Executed over algorithmic backward flops: 5/4 when dS is kept between the
    # dK/dV and dQ passes (S recomputed), 7/4 when the dQ pass recomputes S, dP.
    # executed / algorithmic work of the attention backward: S again (1.25), S
    # and dP again in the dQ pass too (1.75), or nothing again (kept scores)
    bwd_exec = 1.0 if args.attn_keep_scores else 1.75 if args.attn_ds_bytes == 0 else 1.25
    dom = max(prof, key=lambda k: prof[k].total_ms)
    p = prof[dom]
    per_launch_flops = p.flops / max(p.launches, 1)
    avg_ms = p.total_ms / max(p.launches, 1)
    achieved = per_launch_flops / (avg_ms / 1e3) / 1e12 if avg_ms > 0 else 0.0
    all_fl = sum(v.flops for v in prof.values())
    all_ms = sum(v.total_ms for v in prof.values())

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded uniform token ids, assistant-prefix loss mask (20-60% of each "
                "row), weights ~N(0,0.02), norm weights 1",
        "config": {"workload": f"{args.workload} B{B} T{T} "
                               f"{'recompute' if ckpt else 'no-recompute'}"
                               f"{'+offload' if offload else ''}",
                   "batch": B, "seq_len": T, "parallelism": "none (1 GPU)",
                   "gradient_checkpointing": ckpt, "offload_optimizer": offload,
                   "params": n_params,
                   **({"attention_keeps_scores": True} if args.attn_keep_scores else {})},
        # The device memory the process holds (hipMemGetInfo total - free, peak
        # of the samples taken at every segment the allocator obtains and at
        # each step's phase boundaries), then the allocator's own figures: the
        # live-tensor high-water mark and the bytes it held from the driver.
        "peak_hbm_gb": round(mem.peak_device_used / 1e9, 3),
        "peak_hbm_live_gb": round(mem.peak_allocated / 1e9, 3),
        "peak_hbm_reserved_gb": round(mem.peak_reserved / 1e9, 3),
        "hbm_device_used_gb": round(mem.device_used / 1e9, 3),
        "hbm_runtime_gb": round(base_used / 1e9, 3),
        "allocator": {"reserved_over_live": round(mem.peak_reserved / max(mem.peak_allocated, 1), 4),
                      "segments_obtained": int(mem.device_mallocs),
                      "cache_flushes": int(mem.cache_flushes)},
        "pinned_host_gb": round(mem.pinned_host / 1e9, 3),
        "active_tokens_per_s": round(mask_sum / (ms_step / 1e3), 2),
        # The fused LM head + loss computes only rows whose mask value is
        # nonzero (the rest add nothing to the loss or any gradient).
        "lm_head_rows": {"computed": int(mask_sum), "of": B * T},
        "phase_ms": {k: round(avg(k + "_ms"), 2) for k in
                     ("forward", "backward", "clip", "optimizer", "optimizer_stream")},
        "loss": round(times[-1].loss, 5),
        "offload": {"bytes_per_direction": bytes_dir,
                    "optimizer_stream_ms": round(opt_ms, 2) if offload else None,
                    "optimizer_phase_gbps_per_direction":
                        round(bytes_dir / (opt_ms / 1e3) / 1e9, 2) if offload and opt_ms > 0 else None,
                    "overlapped_with_next_forward": bool(offload),
                    "prefetched_bytes_per_direction": prefetched,
                    "pcie_gen5_x16_gbps": PCIE_GEN5_X16_GBPS},
        # Each direction over its own active window in the last timed step's
        # offloaded update (running beside the next forward): copies in from
        # the first to the last, copies out (with the updates between them)
        # from the first to the last.
        "gemm_all": {"launches": sum(v.launches for v in prof.values()),
                     "tflops": round(all_fl / (all_ms / 1e3) / 1e12, 2) if all_ms else None,
                     "frac_of_fp32_mfma_peak":
                         round(all_fl / (all_ms / 1e3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)
                         if all_ms else None,
                     "ms_per_step": round(all_ms / args.steps, 2)},
        "attention": {
            k: {"launches": a.launches, "ms_per_step": round(a.total_ms / args.steps, 2),
                "avg_launch_ms": round(a.total_ms / max(a.launches, 1), 4),
                "tflops": round(a.flops / (a.total_ms / 1e3) / 1e12, 2) if a.total_ms else None,
                "frac_of_fp32_mfma_peak":
                    round(a.flops / (a.total_ms / 1e3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)
                    if a.total_ms else None,
                "executed_tflops": round(a.flops * (1.0 if k == "attn_fwd" else bwd_exec)
                                         / (a.total_ms / 1e3) / 1e12, 2) if a.total_ms else None}
            for k, a in attn.items()},
        "roofline": {"kernel": kname[dom], "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "launches": p.launches, "avg_launch_ms": round(avg_ms, 4),
                     "flops_per_launch": per_launch_flops, "traffic": None},
    }
    if step_dirs is not None:
        gb = lambda b, ms: round(b / (ms / 1e3) / 1e9, 2) if ms > 0 else None  # noqa: E731
        result["offload"]["in_step"] = {
            "h2d_bytes": step_dirs.h2d_bytes, "h2d_ms": round(step_dirs.h2d_ms, 2),
            "h2d_gbps": gb(step_dirs.h2d_bytes, step_dirs.h2d_ms),
            "d2h_bytes": step_dirs.d2h_bytes, "d2h_ms": round(step_dirs.d2h_ms, 2),
            "d2h_gbps": gb(step_dirs.d2h_bytes, step_dirs.d2h_ms),
            "h2d_frac_of_pcie": round(gb(step_dirs.h2d_bytes, step_dirs.h2d_ms) /
                                      PCIE_GEN5_X16_GBPS, 4) if step_dirs.h2d_ms > 0 else None,
            "d2h_frac_of_pcie": round(gb(step_dirs.d2h_bytes, step_dirs.d2h_ms) /
                                      PCIE_GEN5_X16_GBPS, 4) if step_dirs.d2h_ms > 0 else None,
            "skipped_bytes_no_grad": step_dirs.skipped_bytes}
    traffic, src = profiled_traffic(args.workload, dom)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic
        result["roofline"]["traffic_source"] = src

    if offload:
        # The same offloaded step with nothing running beside it: the link rate
        # the transfer pipeline reaches on its own.
        tr.forward_backward(True)
        tr.clip(args.max_norm)
        tr.synchronize()
        tr.opt_step()
        tr.zero_grad()
        iso_ms, iso_bytes, _ = tr.offload_stats()
        iso = tr.offload_detail()
        gbps = iso_bytes / (iso_ms / 1e3) / 1e9 if iso_ms > 0 else 0.0
        result["offload"]["isolated_h2d_gbps"] = round(
            iso.h2d_bytes / (iso.h2d_ms / 1e3) / 1e9, 2) if iso.h2d_ms > 0 else None
        result["offload"]["isolated_d2h_gbps"] = round(
            iso.d2h_bytes / (iso.d2h_ms / 1e3) / 1e9, 2) if iso.d2h_ms > 0 else None
        result["offload"]["isolated_step_ms"] = round(iso_ms, 2)
        result["offload"]["isolated_gbps_per_direction"] = round(gbps, 2)
        result["offload"]["isolated_frac_of_pcie"] = round(gbps / PCIE_GEN5_X16_GBPS, 4)
        result["offload"]["isolated_aggregate_gbps"] = round(2 * gbps, 2)
        link = link_probe()
        if link is not None:
            result["offload"]["box_pinned_copy_gbps"] = link
            result["offload"]["isolated_frac_of_box_duplex"] = round(
                gbps / link["duplex_per_direction"], 4)
        log(f"[bench] pinned copies on this box: {link}")
        log(f"[bench] isolated offloaded step: {iso_ms:.0f} ms, {gbps:.1f} GB/s per direction")

    if args.nockpt_steps > 0 and ckpt:
        # without checkpointing every layer's scores would stay until its backward
        TR.set_attn_keep_scores(False)
        tr.set_checkpointing(False)
        st = tr.train_step(args.max_norm)  # warm the allocator for the larger footprint
        TR.reset_peak_memory()
        nts = [tr.train_step(args.max_norm) for _ in range(args.nockpt_steps)]
        mem2 = TR.memory()
        base = sum(s.total_ms for s in nts) / len(nts)
        fb = sum(s.forward_ms + s.backward_ms for s in nts) / len(nts)
        fb_ck = avg("forward_ms") + avg("backward_ms")
        result["no_checkpointing"] = {
            "ms_per_step": round(base, 2),
            "peak_hbm_gb": round(mem2.peak_device_used / 1e9, 3),
            "peak_hbm_live_gb": round(mem2.peak_allocated / 1e9, 3),
            "peak_hbm_reserved_gb": round(mem2.peak_reserved / 1e9, 3),
            "recompute_overhead_step": round(avg("total_ms") / base - 1.0, 4),
            "recompute_overhead_fwd_bwd": round(fb_ck / fb - 1.0, 4),
        }
        tr.set_checkpointing(True)
    if args.decode_tokens > 1:
        result["decode"] = [decode_point(tr, cfg, n_params, P, args.decode_tokens)
                            for P in (128, T)]
    tr.close()

    if not args.skip_cpu:
        t0 = time.time()
        result["cpu_baseline"] = cpu_baseline(cfg, B, T)
        log(f"[bench] cpu baseline {time.time() - t0:.1f}s")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
