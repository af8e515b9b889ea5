"""ctypes front end of include/ctd_capi.h (libctd.so): the C++ Model/AdamW layer.

Used by bench.py and the model-level parity tests.  The library is loaded from
emberlm_amd/lib/ and there is no fallback: a missing build raises.
"""
from __future__ import annotations

import ctypes as C
import math
import os

import numpy as np

from . import capi

LIB_PATH = os.path.join(capi.LIB_DIR, "libctd.so")


class ModelConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32), ("intermediate_size", C.c_int32),
        ("num_layers", C.c_int32), ("num_heads", C.c_int32), ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("qk_norm", C.c_int32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("rope_factor", C.c_float),
        ("rope_low_freq_factor", C.c_float), ("rope_high_freq_factor", C.c_float),
        ("rope_original_max_pos", C.c_int32),
    ]


class StepTimes(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("forward_ms", "backward_ms", "clip_ms", "optimizer_ms",
                                         "total_ms", "loss", "grad_norm", "mask_sum",
                                         "optimizer_stream_ms")]


class Memory(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("allocated", "peak_allocated", "reserved",
                                          "peak_reserved", "pinned_host", "device_used",
                                          "device_total", "peak_device_used", "device_mallocs",
                                          "cache_flushes", "limit")]


class OffloadDetail(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("stream_ms", "h2d_ms", "d2h_ms", "h2d_bytes",
                                          "d2h_bytes", "prefetch_bytes", "skipped_bytes")]


class AllocReplay(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("peak_allocated", "peak_reserved", "reserved_end",
                                          "segments_obtained", "cache_flushes")]


class GemmProfile(C.Structure):
    _fields_ = [("launches", C.c_int64), ("flops", C.c_double), ("total_ms", C.c_double)]


_lib = None
vp, i64, i32, f32, u64 = C.c_void_p, C.c_int64, C.c_int32, C.c_float, C.c_uint64
fptr = C.POINTER(C.c_float)
lptr = C.POINTER(C.c_int64)

_SIGS = {
    "ctd_last_error": (C.c_char_p, []),
    "ctd_preset_config": (i32, [C.c_char_p, C.POINTER(ModelConfig)]),
    "ctd_trainer_create": (i32, [C.POINTER(ModelConfig), u64, f32, f32, C.POINTER(vp)]),
    "ctd_trainer_destroy": (i32, [vp]),
    "ctd_trainer_num_params": (i32, [vp, lptr]),
    "ctd_trainer_param_info": (i32, [vp, i64, C.c_char_p, C.c_size_t, lptr, C.POINTER(i32)]),
    "ctd_trainer_set_param": (i32, [vp, i64, fptr, i64]),
    "ctd_trainer_get_param": (i32, [vp, i64, fptr, i64]),
    "ctd_trainer_get_grad": (i32, [vp, i64, fptr, i64]),
    "ctd_trainer_set_checkpointing": (i32, [vp, i32]),
    "ctd_trainer_set_batch": (i32, [vp, lptr, lptr, fptr, i64, i64]),
    "ctd_trainer_synthetic_batch": (i32, [vp, i64, i64, u64, i32]),
    "ctd_trainer_forward_backward": (i32, [vp, i32, fptr]),
    "ctd_trainer_hidden": (i32, [vp, fptr, i64]),
    "ctd_trainer_block_step": (i32, [vp, i64, fptr, fptr, i64, i64, i32, fptr, fptr]),
    "ctd_trainer_make_optimizer": (i32, [vp, f32, f32, f32, f32, f32, i32, i64]),
    "ctd_trainer_clip": (i32, [vp, f32, fptr]),
    "ctd_trainer_opt_step": (i32, [vp]),
    "ctd_trainer_zero_grad": (i32, [vp]),
    "ctd_trainer_get_opt_state": (i32, [vp, i64, fptr, fptr, i64]),
    "ctd_trainer_step_count": (i32, [vp, lptr]),
    "ctd_trainer_offload_stats": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                        C.POINTER(C.c_double)]),
    "ctd_trainer_set_prefetch_chunks": (i32, [vp, i64]),
    "ctd_trainer_offload_detail": (i32, [vp, C.POINTER(OffloadDetail)]),
    "ctd_trainer_set_prefetch_layer": (i32, [vp, i32]),
    "ctd_trainer_train_step": (i32, [vp, f32, C.POINTER(StepTimes)]),
    "ctd_trainer_synchronize": (i32, [vp]),
    "ctd_memory_stats": (i32, [C.POINTER(Memory)]),
    "ctd_reset_peak_memory": (i32, []),
    "ctd_set_device_memory_limit": (i32, [u64]),
    "ctd_empty_device_cache": (i32, []),
    "ctd_alloc_history_start": (i32, []),
    "ctd_alloc_history_mark": (i32, [C.c_char_p]),
    "ctd_alloc_history_stop": (i32, [C.c_char_p]),
    "ctd_alloc_replay": (i32, [C.c_char_p, u64, C.POINTER(AllocReplay)]),
    "ctd_gemm_profile_enable": (i32, [i32]),
    "ctd_gemm_profile_collect": (i32, [C.POINTER(GemmProfile)]),
    "ctd_trainer_save": (i32, [vp, C.c_char_p]),
    "ctd_trainer_load": (i32, [vp, C.c_char_p]),
    "ctd_trainer_accumulate": (i32, [vp, f32, fptr]),
    "ctd_trainer_set_lr": (i32, [vp, f32]),
    "ctd_train_run": (i32, [C.c_char_p]),
    "ctd_train_lr_at_step": (i32, [i32, i32, i32, f32, f32, fptr]),
    "ctd_train_host_batch": (i32, [C.c_char_p, C.c_char_p, i32, lptr, i64, lptr, lptr, fptr, fptr,
                                   lptr]),
    "ctd_train_event_json": (i32, [i32, f32, f32, f32, C.c_double, C.c_double, i32, C.c_char_p,
                                   C.c_size_t]),
    "ctd_kvcache_create": (i32, [vp, i64, i64, C.POINTER(vp)]),
    "ctd_kvcache_destroy": (i32, [vp]),
    "ctd_kvcache_len": (i32, [vp, lptr]),
    "ctd_trainer_forward_cached": (i32, [vp, vp, lptr, i64, i64, i32, i32, fptr, i64]),
    "ctd_sample": (i32, [fptr, i64, i64, f32, i32, f32, u64, i32, i32, lptr]),
    "ctd_set_head_chunk_rows": (i32, [i64]),
    "ctd_set_head_active_rows": (i32, [i32]),
    "ctd_set_attn_ds_bytes": (i32, [i64]),
    "ctd_set_attn_keep_scores": (i32, [i32]),
    "ctd_trainer_generate": (i32, [vp, lptr, i64, i32, f32, i32, f32, u64, i64, lptr,
                                   C.POINTER(C.c_double), C.POINTER(C.c_double)]),
}


class CtdError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        capi.lib()  # the kernel library first (libctd links against it)
        if not os.path.exists(LIB_PATH):
            raise CtdError(f"{LIB_PATH} is missing: run `python -m emberlm_amd.build` first")
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _ck(rc, what):
    if rc != 0:
        raise CtdError(f"{what}: {lib().ctd_last_error().decode()} (status {rc})")


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(fptr)


def preset(name: str) -> ModelConfig:
    c = ModelConfig()
    _ck(lib().ctd_preset_config(name.encode(), C.byref(c)), "preset")
    return c


def make_config(**kw) -> ModelConfig:
    c = ModelConfig()
    d = dict(qk_norm=0, rms_norm_eps=1e-5, rope_theta=1e4, rope_factor=0.0,
             rope_low_freq_factor=1.0, rope_high_freq_factor=4.0, rope_original_max_pos=8192)
    d.update(kw)
    for k, v in d.items():
        setattr(c, k, v)
    return c


def memory() -> Memory:
    m = Memory()
    _ck(lib().ctd_memory_stats(C.byref(m)), "memory")
    return m


def reset_peak_memory():
    _ck(lib().ctd_reset_peak_memory(), "reset_peak_memory")


def set_memory_limit(nbytes: int):
    """Caps the bytes the device allocator holds (0: no cap)."""
    _ck(lib().ctd_set_device_memory_limit(int(nbytes)), "set_memory_limit")


def empty_cache():
    _ck(lib().ctd_empty_device_cache(), "empty_cache")


def alloc_history_start():
    _ck(lib().ctd_alloc_history_start(), "alloc_history_start")


def alloc_history_stop(path: str):
    _ck(lib().ctd_alloc_history_stop(str(path).encode()), "alloc_history_stop")


def alloc_replay(path: str, limit: int = 0) -> AllocReplay:
    """Replays a recorded allocation history on the allocator's placement
    policy (host only, no GPU)."""
    r = AllocReplay()
    _ck(lib().ctd_alloc_replay(str(path).encode(), int(limit), C.byref(r)), "alloc_replay")
    return r


def gemm_profile(enable=None):
    if enable is not None:
        _ck(lib().ctd_gemm_profile_enable(int(enable)), "gemm_profile_enable")
        return None
    g = (GemmProfile * 6)()
    _ck(lib().ctd_gemm_profile_collect(g), "gemm_profile_collect")
    return {name: g[i] for i, name in enumerate(("NN", "NT", "TN", "TT", "attn_fwd", "attn_bwd"))}


class Trainer:
    """Model + AdamW on the GPU (C++ layer), seeded synthetic weights."""

    def __init__(self, cfg: ModelConfig, seed=0, init_std=0.02, norm_value=1.0):
        self.cfg = cfg
        h = vp()
        _ck(lib().ctd_trainer_create(C.byref(cfg), seed, init_std,
                                     float("nan") if norm_value is None else norm_value,
                                     C.byref(h)), "create")
        self.h = h
        n = C.c_int64()
        _ck(lib().ctd_trainer_num_params(h, C.byref(n)), "num_params")
        self.names, self.numels, self.decay = [], [], []
        buf = C.create_string_buffer(256)
        for i in range(n.value):
            ne, dc = C.c_int64(), C.c_int32()
            _ck(lib().ctd_trainer_param_info(h, i, buf, 256, C.byref(ne), C.byref(dc)), "info")
            self.names.append(buf.value.decode())
            self.numels.append(ne.value)
            self.decay.append(bool(dc.value))

    def close(self):
        if self.h:
            _ck(lib().ctd_trainer_destroy(self.h), "destroy")
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_param(self, i, arr):
        a, p = _f32(arr)
        _ck(lib().ctd_trainer_set_param(self.h, i, p, a.size), "set_param")

    def get_param(self, i):
        out = np.empty(self.numels[i], np.float32)
        _ck(lib().ctd_trainer_get_param(self.h, i, out.ctypes.data_as(fptr), out.size), "get_param")
        return out

    def get_grad(self, i):
        out = np.empty(self.numels[i], np.float32)
        rc = lib().ctd_trainer_get_grad(self.h, i, out.ctypes.data_as(fptr), out.size)
        if rc == -1:
            return None
        _ck(rc, "get_grad")
        return out

    def set_checkpointing(self, on):
        _ck(lib().ctd_trainer_set_checkpointing(self.h, int(on)), "set_checkpointing")

    def set_batch(self, ids, targets, mask=None):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        tg = np.ascontiguousarray(targets, dtype=np.int64)
        B, T = ids.shape
        mp = None
        if mask is not None:
            m, mp = _f32(mask)
            self._mask_keep = m
        _ck(lib().ctd_trainer_set_batch(self.h, ids.ctypes.data_as(lptr), tg.ctypes.data_as(lptr),
                                        mp, B, T), "set_batch")

    def synthetic_batch(self, B, T, seed=0, masked=True):
        _ck(lib().ctd_trainer_synthetic_batch(self.h, B, T, seed, int(masked)), "synthetic_batch")

    def forward_backward(self, backward=True):
        loss = C.c_float()
        _ck(lib().ctd_trainer_forward_backward(self.h, int(backward), C.byref(loss)), "fwd/bwd")
        return loss.value

    def block_step(self, layer, x, dy, checkpoint=False):
        x, px = _f32(x)
        dy, pdy = _f32(dy)
        B, T, d = x.shape
        y = np.empty_like(x)
        dx = np.empty_like(x)
        _ck(lib().ctd_trainer_block_step(self.h, layer, px, pdy, B, T, int(checkpoint),
                                         y.ctypes.data_as(fptr), dx.ctypes.data_as(fptr)),
            "block_step")
        return y, dx

    def make_optimizer(self, lr=1e-4, weight_decay=0.1, beta1=0.9, beta2=0.95, eps=1e-8,
                       offload=False, chunk_elems=0):
        _ck(lib().ctd_trainer_make_optimizer(self.h, lr, weight_decay, beta1, beta2, eps,
                                             int(offload), chunk_elems), "make_optimizer")

    def clip(self, max_norm):
        n = C.c_float()
        _ck(lib().ctd_trainer_clip(self.h, max_norm, C.byref(n)), "clip")
        return n.value

    def opt_step(self):
        _ck(lib().ctd_trainer_opt_step(self.h), "opt_step")

    def zero_grad(self):
        _ck(lib().ctd_trainer_zero_grad(self.h), "zero_grad")

    def opt_state(self, i):
        m = np.empty(self.numels[i], np.float32)
        v = np.empty(self.numels[i], np.float32)
        _ck(lib().ctd_trainer_get_opt_state(self.h, i, m.ctypes.data_as(fptr),
                                            v.ctypes.data_as(fptr), m.size), "opt_state")
        return m, v

    def accumulate(self, scale):
        """Forward + backward of loss * scale, gradients accumulating; returns the loss."""
        loss = C.c_float()
        _ck(lib().ctd_trainer_accumulate(self.h, scale, C.byref(loss)), "accumulate")
        return loss.value

    def set_lr(self, lr):
        _ck(lib().ctd_trainer_set_lr(self.h, lr), "set_lr")

    def train_step(self, max_norm=1.0) -> StepTimes:
        t = StepTimes()
        _ck(lib().ctd_trainer_train_step(self.h, max_norm, C.byref(t)), "train_step")
        return t

    def offload_stats(self):
        """(stream_ms, bytes_per_direction, prefetched_bytes) of the last offloaded
        step, after it finished: its device time from first copy in to last copy
        out, the m/v bytes it moved per direction, and how many of those a
        prefetch during train_step's backward had copied in before the step."""
        ms, b, pf = C.c_double(), C.c_double(), C.c_double()
        _ck(lib().ctd_trainer_offload_stats(self.h, C.byref(ms), C.byref(b), C.byref(pf)),
            "offload_stats")
        return ms.value, b.value, pf.value

    def offload_detail(self) -> OffloadDetail:
        """Per-direction device times and bytes of the last finished offloaded step."""
        d = OffloadDetail()
        _ck(lib().ctd_trainer_offload_detail(self.h, C.byref(d)), "offload_detail")
        return d

    def set_prefetch_chunks(self, chunks):
        """Cap (in optimizer-state chunks) of the m/v that train_step's backward
        stages on the device for the offloaded step; 0 turns it off."""
        _ck(lib().ctd_trainer_set_prefetch_chunks(self.h, int(chunks)), "set_prefetch_chunks")

    def set_prefetch_layer(self, layer):
        """Layer whose re-run in train_step's backward starts the prefetch:
        an index, -1 for none, -2 (default) for the estimate from the model
        and batch."""
        _ck(lib().ctd_trainer_set_prefetch_layer(self.h, int(layer)), "set_prefetch_layer")

    def synchronize(self):
        _ck(lib().ctd_trainer_synchronize(self.h), "synchronize")

    def save(self, path):
        _ck(lib().ctd_trainer_save(self.h, str(path).encode()), "save")

    def load(self, path):
        _ck(lib().ctd_trainer_load(self.h, str(path).encode()), "load")

    def num_params(self):
        return len(self.names)

    def generate(self, prompt, max_new, temperature=0.0, top_k=0, top_p=0.0, seed=0,
                 max_seq=None):
        """ctd_generate's loop (batch 1): (tokens, prefill_ms, decode_ms)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int64)
        toks = np.zeros(max_new, np.int64)
        pf, dc = C.c_double(), C.c_double()
        _ck(lib().ctd_trainer_generate(self.h, prompt.ctypes.data_as(lptr), prompt.size, max_new,
                                       temperature, top_k, top_p, seed,
                                       max_seq or prompt.size + max_new,
                                       toks.ctypes.data_as(lptr), C.byref(pf), C.byref(dc)),
            "generate")
        return toks, pf.value, dc.value

    def kv_cache(self, batch, max_seq):
        return KVCache(self, batch, max_seq)

    def forward(self, ids, cache=None, position_start=0, last_only=False):
        """Model::forward (or forward_last_logits) of host int64 ids [B,T] -> logits."""
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        B, T = ids.shape
        out = np.empty((B, 1 if last_only else T, self.cfg.vocab_size), np.float32)
        _ck(lib().ctd_trainer_forward_cached(self.h, cache.h if cache is not None else None,
                                             ids.ctypes.data_as(lptr), B, T, position_start,
                                             int(last_only), out.ctypes.data_as(fptr), out.size),
            "forward")
        return out


class KVCache:
    """nn::KVCache for a trainer's model (zero-filled, batch x max_seq rows)."""

    def __init__(self, tr: Trainer, batch, max_seq):
        h = vp()
        _ck(lib().ctd_kvcache_create(tr.h, batch, max_seq, C.byref(h)), "kv_cache")
        self.h = h

    @property
    def current_len(self):
        n = C.c_int64()
        _ck(lib().ctd_kvcache_len(self.h, C.byref(n)), "kv_cache_len")
        return n.value

    def close(self):
        if self.h:
            _ck(lib().ctd_kvcache_destroy(self.h), "kv_cache_destroy")
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample(logits, temperature=1.0, top_k=0, top_p=0.0, seed=0, draws=1, on_device=False):
    """ctd::sample over host logits [B, V]: `draws` consecutive draws from one
    mt19937_64(seed) -> int64 [draws, B]."""
    x, p = _f32(logits)
    B, V = x.shape
    out = np.zeros((draws, B), np.int64)
    _ck(lib().ctd_sample(p, B, V, temperature, top_k, top_p, seed, draws, int(on_device),
                         out.ctypes.data_as(lptr)), "sample")
    return out


def set_attn_ds_bytes(nbytes):
    """Device bytes the attention backward may keep dS in (-1 default, 0 none)."""
    _ck(lib().ctd_set_attn_ds_bytes(int(nbytes)), "set_attn_ds_bytes")


def set_attn_keep_scores(on):
    """Whether a recorded attention forward keeps its scores for its backward."""
    _ck(lib().ctd_set_attn_keep_scores(int(bool(on))), "set_attn_keep_scores")


def set_head_chunk_rows(rows):
    """Rows per chunk of the fused LM head + loss (0 = automatic)."""
    _ck(lib().ctd_set_head_chunk_rows(rows), "set_head_chunk_rows")


def set_head_active_rows(on):
    """Whether the fused LM head + loss skips rows whose mask value is 0."""
    _ck(lib().ctd_set_head_active_rows(int(bool(on))), "set_head_active_rows")


def train_run(config_path):
    """Runs the ctd_train driver in this process (include/ctd/train.h)."""
    _ck(lib().ctd_train_run(str(config_path).encode()), "ctd_train")


def lr_at_step(step, warmup_steps, total_steps, lr, min_lr_ratio):
    out = C.c_float()
    _ck(lib().ctd_train_lr_at_step(step, warmup_steps, total_steps, lr, min_lr_ratio,
                                   C.byref(out)), "lr_at_step")
    return out.value


def host_batch(tok_path, mask_path, seq_len, docs):
    """(ids, targets, mask, sum_mask, num_docs) of the driver's batch of `docs`."""
    docs = np.ascontiguousarray(docs, dtype=np.int64)
    B, T = docs.size, seq_len - 1
    ids = np.zeros((B, T), np.int64)
    tgt = np.zeros((B, T), np.int64)
    mask = np.zeros((B, T), np.float32)
    sm, nd = C.c_float(), C.c_int64()
    _ck(lib().ctd_train_host_batch(str(tok_path).encode(), str(mask_path).encode(), seq_len,
                                   docs.ctypes.data_as(lptr), B, ids.ctypes.data_as(lptr),
                                   tgt.ctypes.data_as(lptr), mask.ctypes.data_as(fptr),
                                   C.byref(sm), C.byref(nd)), "host_batch")
    return ids, tgt, mask, sm.value, nd.value


def event_json(step, loss, lr=0.0, grad_norm=0.0, tokens_per_sec=0.0, wall_s=0.0, val=False):
    buf = C.create_string_buffer(512)
    _ck(lib().ctd_train_event_json(step, loss, lr, grad_norm, tokens_per_sec, wall_s, int(val), buf,
                                   512), "event_json")
    return buf.value.decode()


def param_count(cfg: ModelConfig) -> int:
    d, I, H, Hk, D, V, L = (cfg.hidden_size, cfg.intermediate_size, cfg.num_heads,
                            cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size, cfg.num_layers)
    per = 2 * d + 2 * H * D * d + 2 * Hk * D * d + 3 * I * d + (2 * D if cfg.qk_norm else 0)
    return V * d + d + L * per


__all__ = ["ModelConfig", "Trainer", "preset", "make_config", "memory", "reset_peak_memory",
           "set_memory_limit", "empty_cache", "alloc_history_start", "alloc_history_stop",
           "alloc_replay", "gemm_profile", "param_count", "StepTimes", "train_run", "lr_at_step", "host_batch",
           "event_json", "KVCache", "sample", "math"]
