"""ctypes binding of the C ABI in include/ember_hip.h (libember_hip.so).

This is the binding a Python caller of the kernels uses (tests and the bench
harness among them).  It loads the in-tree library and fails loudly when it is
missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libember_hip.so")

vp, i64, f32, i32, sz = C.c_void_p, C.c_int64, C.c_float, C.c_int, C.c_size_t
u64 = C.c_uint64

# name -> (restype, argtypes)
SIGNATURES = {
    "ember_status_string": (C.c_char_p, [i32]),
    "ember_get_device_count": (i32, [C.POINTER(i32)]),
    "ember_set_device": (i32, [i32]),
    "ember_get_device": (i32, [C.POINTER(i32)]),
    "ember_device_malloc": (i32, [C.POINTER(vp), sz]),
    "ember_device_free": (i32, [vp]),
    "ember_host_malloc_pinned": (i32, [C.POINTER(vp), sz]),
    "ember_host_free_pinned": (i32, [vp]),
    "ember_memcpy_async": (i32, [vp, vp, sz, i32, vp]),
    "ember_memcpy": (i32, [vp, vp, sz, i32]),
    "ember_mem_get_info": (i32, [C.POINTER(sz), C.POINTER(sz)]),
    "ember_device_synchronize": (i32, []),
    "ember_stream_create": (i32, [C.POINTER(vp)]),
    "ember_stream_destroy": (i32, [vp]),
    "ember_stream_synchronize": (i32, [vp]),
    "ember_event_create": (i32, [C.POINTER(vp)]),
    "ember_event_destroy": (i32, [vp]),
    "ember_event_record": (i32, [vp, vp]),
    "ember_event_synchronize": (i32, [vp]),
    "ember_event_query": (i32, [vp]),
    "ember_stream_wait_event": (i32, [vp, vp]),
    "ember_event_elapsed_ms": (i32, [C.POINTER(f32), vp, vp]),
    "ember_device_info": (i32, [C.c_char_p, sz, C.POINTER(i32), C.POINTER(sz)]),
    "ember_fill_normal": (i32, [vp, i64, u64, u64, f32, f32, vp]),
    "ember_fill": (i32, [vp, i64, f32, vp]),
    "ember_gemm_f32": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64, f32, vp,
                             i64, i64, i64, vp]),
    "ember_gemm_f32_workspace_bytes": (sz, [i64, i64, i64, i64]),
    "ember_gemm_f32_ws": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64, f32, vp,
                                i64, i64, i64, vp, sz, vp]),
    "ember_gemm_f32_dyn": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64,
                                 vp, i64, i32, vp, sz, vp]),
    "ember_gemm_f32_add": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, vp, i64, vp,
                                 i64, vp, sz, vp]),
    "ember_rmsnorm_fwd": (i32, [vp, vp, vp, vp, i64, i64, f32, vp]),
    "ember_qknorm_rope_fwd": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, f32, i64, vp, vp]),
    "ember_qknorm_rope_bwd": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, f32, i64, vp, vp,
                                    sz, vp]),
    "ember_rmsnorm_bwd_workspace_bytes": (sz, [i64, i64]),
    "ember_rmsnorm_bwd": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, f32, vp, sz, vp]),
    "ember_rmsnorm_bwd_accumulate": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, f32, vp, sz, vp]),
    "ember_rmsnorm_bwd_noalloc": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, f32, vp]),
    "ember_rope_freqs_host": (i32, [C.POINTER(f32), i32, f32, f32, f32, f32, i32]),
    "ember_rope": (i32, [vp, vp, i64, i64, i64, i64, i64, C.POINTER(f32), f32, vp]),
    "ember_add": (i32, [vp, vp, vp, i64, vp]),
    "ember_sub": (i32, [vp, vp, vp, i64, vp]),
    "ember_mul": (i32, [vp, vp, vp, i64, vp]),
    "ember_scale": (i32, [vp, f32, vp, i64, vp]),
    "ember_accumulate": (i32, [vp, vp, i64, vp]),
    "ember_silu": (i32, [vp, vp, i64, vp]),
    "ember_silu_bwd": (i32, [vp, vp, vp, i64, vp]),
    "ember_swiglu_fwd": (i32, [vp, vp, vp, i64, vp]),
    "ember_swiglu_bwd": (i32, [vp, vp, vp, vp, vp, i64, vp]),
    "ember_softmax_fwd": (i32, [vp, vp, i64, i64, vp]),
    "ember_softmax_bwd": (i32, [vp, vp, vp, i64, i64, vp]),
    "ember_causal_mask": (i32, [vp, vp, i64, i64, i64, i64, f32, vp]),
    "ember_repeat_kv": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "ember_repeat_kv_sum": (i32, [vp, vp, i64, i64, i64, i64, vp]),
    "ember_permute": (i32, [vp, vp, i32, C.POINTER(i64), C.POINTER(i32), vp]),
    "ember_attn_fwd": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, f32, vp]),
    "ember_attn_bwd_workspace_bytes": (sz, [i64, i64, i64]),
    "ember_attn_bwd_workspace_bytes_min": (sz, [i64, i64, i64]),
    "ember_attn_bwd": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, f32,
                             vp, sz, vp]),
    "ember_attn_bwd_ds_row_bytes": (sz, [i64, i64, i64]),
    "ember_attn_bwd_scattered": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                       f32, vp, sz, C.POINTER(vp), C.POINTER(sz), i32, vp]),
    "ember_attn_scores_workspace_bytes": (sz, [i64, i64]),
    "ember_attn_fwd_scores": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, f32,
                                    C.POINTER(vp), C.POINTER(sz), i32, vp, sz, vp]),
    "ember_attn_bwd_from_scores": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                         i64, f32, vp, sz, C.POINTER(vp), C.POINTER(sz), i32, vp]),
    "ember_ce_masked_fwd_workspace_bytes": (sz, [i64]),
    "ember_ce_masked_fwd": (i32, [vp, vp, vp, i64, i64, vp, vp, vp, vp, sz, vp]),
    "ember_ce_masked_bwd": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, vp, vp]),
    "ember_ce_masked_rows": (i32, [vp, vp, vp, i64, i64, vp, vp, vp]),
    "ember_mask_rows": (i32, [vp, i64, vp, vp, vp]),
    "ember_rows_gather": (i32, [vp, i64, i64, vp, vp, i64, i64, vp, vp]),
    "ember_rows_scatter": (i32, [vp, i64, vp, vp, i64, i64, vp, i64, vp]),
    "ember_ce_masked_rows_idx": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, vp, vp, vp]),
    "ember_ce_masked_bwd_idx": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, vp, vp, vp, vp]),
    "ember_ce_masked_reduce": (i32, [vp, vp, i64, vp, vp, vp]),
    "ember_embedding_fwd": (i32, [vp, vp, vp, i64, i64, i64, vp]),
    "ember_embedding_bwd_workspace_bytes": (sz, [i64, i64, i64]),
    "ember_embedding_bwd": (i32, [vp, vp, vp, i64, i64, i64, i32, vp, sz, vp]),
    "ember_sgd": (i32, [vp, vp, i64, f32, vp]),
    "ember_adamw": (i32, [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, f32, f32, vp]),
    "ember_adamw_bounded": (i32, [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, f32, f32, i32, vp]),
    "ember_sumsq_workspace_bytes": (sz, [i32]),
    "ember_sumsq_multi": (i32, [C.POINTER(vp), C.POINTER(i64), i32, vp, vp, sz, vp]),
    "ember_scale_multi_workspace_bytes": (sz, [i32]),
    "ember_scale_multi": (i32, [C.POINTER(vp), C.POINTER(i64), i32, f32, vp, sz, vp]),
    "ember_kv_write": (i32, [vp, vp, i64, i64, i64, i64, i64, i64, vp]),
    "ember_kv_read_expanded": (i32, [vp, vp, i64, i64, i64, i64, i64, i64, vp]),
    "ember_attn_decode_workspace_bytes": (sz, [i64, i64, i64, i64, i64, i64]),
    "ember_attn_decode": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                                f32, vp, sz, vp]),
    "ember_argmax_rows": (i32, [vp, i64, i64, vp, vp]),
    "ember_argmax_rows_workspace_bytes": (sz, [i64, i64]),
    "ember_argmax_rows_ws": (i32, [vp, i64, i64, vp, vp, sz, vp]),
    "ember_decode_gemv": (i32, [vp, i64, i64, vp, f32, i32, C.POINTER(vp), C.POINTER(i64),
                                C.POINTER(vp), C.POINTER(vp), vp]),
    "ember_decode_gateup": (i32, [vp, i64, i64, vp, f32, vp, vp, i64, vp, vp]),
    "ember_decode_qkv_post": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, f32,
                                    C.POINTER(f32), i64, vp, vp, vp, i64, vp]),
    "ember_attn_decode_qkv": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, f32,
                                    C.POINTER(f32), i64, vp, vp, i64, f32, vp, vp, sz, vp]),
}

_lib = None


class EmberError(RuntimeError):
    pass


def lib():
    """Load libember_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EmberError(f"{LIB_PATH} is missing: run `python -m emberlm_amd.build` first "
                             "(the HIP path has no fallback)")
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().ember_status_string(rc).decode()
        raise EmberError(f"{what}: status {rc} ({msg})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
