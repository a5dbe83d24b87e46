"""ctypes binding of libexl3moe.so, the C-ABI of this library (include/exl3moe.h).

The torch op library (_moe.so) is the usual entry; this module lets callers without torch custom ops (and the tests)
call the C functions directly with raw device pointers and a HIP stream handle. torch is imported first so that the
process has one HIP runtime (torch's) when the library is loaded next to it.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libexl3moe.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "exl3moe.h")
_lib = None

c_i32, c_i64, c_sz, c_p = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

SIGNATURES = {
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_blob_bytes": (c_i64, [c_i32, c_i32, c_i32]),
    "exl3_set_tier": (c_i32, [c_p, c_p, c_i64, c_p]),
    "exl3_set_victims": (c_i32, [c_p]),
    "exl3_set_victim_addrs": (c_i32, [c_p]),
    "exl3_set_record_pool": (c_i32, [c_p, c_p, c_p, c_i64]),
    "exl3_set_victim_ring": (c_i32, [c_p, c_p, c_p, c_i64, c_i64]),
    "exl3_set_host_stride": (c_i32, [c_i64]),
    "exl3_set_slot_stride": (c_i32, [c_i64]),
    "exl3_set_fused_ensure": (c_i32, [c_i64]),
    "exl3_set_prefill_min_m": (c_i32, [c_i64]),
    "exl3_set_pair_max_m": (c_i32, [c_i64]),
    "exl3_set_splits": (c_i32, [c_i64, c_i64]),
    "exl3_set_mr": (c_i32, [c_i64]),
    "exl3_set_debug": (c_i32, [c_i64]),
    "exl3_set_decision_log": (c_i32, [c_p, c_i64]),
    "exl3_moe_forward_workspace": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "exl3_moe_forward": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_p, c_p, c_i32, c_p, c_i32, c_i32, c_i32, c_p, c_i64,
                                 c_p, c_sz, c_p]),
    "exl3_moe_forward_cached": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_p, c_p, c_i32, c_p, c_i32, c_p, c_p, c_p, c_p,
                                        c_i32, c_p, c_i64, c_p, c_p, c_i32, c_i32, c_i32, c_i32, c_p, c_i64, c_p, c_sz,
                                        c_p]),
    "exl3_moe_forward_cached_static": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_p, c_p, c_i32, c_p, c_i32, c_p, c_p,
                                               c_p, c_p, c_i32, c_p, c_i64, c_p, c_p, c_i32, c_i32, c_i32, c_i32, c_p,
                                               c_i64, c_p]),
    "exl3_moe_prefetch": (c_i32, [c_p, c_i32, c_p, c_i32, c_p, c_p, c_p, c_p, c_i32, c_p, c_i64, c_p, c_p, c_i32, c_i32,
                                  c_i64, c_p]),
    "exl3_moe_prefetch_plan": (c_i32, [c_p, c_i32, c_p, c_i32, c_p, c_p, c_p, c_p, c_i32, c_p, c_i64, c_p, c_p, c_p,
                                       c_p, c_p, c_p, c_i32, c_i32, c_i32, c_i64, c_p]),
    "exl3_prefetch_worker_start": (c_i32, [c_p, c_p, c_i64, c_i64, c_p, c_p, c_i32, c_i32, c_p]),
    "exl3_prefetch_worker_stop": (c_i32, [c_p]),
    "exl3_set_prefetch_commit": (c_i32, [c_p, c_p, c_i32]),
    "exl3_moe_align_workspace": (c_sz, [c_i32, c_i32, c_i32]),
    "exl3_moe_align": (c_i32, [c_p, c_p, c_i32, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_sz, c_p]),
    "exl3_dequant": (c_i32, [c_p, c_i32, c_i32, c_i32, c_p, c_p]),
    "exl3_device_status": (c_i32, [c_p, c_p]),
    "exl3_device_status_address": (c_i32, [c_p]),
    "exl3_set_status_mirror": (c_i32, [c_p]),
    "exl3_scatter_flags": (c_i32, [c_p, c_i64, c_p, c_i64, c_p]),
    "exl3_tier_exchange": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_p, c_p, c_p, c_p, c_i32, c_p]),
    "exl3_tier_exchange_pool": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_p, c_p, c_p, c_p, c_i32,
                                        c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_p]),
    "exl3_admit_decide": (c_i32, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p]),
    "exl3_host_alloc": (c_p, [c_i64]),
    "exl3_host_free": (c_i32, [c_p]),
    "exl3_usm_kind": (c_i32, [c_p]),
    "exl3_memcpy_async": (c_i32, [c_p, c_p, c_i64, c_p]),
    "exl3_copy_batch": (c_i32, [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_p]),
    "exl3_table_update": (c_i32, [c_p, c_p, c_p, c_p, c_p, c_i64, c_p]),
    "exl3_linear_supported": (c_i32, [c_i32, c_i32]),
    "exl3_linear_workspace": (c_sz, [c_i32, c_i32, c_i32]),
    "exl3_linear_small": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_i32, c_p, c_i32, c_i32, c_p, c_i32, c_p, c_p, c_p,
                                  c_i32, c_i64, c_p, c_sz, c_p]),
    "exl3_had_in": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_p, c_i32, c_p, c_p]),
    "exl3_had_out": (c_i32, [c_p, c_i32, c_i32, c_p, c_p, c_i32, c_i64, c_p]),
    "exl3_reconstruct": (c_i32, [c_p, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_p, c_p]),
    "exl3_had_in_q8": (c_i32, [c_p, c_i32, c_i64, c_i32, c_i32, c_p, c_i32, c_p, c_p, c_i64, c_p]),
    "exl3_reconstruct_q8": (c_i32, [c_p, c_i32, c_i32, c_i32, c_i32, c_i32, c_p, c_p]),
    "exl3_had_out_q8": (c_i32, [c_p, c_i32, c_i32, c_p, ctypes.c_float, c_p, c_p, c_i32, c_i64, c_p]),
}


def declared_functions(header: str = HEADER) -> list:
    """Function names declared in include/exl3moe.h."""
    txt = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", txt)))


def lib():
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (one HIP runtime per process: torch's)
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"exl3xpu: {LIB_PATH} not built; run qwen38-flash-next-b70-offload_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "exl3") -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: error {rc}: {lib().exl3_last_error().decode()}")


def stream_handle(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)
