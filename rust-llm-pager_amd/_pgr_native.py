"""ctypes binding of libpgr.so (the C ABI declared in include/pgr.h).

Torch-free on purpose: ``pager`` (the placement policy) uses it without importing torch.
The library is loaded from this directory; there is no fallback implementation, so a
missing or stale build raises ImportError here.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PGR_LIBRARY", os.path.join(_HERE, "libpgr.so"))

PGR_OK = 0
PGR_ERR_INVALID = -1
PGR_ERR_UNSUPPORTED = -2
PGR_ERR_HIP = -3
PGR_ERR_CAPACITY = -4
PGR_ERR_STATE = -5
PGR_ERR_KEY = -6
PGR_ERR_BUDGET = -7
PGR_ERR_INTERNAL = -8

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2  # operator API and finalize only

MODE_FOLD = 0
MODE_STATS = 1
MODE_ACCUMULATE = 2
MODE_FOLD_FIXED = 3

STREAM_DIRECT = 0
STREAM_STAGED = 1
STREAM_MIRROR = 2

ABI_VERSION = 10

c_i32, c_i64, c_u8, c_u32, c_u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64
c_f32, c_f64, c_size, c_vp = ctypes.c_float, ctypes.c_double, ctypes.c_size_t, ctypes.c_void_p
P = ctypes.POINTER


class PagerMetrics(ctypes.Structure):
    _fields_ = [
        ("tokens", c_u64),
        ("vram_peak", c_u64),
        ("ram_peak", c_u64),
        ("swap_vram_ram", c_u64),
        ("swap_ram_ssd", c_u64),
        ("attention_mass_total", c_f64),
        ("attention_mass_vram", c_f64),
    ]


class KVConfig(ctypes.Structure):
    _fields_ = [
        ("num_layers", c_i32),
        ("kv_heads", c_i32),
        ("query_heads", c_i32),
        ("head_dim", c_i32),
        ("tokens_per_block", c_i32),
        ("dtype", c_i32),
        ("pool_slots", c_i64),
        ("host_records", c_i64),
        ("staging_slots", c_i64),
        ("staging_buffers", c_i32),
        ("blocks_per_workgroup", c_i32),
        ("target_workgroups", c_i32),
        ("stream_mode", c_i32),
    ]


class KVStats(ctypes.Structure):
    _fields_ = [
        ("gpu_to_cpu_bytes", c_u64),
        ("cpu_to_gpu_bytes", c_u64),
        ("gpu_to_cpu_copies", c_u64),
        ("cpu_to_gpu_copies", c_u64),
        ("gpu_to_cpu_sec", c_f64),
        ("cpu_to_gpu_sec", c_f64),
        ("evict_bytes_copied", c_u64),
        ("load_bytes_copied", c_u64),
        ("stream_bytes", c_u64),
        ("stream_copies", c_u64),
    ]


class KVStepStats(ctypes.Structure):
    _fields_ = [
        ("resident_tokens", c_i64),
        ("host_tokens", c_i64),
        ("host_blocks", c_i64),
        ("copies", c_i64),
        ("chunks", c_i64),
        ("launches", c_i64),
        ("work_items", c_i64),
        ("gather_blocks", c_i64),
        ("plan_wait_ns", c_i64),
    ]


# name -> (restype, argtypes). Every symbol declared in include/pgr.h.
SIGNATURES: dict[str, tuple] = {
    "pgr_abi_version": (ctypes.c_int, []),
    "pgr_last_error": (ctypes.c_char_p, []),
    "pgr_attn_workspace_bytes": (c_size, [c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_i64]),
    "pgr_attn_step": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_f32,
         c_f32, c_vp, c_size, c_vp],
    ),
    "pgr_attn_step_noalloc": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_f32,
         c_f32, c_vp],
    ),
    "pgr_attn_stats_step": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_f32, c_f32, c_vp,
         c_size, c_vp],
    ),
    "pgr_attn_accumulate_step": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
         c_i64, ctypes.c_int, c_f32, c_f32, c_vp, c_size, c_vp],
    ),
    "pgr_attn_fold_fixed_step": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_f32, c_f32,
         c_vp, c_size, c_vp],
    ),
    "pgr_bench_stream_read": (ctypes.c_int, [P(c_vp), c_i32, c_i64, c_i32, c_i32, P(c_f64), c_vp]),
    "pgr_bench_stream_read_back_to_back": (ctypes.c_int, [P(c_vp), c_i32, c_i64, c_i32, c_i32, P(c_f64), c_vp]),
    "pgr_attn_bench_step": (ctypes.c_int, [c_vp, P(c_vp), P(c_vp), c_i32, c_i64, c_i64, c_i64, c_i64, c_i64,
                                            ctypes.c_int, c_f32, c_vp, c_size, c_i32, P(c_f64), P(c_i64), c_vp]),
    "pgr_attn_set_timing": (ctypes.c_int, [c_i32]),
    "pgr_attn_kernel_time": (ctypes.c_int, [P(c_f64), P(c_i64), P(c_i64)]),
    "pgr_attn_state_init": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_vp]),
    "pgr_attn_finalize": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int, c_vp]),
    "pgr_pager_new": (c_vp, [c_u64, c_u64, c_u64, c_u64, c_f32, c_f32, ctypes.c_char_p]),
    "pgr_pager_free": (None, [c_vp]),
    "pgr_pager_on_step": (ctypes.c_int, [c_vp, c_u64, c_u32, P(c_f32), c_size]),
    "pgr_pager_force_rebalance": (ctypes.c_int, [c_vp, c_u64]),
    "pgr_pager_num_blocks": (c_size, [c_vp]),
    "pgr_pager_tiers": (c_size, [c_vp, P(c_u8), c_size]),
    "pgr_pager_vram_block_ids": (c_size, [c_vp, P(c_u64), c_size]),
    "pgr_pager_metrics": (ctypes.c_int, [c_vp, P(PagerMetrics)]),
    "pgr_kv_create": (c_vp, [P(KVConfig)]),
    "pgr_kv_destroy": (None, [c_vp]),
    "pgr_kv_add_session": (ctypes.c_int, [c_vp, c_i32, c_i64, P(c_i32)]),
    "pgr_kv_remove_session": (ctypes.c_int, [c_vp, c_i32]),
    "pgr_kv_set_lo": (ctypes.c_int, [c_vp, c_i32, P(c_i32)]),
    "pgr_kv_reorder_rows": (ctypes.c_int, [c_vp, c_i32, P(c_i32), c_i32, c_vp]),
    "pgr_kv_step_signature": (ctypes.c_int, [c_vp, P(c_i64), c_i64]),
    "pgr_kv_step_replayed": (ctypes.c_int, [c_vp, c_vp]),
    "pgr_kv_set_length": (ctypes.c_int, [c_vp, c_i32, c_i64]),
    "pgr_kv_import": (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_i64, c_vp]),
    "pgr_kv_export": (ctypes.c_int, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp]),
    "pgr_kv_put_block": (ctypes.c_int, [c_vp, c_i32, c_i64, c_vp, c_vp, c_vp]),
    "pgr_kv_get_block": (ctypes.c_int, [c_vp, c_i32, c_i64, c_vp, c_vp, c_vp]),
    "pgr_kv_apply_tiers": (
        ctypes.c_int,
        [c_vp, c_i32, P(c_u8), c_i64, P(c_i64), P(c_i64), P(c_i64), P(c_i64), P(c_i64), c_vp],
    ),
    "pgr_kv_set_ram_budget": (ctypes.c_int, [c_vp, c_i64]),
    "pgr_kv_begin_step": (ctypes.c_int, [c_vp, P(c_i32), c_i32, c_vp]),
    "pgr_kv_decode_layer": (
        ctypes.c_int,
        [c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_f32, c_f32, c_i32, c_vp],
    ),
    "pgr_kv_end_step": (ctypes.c_int, [c_vp, P(c_i32), P(c_i32)]),
    "pgr_kv_attach_pager": (ctypes.c_int, [c_vp, c_i32, c_vp, c_i32]),
    "pgr_kv_end_step_place": (
        ctypes.c_int,
        [c_vp, c_vp, c_i64, c_i32, P(c_i32), P(c_i32), P(c_i64), P(c_i64), c_i64, P(c_f64), c_i64, c_vp],
    ),
    "pgr_kv_session_info": (ctypes.c_int, [c_vp, c_i32, P(c_i64)]),
    "pgr_kv_block_ids": (ctypes.c_int, [c_vp, c_i32, c_i32, P(c_i64), c_i64]),
    "pgr_kv_step_host_blocks": (ctypes.c_int, [c_vp, c_i32, P(c_i64), c_i64]),
    "pgr_kv_step_stats": (ctypes.c_int, [c_vp, P(KVStepStats)]),
    "pgr_kv_stats": (ctypes.c_int, [c_vp, P(KVStats)]),
    "pgr_kv_resident_bytes": (ctypes.c_int, [c_vp, P(c_i64), P(c_i64)]),
    "pgr_kv_hbm_bytes": (ctypes.c_int, [c_vp, P(c_i64)]),
    "pgr_kv_block_bytes": (ctypes.c_int, [c_vp, c_i32, P(c_i64)]),
    "pgr_kv_set_timing": (ctypes.c_int, [c_vp, c_i32]),
    "pgr_kv_kernel_time": (ctypes.c_int, [c_vp, P(c_f64), P(c_i64), P(c_i64)]),
    "pgr_kv_bench_attention": (ctypes.c_int, [c_vp, P(c_vp), P(c_vp), P(c_vp), c_f32, c_f32, c_i32, P(c_f64), P(c_i64),
                                               c_vp]),
    "pgr_kv_copy_time": (ctypes.c_int, [c_vp, P(c_f64), P(c_i64), P(c_i64)]),
    "pgr_kv_sync": (ctypes.c_int, [c_vp]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libpgr.so once and attach the prototypes; raises ImportError if it is missing."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libpgr.so not found at {LIB_PATH}; build it with `python rust-llm-pager_amd/build.py` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(LIB_PATH)
        lib.pgr_abi_version.restype = ctypes.c_int
        lib.pgr_abi_version.argtypes = []
        if lib.pgr_abi_version() != ABI_VERSION:  # before any other symbol: a stale build fails here
            raise ImportError(f"libpgr.so ABI {lib.pgr_abi_version()} does not match the bindings ({ABI_VERSION}); "
                              "rebuild it")
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().pgr_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


_EXC = {
    PGR_ERR_INVALID: ValueError,
    PGR_ERR_UNSUPPORTED: NotImplementedError,
    PGR_ERR_HIP: RuntimeError,
    PGR_ERR_CAPACITY: MemoryError,
    PGR_ERR_STATE: RuntimeError,
    PGR_ERR_KEY: KeyError,
    PGR_ERR_BUDGET: RuntimeError,
    PGR_ERR_INTERNAL: RuntimeError,
}


def check(rc: int, what: str = "") -> int:
    """Raise the Python exception for a negative status code; pass through non-negative values."""
    if rc >= 0:
        return rc
    exc = _EXC.get(rc, RuntimeError)
    msg = last_error()
    raise exc(f"{what}: {msg}" if what else msg)
