"""ctypes binding of libnitro_paged_attn.so (the C ABI in include/nitro_paged_attn.h).

Loading fails loudly when the library has not been built: there is no
fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# NITRO_LIB_PATH selects another build of the same library (e.g. for A/B timing).
LIB_PATH = os.environ.get("NITRO_LIB_PATH") or os.path.join(_HERE, "libnitro_paged_attn.so")

STATUS = {
    0: "NITRO_OK",
    1: "NITRO_ERR_INVALID_ARGUMENT",
    2: "NITRO_ERR_UNSUPPORTED",
    3: "NITRO_ERR_DEVICE_ALLOC",
    4: "NITRO_ERR_OUT_OF_PAGES",
    5: "NITRO_ERR_BAD_BLOCK_TABLE",
    6: "NITRO_ERR_HIP",
    7: "NITRO_ERR_NO_BATCH",
}
OK, INVALID_ARGUMENT, UNSUPPORTED, DEVICE_ALLOC, OUT_OF_PAGES, BAD_BLOCK_TABLE, HIP, NO_BATCH = range(8)


class NitroError(RuntimeError):
    def __init__(self, status: int, func: str, message: str):
        super().__init__(f"{func}: {STATUS.get(status, status)}: {message}")
        self.status = status


class nitro_block_info(ctypes.Structure):
    _fields_ = [("num_tokens", ctypes.c_int32), ("ref_count", ctypes.c_int32),
                ("parent_id", ctypes.c_int32), ("child_count", ctypes.c_int32)]


_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_vp = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_fp = ctypes.c_void_p  # device float pointers are passed as raw addresses

# name -> argtypes (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "nitro_status_string": [ctypes.c_int],
    "nitro_last_error": [],
    "nitro_hash_block_state": [_u64, _i32p, _i32],
    "nitro_bm_create": [_i32, ctypes.POINTER(_vp)],
    "nitro_bm_destroy": [_vp],
    "nitro_bm_allocate_block": [_vp, _i32p],
    "nitro_bm_inc_ref_count": [_vp, _i32],
    "nitro_bm_free_block": [_vp, _i32],
    "nitro_bm_force_free_block": [_vp, _i32],
    "nitro_bm_get_free_count": [_vp, _i32p],
    "nitro_bm_get_block": [_vp, _i32, ctypes.POINTER(nitro_block_info)],
    "nitro_bm_is_cached": [_vp, _i32, _i32p],
    "nitro_bm_check_cache": [_vp, _u64, _i32p],
    "nitro_bm_insert_cache": [_vp, _u64, _i32, _i32],
    "nitro_bm_evict_lru_block": [_vp],
    "nitro_bm_free_list": [_vp, _i32p, _i32, _i32p],
    "nitro_bm_evictable_leaves": [_vp, _i32p, _i32, _i32p],
    "nitro_bm_cache_entries": [_vp, _u64p, _i32p, _i32, _i32p],
    "nitro_bm_reverse_entries": [_vp, _i32p, _u64p, _i32, _i32p],
    "nitro_seq_create": [_i32, ctypes.POINTER(_vp)],
    "nitro_seq_destroy": [_vp],
    "nitro_seq_allocate_next_token": [_vp, _vp, _i32],
    "nitro_seq_flush_cache": [_vp, _vp],
    "nitro_seq_release": [_vp, _vp],
    "nitro_seq_prefix_walk": [_vp, _vp, _i32p, _i32, _i32, _i32, _i32p],
    "nitro_seq_ingest_prompt": [_vp, _vp, _i32p, _i32, _i32, _i32p],
    "nitro_seq_state": [_vp, _i32p, _u64p, _i32p, _i32p],
    "nitro_seq_block_table": [_vp, _i32p, _i32, _i32p],
    "nitro_seq_token_buffer": [_vp, _i32p, _i32, _i32p],
    "nitro_pack_block_tables": [ctypes.POINTER(_vp), _i32, _i32, _i32p],
    "nitro_kvpool_create": [_i32, _i32, _i32, ctypes.POINTER(_vp)],
    "nitro_kvpool_wrap": [_fp, _fp, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    "nitro_kvpool_wrap_contiguous": [_fp, _fp, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    "nitro_kvpool_destroy": [_vp],
    "nitro_kvpool_data": [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "nitro_kvpool_shape": [_vp, _i32p, _i32p, _i32p],
    "nitro_decode_batch_upload": [_vp, _i32p, _i32p, _i32, _i32, _vp],
    "nitro_kv_append": [_vp, _i32, _fp, _fp, _vp],
    "nitro_paged_attn_decode": [_vp, _i32, _fp, _fp, _i32, _i32, _i32, _vp],
    "nitro_paged_attn_decode_append": [_vp, _i32, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _vp],
    "nitro_paged_attn_decode_static": [_vp, _i32, _fp, _fp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                       _i32, _vp],
    "nitro_prefill_batch_upload": [_vp, _i32p, _i32p, _i32p, _i32, _i32, _vp],
    "nitro_kv_append_prefill": [_vp, _i32, _fp, _fp, _vp],
    "nitro_paged_attn_prefill": [_vp, _i32, _fp, _fp, _i32, _i32, _i32, _vp],
    "nitro_paged_attn_prefill_append": [_vp, _i32, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _vp],
    "nitro_rope_kv_append": [_vp, _i32, _fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32, _vp],
    "nitro_rope_kv_append_prefill": [_vp, _i32, _fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32, _i32,
                                     _vp],
    "nitro_q8_matmul": [_vp, _fp, _fp, _i32, _i32, _i32, _i32, _vp],
    "nitro_model_create": [_vp, ctypes.c_uint64, ctypes.POINTER(_vp)],
    "nitro_model_destroy": [_vp],
    "nitro_model_config": [_vp, _i32p],
    "nitro_forward_decode_batch": [_vp, _vp, _i32p, _i32, _fp, _i32, _vp],
    "nitro_forward_prefill": [_vp, _vp, _i32p, _i32, _fp, _i32, _vp],
    "nitro_sched_create": [_vp, _i32, _i32, ctypes.POINTER(_vp)],
    "nitro_sched_destroy": [_vp],
    "nitro_sched_add_request": [_vp, _i32, _i32p, _i32],
    "nitro_sched_set_limits": [_vp, _i32, _i32],
    "nitro_sched_has_active_requests": [_vp, _i32p],
    "nitro_sched_plan": [_vp, _i32p, _i32p, _i32p, _i32p, _i32, _i32p],
    "nitro_sched_commit": [_vp, _i32, _i32p, _i32],
    "nitro_sched_step": [_vp, _vp, _vp, _i32, _vp],
    "nitro_sched_last_logits": [_vp, ctypes.POINTER(ctypes.c_float), _i32, _i32p],
    "nitro_argmax": [_fp, _i32, _i32, _fp, _vp],
    "nitro_sched_state": [_vp, _i32p, _i32, _i32p],
    "nitro_sched_generated": [_vp, _i32, _i32p, _i32, _i32p],
    "nitro_sched_request_status": [_vp, _i32, _i32p],
    "nitro_sched_drop_request": [_vp, _i32],
    "nitro_rpc_encode_ints": [_i32p, _i32, ctypes.POINTER(ctypes.c_uint8), _u64, _u64p],
    "nitro_rpc_decode_ints": [ctypes.POINTER(ctypes.c_uint8), _u64, _i32p, _i32, _i32p, _u64p],
    "nitro_rpc_encode_structured_query": [_u64, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_float),
                                          _i32, ctypes.POINTER(ctypes.c_uint8), _u64, _u64p],
    "nitro_rpc_send_ints": [_i32, _i32p, _i32],
    "nitro_rpc_recv_ints": [_i32, _i32p, _i32, _i32p],
    "nitro_rpc_recv_structured_query": [_i32, _i32, _u64p, ctypes.POINTER(ctypes.c_float),
                                        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)],
    "nitro_server_create": [_vp, _vp, _vp, _i32, _i32, ctypes.POINTER(_vp)],
    "nitro_server_destroy": [_vp],
    "nitro_server_accept_fd": [_vp, _i32, _i32p],
    "nitro_server_step": [_vp, _vp, _i32p],
    "nitro_kvpool_take_device_errors": [_vp, _i32p],
    "nitro_kvpool_decode_counts": [_vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "nitro_kvpool_prefill_counts": [_vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
}
_RESTYPES = {
    "nitro_status_string": ctypes.c_char_p,
    "nitro_last_error": ctypes.c_char_p,
    "nitro_hash_block_state": _u64,
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built.

    torch is imported first when it is installed: its wheel ships its own
    libamdhip64.so.7, and loading it before this library makes the dynamic
    linker bind this library to that same runtime (same soname), so torch's
    streams and allocations are valid here.  Two HIP runtimes in one process
    would not share streams."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m nitrorag_amd.build` "
                "(there is no fallback path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Calls a status-returning entry point and raises NitroError on failure."""
    st = getattr(lib(), name)(*args)
    if st != OK:
        raise NitroError(st, name, lib().nitro_last_error().decode())


def last_error() -> str:
    return lib().nitro_last_error().decode()
