"""ctypes binding of libzealot_kv.so (the C ABI declared in include/zealot_kv.h,
include/zealot_sched.h and include/zealot_dense.h).

The library is the product: there is no Python or CPU fallback.  If the
shared library is missing, importing any op raises immediately.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzealot_kv.so")

# zk_status
OK = 0
ERR_BLOCK_ALREADY_ALLOCATED = 1
ERR_BLOCK_NOT_ALLOCATED = 2
ERR_OUT_OF_BLOCKS = 3
ERR_INVALID_BLOCK_SIZE = 4
ERR_STALE_HANDLE = 5
ERR_SEQUENCE_TOO_LONG = 6
ERR_FAILED_PRECONDITION = 7
ERR_ALREADY_EXISTS = 8
ERR_INTERNAL = 9
ERR_INVALID_ARGUMENT = 10
ERR_HIP = 11

# zk_dtype
F32, BF16, FP8_E4M3 = 0, 1, 2
# zk_gqa_mapping
GQA_GROUPED, GQA_MODULO = 0, 1


class BlockHandleC(ctypes.Structure):
    _fields_ = [("block_id", ctypes.c_uint64), ("generation", ctypes.c_uint64)]


class SchedConfigC(ctypes.Structure):
    _fields_ = [("max_num_seqs", ctypes.c_size_t), ("block_size", ctypes.c_size_t),
                ("num_gpu_blocks", ctypes.c_size_t), ("max_prefill_tokens", ctypes.c_size_t),
                ("prefill_chunk_size", ctypes.c_size_t), ("swap_blocks", ctypes.c_size_t)]


class SchedEntryC(ctypes.Structure):
    _fields_ = [("request_id", ctypes.c_char_p), ("is_prefill", ctypes.c_int),
                ("is_final_chunk", ctypes.c_int), ("num_tokens", ctypes.c_size_t),
                ("tokens_before", ctypes.c_size_t), ("len", ctypes.c_size_t),
                ("num_blocks", ctypes.c_size_t), ("blocks", ctypes.POINTER(BlockHandleC)),
                ("block_offset", ctypes.c_size_t)]


class SchedOutputC(ctypes.Structure):
    _fields_ = [("batch", ctypes.POINTER(SchedEntryC)), ("batch_len", ctypes.c_size_t),
                ("preempted", ctypes.POINTER(ctypes.c_char_p)), ("num_preempted", ctypes.c_size_t),
                ("blocks", ctypes.POINTER(BlockHandleC)),
                ("swapped_out", ctypes.POINTER(ctypes.c_char_p)), ("num_swapped_out", ctypes.c_size_t),
                ("swapped_in", ctypes.POINTER(ctypes.c_char_p)), ("num_swapped_in", ctypes.c_size_t)]


class SchedSeqInfoC(ctypes.Structure):
    _fields_ = [("state", ctypes.c_int), ("is_prefill", ctypes.c_int), ("prompt_len", ctypes.c_size_t),
                ("output_len", ctypes.c_size_t), ("prefill_pos", ctypes.c_size_t),
                ("chunk_size", ctypes.c_size_t), ("len", ctypes.c_size_t), ("num_blocks", ctypes.c_size_t),
                ("swapped", ctypes.c_int)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_CP = ctypes.c_char_p

# name -> (restype, argtypes); every symbol declared in include/*.h.
SIGNATURES = {
    "zk_last_error": (ctypes.c_char_p, []),
    "zk_last_error_detail": (_I, [ctypes.POINTER(ctypes.c_uint64)]),
    "zk_abi_version": (_I, []),
    "zk_bm_create": (_I, [_SZ, _SZ, ctypes.POINTER(_P)]),
    "zk_bm_destroy": (None, [_P]),
    "zk_bm_allocate": (_I, [_P, ctypes.POINTER(BlockHandleC)]),
    "zk_bm_free": (_I, [_P, BlockHandleC]),
    "zk_bm_reference": (_I, [_P, BlockHandleC]),
    "zk_bm_available": (_SZ, [_P]),
    "zk_bm_num_gpu_blocks": (_SZ, [_P]),
    "zk_bm_block_size": (_SZ, [_P]),
    "zk_bm_refcount": (_SZ, [_P, ctypes.c_uint64]),
    "zk_bm_check": (_I, [_P, BlockHandleC]),
    "zk_append": (_I, [_P, _P, _I, _P, _P, _I, _P, _I64, _I, _I, _I, _I64, _P, _P, _P, _P]),
    "zk_fp8_scales": (_I, [_P, _I, _P, _I, _I, _I, _P, _P]),
    "zk_gather": (_I, [_P, _P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I64, _P]),
    "zk_copy_blocks": (_I, [_P, _I, _I64, _I64, _P, _P, _I64, _P]),
    "zk_paged_decode_workspace_size": (_SZ, [_I, _I, _I, _I, _I]),
    "zk_paged_decode": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I64, _F, _I,
                             _P, _P, _P, _SZ, _P]),
    "zk_paged_decode_noalloc": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I64, _F, _I,
                                     _P, _P, _P]),
    "zk_paged_prefill_workspace_size": (_SZ, [_I, _I64, _I, _I]),
    "zk_paged_prefill": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _P, _I, _I64, _I, _I, _I, _I, _I, _I64, _F, _I,
                              _I, _P, _P, _P, _SZ, _P]),
    "zk_cache_create": (_I, [_SZ, _SZ, _SZ, _SZ, _SZ, _I, _SZ, _SZ, _P, ctypes.POINTER(_P)]),
    "zk_cache_destroy": (None, [_P]),
    "zk_cache_register_seq": (_I, [_P, _CP, _SZ]),
    "zk_cache_alloc_block": (_I, [_P, _CP, _P, ctypes.POINTER(_SZ)]),
    "zk_cache_release_seq": (_I, [_P, _CP]),
    "zk_cache_fork_seq": (_I, [_P, _CP, _CP]),
    "zk_cache_store_kv": (_I, [_P, _SZ, _CP, _P, _P, _I, _SZ, _SZ]),
    "zk_cache_append_kv": (_I, [_P, _SZ, _CP, _P, _P, _I]),
    "zk_cache_append_kv_batch": (_I, [_P, _SZ, ctypes.POINTER(_CP), _I, _P, _P, _I]),
    "zk_cache_bind_blocks": (_I, [_P, _P, ctypes.POINTER(_CP), _I, _P, _P, _P]),
    "zk_cache_write_batch": (_I, [_P, _SZ, ctypes.POINTER(_CP), _P, _I, _P, _P, _I, _I64]),
    "zk_cache_write_batch_qkv": (_I, [_P, _SZ, ctypes.POINTER(_CP), _P, _I, _P, _P, _I64, _I, _P]),
    "zk_cache_enable_swap": (_I, [_P, _SZ]),
    "zk_cache_swap_space": (_I, [_P, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "zk_cache_swap_out": (_I, [_P, ctypes.POINTER(_CP), _I]),
    "zk_cache_swap_in": (_I, [_P, ctypes.POINTER(_CP), _I, _P]),
    "zk_cache_seq_swapped": (_I, [_P, _CP, ctypes.POINTER(ctypes.c_int)]),
    "zk_cache_set_fp8_scales": (_I, [_P, _CP, _P, _P]),
    "zk_cache_block_table_ptr": (_I, [_P, _CP, ctypes.POINTER(_P)]),
    "zk_cache_k_pool_ptr": (_P, [_P, _SZ]),
    "zk_cache_v_pool_ptr": (_P, [_P, _SZ]),
    "zk_cache_max_blocks": (_I, [_P, _CP, ctypes.POINTER(_SZ)]),
    "zk_cache_seq_state": (_I, [_P, _CP, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ),
                                ctypes.POINTER(_SZ)]),
    "zk_cache_block_ids": (_I, [_P, _CP, ctypes.POINTER(_I64), ctypes.POINTER(_SZ)]),
    "zk_cache_paged_decode": (_I, [_P, _SZ, ctypes.POINTER(_CP), _I, _P, _I, _P, _I, _F, _I]),
    "zk_cache_decode_append": (_I, [_P, _SZ, ctypes.POINTER(_CP), _I, _P, _P, _I, _P, _I, _P, _I, _F, _I]),
    "zk_cache_attention_batch": (_I, [_P, _SZ, ctypes.POINTER(_CP), _P, _I, _P, _I, _I64, _P, _I, _F, _I]),
    "zk_cache_decode_sharing": (_I, [_P, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int64)]),
    "zk_timing_enable": (_I, [_I]),
    "zk_timing_reset": (_I, []),
    "zk_timing_query": (_I, [_CP, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double)]),
    "zk_stream_copy": (_I, [_P, _P, _SZ, _P]),
    "zk_stream_read": (_I, [_P, _SZ, _P, _P]),
    "zk_rms_norm": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, _I, _P]),
    "zk_silu_mul": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P]),
    "zk_add": (_I, [_P, _P, _P, _I64, _I, _P]),
    "zk_embedding": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "zk_linear": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _I, _P]),
    "zk_linear_rms_norm": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _F, _P, _P, _P]),
    "zk_linear_choice": (_I, [_I64, _I64, _I64, _I, _I, _P]),
    "zk_linear_silu_mul": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "zk_weight_tile": (_I, [_P, _P, _I64, _I64, _P]),
    "zk_linear_tiled": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "zk_linear_rms_norm_tiled": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _F, _P, _P, _P]),
    "zk_linear_silu_mul_tiled": (_I, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "zk_linear_tiled_choice": (_I, [_I64, _I64, _I64, _I, _P]),
    "zk_linear_skinny": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P]),
    "zk_linear_tuning": (_I, [_I]),
    "zk_linear_pin_split": (_I, [_I64, _I64, _I64, _I, _I, _I, _I, _I]),
    "zk_sched_create": (_I, [ctypes.POINTER(SchedConfigC), _P, ctypes.POINTER(_P)]),
    "zk_sched_destroy": (None, [_P]),
    "zk_sched_block_manager": (_P, [_P]),
    "zk_sched_make_sequence": (_I, [_P, _CP, _P, _SZ, _SZ, _I, ctypes.POINTER(_P)]),
    "zk_sequence_destroy": (None, [_P]),
    "zk_sched_add": (_I, [_P, _P]),
    "zk_sched_schedule": (_I, [_P, ctypes.POINTER(SchedOutputC)]),
    "zk_sched_push_token": (_I, [_P, _CP, _I64]),
    "zk_sched_mark_prefilled": (_I, [_P, _CP]),
    "zk_sched_promote_to_decoding": (None, [_P, _CP]),
    "zk_sched_advance_prefill": (None, [_P, _CP]),
    "zk_sched_finish": (_I, [_P, _CP, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "zk_sched_cancel": (_I, [_P, _CP, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "zk_sched_is_idle": (_I, [_P]),
    "zk_sched_step_input": (_I, [_P, _CP, ctypes.POINTER(_I64), ctypes.POINTER(_SZ)]),
    "zk_sched_seq_info": (_I, [_P, _CP, ctypes.POINTER(SchedSeqInfoC)]),
}

_lib = None


# Field names of the typed ZealotError variants (src/error.rs:4-37), in the
# order zk_last_error_detail returns them.
ERROR_FIELDS = {
    ERR_BLOCK_ALREADY_ALLOCATED: ("block_id",),
    ERR_BLOCK_NOT_ALLOCATED: ("block_id",),
    ERR_OUT_OF_BLOCKS: ("requested", "available"),
    ERR_INVALID_BLOCK_SIZE: ("block_size",),
    ERR_STALE_HANDLE: ("block_id", "handle_gen", "current_gen"),
    ERR_SEQUENCE_TOO_LONG: ("required", "capacity"),
}


class ZealotError(RuntimeError):
    """Error raised from a zk_status; str() is the reference's message and
    ``fields`` the variant's named fields (empty for untyped errors)."""

    def __init__(self, code: int, message: str, fields: dict | None = None):
        super().__init__(message)
        self.code = code
        self.fields = dict(fields or {})


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m zealot_amd.build` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error_detail() -> tuple[int, dict]:
    """(status, named fields) of this thread's last failure (zk_last_error_detail)."""
    raw = (ctypes.c_uint64 * 3)()
    code = lib().zk_last_error_detail(raw)
    return code, dict(zip(ERROR_FIELDS.get(code, ()), (int(x) for x in raw)))


def check(rc: int) -> None:
    if rc != OK:
        code, fields = last_error_detail()
        msg = lib().zk_last_error().decode("utf-8", "replace")
        raise ZealotError(rc, msg, fields if code == rc else {})
