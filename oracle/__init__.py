"""CPU oracle for Zealot's paged-KV path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed CPU
baseline).  The product package ``zealot_amd`` never imports it.

The arithmetic lives in ``zk_oracle.c`` (a C restatement of the reference's
Rust CPU path; see the citations there).  This module is a thin ctypes/numpy
front end plus host-side numeric helpers (bf16 and fp8-e4m3 conversions) used
to build inputs.

Parity status of each restated function (how it is pinned, see tests/):
  or_store_kv / or_append_slots / or_gather / or_copy_blocks
      pinned by the reference's layout formula through index-tagged payloads
      (every element encodes its own (token, head, dim)), round trips and
      canary fills -- tests/test_oracle.py.
  or_paged_decode
      pinned against torch's scaled_dot_product_attention in float64 (an
      independent library routine), closed forms (ctx=1, constant K, dominant
      score, shift invariance) and both GQA mappings against
      or_repeat_interleave_kv + or_cpu_attention -- tests/test_oracle.py.
  or_paged_prefill
      pinned against or_paged_decode (a one-row chunk at position p is the
      decode of p + 1 tokens), or_cpu_attention (a non-causal chunk from
      position 0 is CpuAttention::forward on the gathered K/V) and torch's
      causal scaled_dot_product_attention in float64 -- tests/test_oracle.py.
  or_cpu_attention / or_matmul / or_repeat_interleave_kv
      pinned by the reference's own unit tests (attention/mod.rs:121-189,
      model_runner_cpu.rs:153-195) restated as golden fixtures.
  or_e4m3_from_f32 / or_f32_from_e4m3
      pinned exhaustively against torch.float8_e4m3fn (all 256 codes; all
      in-range bf16 values) -- tests/test_oracle.py.
  or_rms_norm / or_silu_gate_mul / or_add / or_embedding / linear
      pinned against numpy float64 restatements of the textbook formulas
      (RMSNorm, SiLU = g * sigmoid(g), x @ W.T) and closed forms (a constant
      row normalises to sign(x) * w; silu(0) = 0, silu(g) -> g for large g;
      index-tagged embedding rows) -- tests/test_oracle_dense.py.
  block_manager_model
      pinned by the reference's known-answer tests (tests/test_block_manager.py,
      block_manager.rs:179-249) and its proptest regression seeds.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, BF16, FP8 = 0, 1, 2
GROUPED, MODULO = 0, 1

_lib = None


def build(force: bool = False) -> str:
    """Compile zk_oracle.c with the Makefile beside it."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float


def _declare(L):
    L.or_bf16_from_f32.restype = ctypes.c_uint16
    L.or_bf16_from_f32.argtypes = [_F]
    L.or_f32_from_bf16.restype = _F
    L.or_f32_from_bf16.argtypes = [ctypes.c_uint16]
    L.or_e4m3_from_f32.restype = ctypes.c_uint8
    L.or_e4m3_from_f32.argtypes = [_F]
    L.or_f32_from_e4m3.restype = _F
    L.or_f32_from_e4m3.argtypes = [ctypes.c_uint8]
    L.or_store_kv.restype = _I
    L.or_store_kv.argtypes = [_P, _P, _I, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I]
    L.or_store_kv_batch.restype = _I
    L.or_store_kv_batch.argtypes = [_P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
    L.or_append_slots.restype = _I
    L.or_append_slots.argtypes = [_P, _P, _I, _P, _P, _I, _P, _I64, _I, _I, _I, _I64, _P, _P, _P]
    L.or_fp8_scales.restype = None
    L.or_fp8_scales.argtypes = [_P, _I, _P, _I, _I, _I, _P]
    L.or_gather.restype = _I64
    L.or_gather.argtypes = [_P, _I, _P, _I64, _I64, _P, _I, _I, _I]
    L.or_copy_blocks.restype = None
    L.or_copy_blocks.argtypes = [_P, _I, _I64, _P, _P, _I64]
    L.or_paged_decode.restype = _I
    L.or_paged_decode.argtypes = [_P, _P, _P, _I, _P, _P, _P, _I64, _P, _I, _I, _I, _I, _I, _F,
                                  _I, _P, _I]
    L.or_paged_prefill.restype = _I
    L.or_paged_prefill.argtypes = [_P, _P, _P, _I, _P, _P, _P, _I64, _P, _P, _I, _I, _I, _I, _I, _F,
                                   _I, _I, _P, _I]
    L.or_cpu_attention.restype = _I
    L.or_cpu_attention.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P]
    L.or_matmul.restype = None
    L.or_matmul.argtypes = [_P, _P, _I, _I, _I, _P]
    L.or_repeat_interleave_kv.restype = None
    L.or_repeat_interleave_kv.argtypes = [_P, _I, _I, _I, _I, _P]
    L.or_rms_norm.restype = None
    L.or_rms_norm.argtypes = [_P, _P, _P, _I64, _I64, _F]
    L.or_silu_gate_mul.restype = None
    L.or_silu_gate_mul.argtypes = [_P, _P, _P, _I64]
    L.or_add.restype = None
    L.or_add.argtypes = [_P, _P, _P, _I64]
    L.or_embedding.restype = None
    L.or_embedding.argtypes = [_P, _P, _P, _I64, _I64]


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------- numerics

def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even (vectorised)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def f32_from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


_E4M3_TABLE = None


def f32_from_e4m3_bits(c: np.ndarray) -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        L = lib()
        _E4M3_TABLE = np.array([L.or_f32_from_e4m3(i) for i in range(256)], dtype=np.float32)
    return _E4M3_TABLE[np.asarray(c, dtype=np.uint8)]


def e4m3_bits_from_f32_scalar(x: float) -> int:
    return int(lib().or_e4m3_from_f32(float(x)))


# ---------------------------------------------------------------- path ops

def elt_size(dtype: int) -> int:
    return {F32: 4, BF16: 2, FP8: 1}[dtype]


def store_kv(k_pool, v_pool, dtype, k, v, block_ids, start_token, n_tokens, num_kv_heads,
             head_dim, block_size) -> int:
    bids = np.ascontiguousarray(block_ids, dtype=np.int64)
    return lib().or_store_kv(_ptr(k_pool), _ptr(v_pool), dtype, _ptr(k), _ptr(v), _ptr(bids),
                             len(bids), start_token, n_tokens, num_kv_heads, head_dim, block_size)


def store_kv_batch(k_pool, v_pool, dtype, k, v, block_lists, start_tokens, n_tokens, num_kv_heads, head_dim,
                   block_size, threads=1) -> int:
    """store_kv for each sequence n: n_tokens[n] rows of k/v (packed in batch
    order) at start_tokens[n] through block_lists[n]; threads > 1 runs the
    sequences on OpenMP threads."""
    bids = np.ascontiguousarray(np.concatenate([np.asarray(b, np.int64) for b in block_lists]), dtype=np.int64)
    boff = np.concatenate([[0], np.cumsum([len(b) for b in block_lists])]).astype(np.int64)
    toff = np.concatenate([[0], np.cumsum(n_tokens)]).astype(np.int64)
    st = np.ascontiguousarray(start_tokens, dtype=np.int64)
    return lib().or_store_kv_batch(_ptr(k_pool), _ptr(v_pool), dtype, _ptr(k), _ptr(v), _ptr(bids), _ptr(boff),
                                   _ptr(toff), _ptr(st), len(block_lists), num_kv_heads, head_dim, block_size,
                                   threads)


def append_slots(k_pool, v_pool, cache_dtype, k, v, src_dtype, slot_mapping, num_kv_heads,
                 head_dim, block_size, num_blocks, k_scales=None, v_scales=None, token_row=None):
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    tr = None if token_row is None else np.ascontiguousarray(token_row, dtype=np.int32)
    ks = None if k_scales is None else np.ascontiguousarray(k_scales, dtype=np.float32)
    vs = None if v_scales is None else np.ascontiguousarray(v_scales, dtype=np.float32)
    return lib().or_append_slots(_ptr(k_pool), _ptr(v_pool), cache_dtype, _ptr(k), _ptr(v),
                                 src_dtype, _ptr(slots), len(slots), num_kv_heads, head_dim,
                                 block_size, num_blocks, _ptr(ks), _ptr(vs), _ptr(tr))


def fp8_scales(x, src_dtype, cu_seqlens, num_kv_heads, head_dim) -> np.ndarray:
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    n = len(cu) - 1
    out = np.zeros((n, num_kv_heads), dtype=np.float32)
    lib().or_fp8_scales(_ptr(x), src_dtype, _ptr(cu), n, num_kv_heads, head_dim, _ptr(out))
    return out


def gather(pool, dtype, block_table, ctx_len, num_kv_heads, head_dim, block_size, out_dtype):
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    out = np.zeros((ctx_len, num_kv_heads, head_dim), dtype=out_dtype)
    n = lib().or_gather(_ptr(pool), dtype, _ptr(bt), len(bt), ctx_len, _ptr(out), num_kv_heads,
                        head_dim, block_size)
    return out[:n]


def copy_blocks(pools, block_bytes, src, dst):
    arr = (ctypes.c_void_p * len(pools))(*[p.ctypes.data for p in pools])
    s = np.ascontiguousarray(src, dtype=np.int32)
    d = np.ascontiguousarray(dst, dtype=np.int32)
    lib().or_copy_blocks(arr, len(pools), block_bytes, _ptr(s), _ptr(d), len(s))


def paged_decode(q, k_pool, v_pool, kv_dtype, block_tables, seq_lens, num_kv_heads, head_dim,
                 block_size, scale, mapping=GROUPED, k_scales=None, v_scales=None, threads=1):
    q = np.ascontiguousarray(q, dtype=np.float32)
    n, h = q.shape[0], q.shape[1]
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    ks = None if k_scales is None else np.ascontiguousarray(k_scales, dtype=np.float32)
    vs = None if v_scales is None else np.ascontiguousarray(v_scales, dtype=np.float32)
    out = np.zeros((n, h, head_dim), dtype=np.float32)
    rc = lib().or_paged_decode(_ptr(q), _ptr(k_pool), _ptr(v_pool), kv_dtype, _ptr(ks), _ptr(vs),
                               _ptr(bt), bt.shape[1], _ptr(sl), n, h, num_kv_heads, head_dim,
                               block_size, scale, mapping, _ptr(out), threads)
    if rc != 0:
        raise RuntimeError(f"or_paged_decode failed: {rc}")
    return out


def paged_prefill(q, k_pool, v_pool, kv_dtype, block_tables, cu_seqlens_q, start_pos, num_kv_heads,
                  head_dim, block_size, scale, causal=True, mapping=GROUPED, k_scales=None, v_scales=None,
                  threads=1):
    """q [T, H, D] (f32 values) -> out [T, H, D] f32; see or_paged_prefill."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    t, h = q.shape[0], q.shape[1]
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cu = np.ascontiguousarray(cu_seqlens_q, dtype=np.int64)
    st = np.ascontiguousarray(start_pos, dtype=np.int32)
    ks = None if k_scales is None else np.ascontiguousarray(k_scales, dtype=np.float32)
    vs = None if v_scales is None else np.ascontiguousarray(v_scales, dtype=np.float32)
    out = np.zeros((t, h, head_dim), dtype=np.float32)
    rc = lib().or_paged_prefill(_ptr(q), _ptr(k_pool), _ptr(v_pool), kv_dtype, _ptr(ks), _ptr(vs),
                                _ptr(bt), bt.shape[1], _ptr(cu), _ptr(st), len(st), h, num_kv_heads, head_dim,
                                block_size, scale, mapping, int(bool(causal)), _ptr(out), threads)
    if rc != 0:
        raise RuntimeError(f"or_paged_prefill failed: {rc}")
    return out


def cpu_attention(q, k, v, num_seqs, num_heads, head_dim, max_seq_len):
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    expected = num_seqs * num_heads * max_seq_len * head_dim
    if q.size != expected or k.size != expected or v.size != expected:
        # attention/mod.rs:39-48
        raise RuntimeError(f"Internal error: dimension mismatch: expected {expected}, got "
                           f"q={q.size} k={k.size} v={v.size}")
    out = np.zeros(expected, dtype=np.float32)
    lib().or_cpu_attention(_ptr(q), _ptr(k), _ptr(v), num_seqs, num_heads, head_dim, max_seq_len,
                           _ptr(out))
    return out


def matmul(a, b, m, k, n):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.zeros(m * n, dtype=np.float32)
    lib().or_matmul(_ptr(a), _ptr(b), m, k, n, _ptr(c))
    return c


def repeat_interleave_kv(src, kv_heads, num_heads, seq_len, head_dim):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(num_heads * seq_len * head_dim, dtype=np.float32)
    lib().or_repeat_interleave_kv(_ptr(src), kv_heads, num_heads, seq_len, head_dim, _ptr(out))
    return out


# ----------------------------------------------------------------- dense ops

def rms_norm(x, w, eps=1e-6):
    """rms_norm.cu:4-55 over the rows of x [rows, dim] (f32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_rms_norm(_ptr(x), _ptr(w), _ptr(out), x.shape[0] if x.ndim > 1 else 1, x.shape[-1], eps)
    return out


def silu_gate_mul(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().or_silu_gate_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def add(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    lib().or_add(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def embedding(ids, table):
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    table = np.ascontiguousarray(table, dtype=np.float32)
    out = np.empty((ids.size, table.shape[1]), np.float32)
    lib().or_embedding(_ptr(ids), _ptr(table), _ptr(out), ids.size, table.shape[1])
    return out


def linear(x, w):
    """y = x @ w.T with or_matmul (attention/mod.rs matmul), w [n, k]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    wt = np.ascontiguousarray(np.asarray(w, dtype=np.float32).T)
    m, k = x.shape
    n = wt.shape[1]
    out = np.empty((m, n), np.float32)
    lib().or_matmul(_ptr(x), _ptr(wt), m, k, n, _ptr(out))
    return out

