"""Stateless torch-facing entry points of the paged-KV path.

Each function validates tensor shapes, dtypes and devices on the host and then
calls one C ABI entry point (include/zealot_kv.h) on torch's current stream.
Pools are 4-D tensors [num_blocks, Hkv, block_size, D] -- the layout of
src/kv_cache.rs:41-50 -- of dtype float32, bfloat16 or float8_e4m3fn (uint8
storage is accepted for fp8).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

_FP8_DTYPES = tuple(d for d in (getattr(torch, "float8_e4m3fn", None), torch.uint8) if d is not None)


def zk_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.F32
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype in _FP8_DTYPES:
        return _lib.FP8_E4M3
    raise TypeError(f"unsupported dtype {t.dtype}")


def _stream(stream=None) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _dev(t: torch.Tensor, name: str, dtype=None, contiguous=True) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU (got {t.device})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    return t.data_ptr()


def _opt(t, name, dtype=None):
    return None if t is None else _dev(t, name, dtype)


def _pool_shape(k_pool: torch.Tensor, v_pool: torch.Tensor):
    if k_pool.dim() != 4 or k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError("k_pool/v_pool must be equal 4-D tensors [num_blocks, Hkv, block_size, D]")
    return tuple(int(x) for x in k_pool.shape)


def append(k_pool, v_pool, k, v, slot_mapping, k_scales=None, v_scales=None, token_row=None,
           stream=None) -> None:
    """Scatter k, v ([T, Hkv, D]) into the pools at slot_mapping[t] (int64)."""
    nb, hkv, bs, d = _pool_shape(k_pool, v_pool)
    if k.dim() != 3 or k.shape != v.shape or k.shape[1] != hkv or k.shape[2] != d:
        raise ValueError(f"k/v must be [T, {hkv}, {d}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if slot_mapping.shape != (k.shape[0],):
        raise ValueError("slot_mapping must be [T]")
    _lib.check(_lib.lib().zk_append(
        _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool"), zk_dtype(k_pool), _dev(k, "k"),
        _dev(v, "v"), zk_dtype(k), _dev(slot_mapping, "slot_mapping", torch.int64), k.shape[0],
        hkv, d, bs, nb, _opt(k_scales, "k_scales", torch.float32),
        _opt(v_scales, "v_scales", torch.float32), _opt(token_row, "token_row", torch.int32),
        _stream(stream)))


def fp8_scales(x, cu_seqlens, stream=None) -> torch.Tensor:
    """Per-(sequence, kv_head) scales amax/448 over x[cu[n]:cu[n+1]] ([T, Hkv, D])."""
    n = cu_seqlens.shape[0] - 1
    out = torch.empty((n, x.shape[1]), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().zk_fp8_scales(
        _dev(x, "x"), zk_dtype(x), _dev(cu_seqlens, "cu_seqlens", torch.int64), n, x.shape[1],
        x.shape[2], out.data_ptr(), _stream(stream)))
    return out


def gather(k_pool, v_pool, block_tables, ctx_lens, out_offsets, k_out, v_out, stream=None) -> None:
    """Copy each sequence's first ctx_lens[n] tokens into rows out_offsets[n].. of k_out/v_out."""
    nb, hkv, bs, d = _pool_shape(k_pool, v_pool)
    n, mb = block_tables.shape
    if k_out.dtype != k_pool.dtype or v_out.dtype != k_pool.dtype:
        raise TypeError("gather outputs must have the pool dtype")
    _lib.check(_lib.lib().zk_gather(
        _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool"), zk_dtype(k_pool),
        _dev(block_tables, "block_tables", torch.int32), mb, _dev(ctx_lens, "ctx_lens", torch.int32),
        _dev(out_offsets, "out_offsets", torch.int64), n, _dev(k_out, "k_out"),
        _dev(v_out, "v_out"), hkv, d, bs, nb, _stream(stream)))


def copy_blocks(pools, src, dst, stream=None) -> None:
    """For each i: block dst[i] := block src[i] in every pool of `pools`."""
    if not pools:
        return
    shape = tuple(pools[0].shape)
    for p in pools:
        if tuple(p.shape) != shape or p.dtype != pools[0].dtype:
            raise ValueError("all pools must share shape and dtype")
    nb = shape[0]
    block_bytes = pools[0][0].numel() * pools[0].element_size()
    arr = (ctypes.c_void_p * len(pools))(*[_dev(p, "pool") for p in pools])
    if src.shape != dst.shape:
        raise ValueError("src and dst must have the same length")
    _lib.check(_lib.lib().zk_copy_blocks(
        arr, len(pools), block_bytes, nb, _dev(src, "src", torch.int32), _dev(dst, "dst", torch.int32),
        src.shape[0], _stream(stream)))


_MAPPINGS = {"grouped": _lib.GQA_GROUPED, "modulo": _lib.GQA_MODULO}


def decode_workspace_bytes(num_seqs, num_heads, head_dim, max_blocks_per_seq, block_size) -> int:
    return int(_lib.lib().zk_paged_decode_workspace_size(num_seqs, num_heads, head_dim,
                                                          max_blocks_per_seq, block_size))


def paged_decode(q, k_pool, v_pool, block_tables, seq_lens, scale=None, mapping="grouped",
                 k_scales=None, v_scales=None, out=None, workspace=None, stream=None):
    """Decode attention: q [N, H, D] (f32/bf16) over paged K/V; returns out [N, H, D]."""
    nb, hkv, bs, d = _pool_shape(k_pool, v_pool)
    if q.dim() != 3 or q.shape[2] != d:
        raise ValueError(f"q must be [N, H, {d}]")
    n, h, _ = q.shape
    if block_tables.dim() != 2 or block_tables.shape[0] != n or seq_lens.shape != (n,):
        raise ValueError("block_tables must be [N, max_blocks] and seq_lens [N]")
    mb = block_tables.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)  # attention/cuda.rs:141
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q")
    need = decode_workspace_bytes(n, h, d, mb, bs)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.check(_lib.lib().zk_paged_decode(
        _dev(q, "q"), zk_dtype(q), _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool"),
        zk_dtype(k_pool), _dev(out, "out"), _dev(block_tables, "block_tables", torch.int32),
        _dev(seq_lens, "seq_lens", torch.int32), n, h, hkv, d, bs, mb, nb, float(scale),
        _MAPPINGS[mapping], _opt(k_scales, "k_scales", torch.float32),
        _opt(v_scales, "v_scales", torch.float32), _dev(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)))
    return out


def prefill_workspace_bytes(num_seqs, total_q, num_heads, num_kv_heads) -> int:
    return int(_lib.lib().zk_paged_prefill_workspace_size(num_seqs, total_q, num_heads, num_kv_heads))


def paged_prefill(q, k_pool, v_pool, block_tables, cu_seqlens_q, start_pos, causal=True, scale=None,
                  mapping="grouped", k_scales=None, v_scales=None, out=None, workspace=None, stream=None):
    """Chunked-prefill attention: q [T, H, D] (f32/bf16), sequence n's chunk is
    rows cu_seqlens_q[n] .. cu_seqlens_q[n+1] (int64) after start_pos[n] (int32)
    cached tokens; its K/V must already be in the pages.  Returns out [T, H, D]."""
    nb, hkv, bs, d = _pool_shape(k_pool, v_pool)
    if q.dim() != 3 or q.shape[2] != d:
        raise ValueError(f"q must be [T, H, {d}]")
    t, h, _ = q.shape
    n = start_pos.shape[0]
    if block_tables.dim() != 2 or block_tables.shape[0] != n or cu_seqlens_q.shape != (n + 1,):
        raise ValueError("block_tables must be [N, max_blocks], cu_seqlens_q [N + 1] and start_pos [N]")
    mb = block_tables.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q")
    need = prefill_workspace_bytes(n, t, h, hkv)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.check(_lib.lib().zk_paged_prefill(
        _dev(q, "q"), zk_dtype(q), _dev(k_pool, "k_pool"), _dev(v_pool, "v_pool"), zk_dtype(k_pool),
        _dev(out, "out"), _dev(block_tables, "block_tables", torch.int32),
        _dev(cu_seqlens_q, "cu_seqlens_q", torch.int64), _dev(start_pos, "start_pos", torch.int32), n, t, h, hkv,
        d, bs, mb, nb, float(scale), int(bool(causal)), _MAPPINGS[mapping],
        _opt(k_scales, "k_scales", torch.float32), _opt(v_scales, "v_scales", torch.float32),
        _dev(workspace, "workspace"), workspace.numel() * workspace.element_size(), _stream(stream)))
    return out
