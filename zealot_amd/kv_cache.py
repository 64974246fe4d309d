"""KVCache over the C ABI -- the host mirror of src/kv_cache.rs:51-356.

Method names and argument meaning follow the reference (register_seq,
alloc_block, release_seq, store_kv, append_kv, block_table_ptr, k_pool_ptr,
v_pool_ptr, max_blocks, seq_state); tensors are torch device tensors and
errors are RuntimeErrors with the reference's messages.  All state and every
launch live in C++ (zealot_amd/csrc/kv_cache.cpp).  Additions: fork_seq
(prefix sharing with copy-on-write), set_fp8_scales (fp8 pools), paged_decode
(batched decode of registered sequences), k_pool/v_pool (tensor views of the
pools, for tests and callers that launch their own kernels).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import torch

from . import _lib
from .block_manager import BlockManager
from .ops import zk_dtype, _stream, _dev

_TORCH_TO_ZK = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
if hasattr(torch, "float8_e4m3fn"):
    _TORCH_TO_ZK[torch.float8_e4m3fn] = _lib.FP8_E4M3
_TORCH_TO_ZK[torch.uint8] = _lib.FP8_E4M3


@dataclass
class SeqKvState:
    """kv_cache.rs:24-35 (block_table is exposed as a device pointer)."""
    block_table: int
    block_ids: list = field(default_factory=list)
    cached_tokens: int = 0
    block_offset: int = 0
    max_blocks: int = 0


def _id(s: str) -> bytes:
    return s.encode("utf-8")


class SeqBatch:
    """A list of sequence ids packed once for the C ABI, for callers that issue
    the same batched call for every layer (append_kv_batch, paged_decode)."""

    def __init__(self, ids):
        self.ids = [str(i) for i in ids]
        self._raw = [_id(i) for i in self.ids]
        self.arr = (ctypes.c_char_p * len(self._raw))(*self._raw)

    def __len__(self) -> int:
        return len(self.ids)


def _batch(ids) -> SeqBatch:
    return ids if isinstance(ids, SeqBatch) else SeqBatch(ids)


def _token_stride(t, name: str, rows: int, heads: int, dim: int) -> int:
    """Elements between consecutive token rows of a [rows, heads, dim] device
    tensor whose inner [heads, dim] block is packed."""
    _dev(t, name, contiguous=False)
    if tuple(t.shape) != (rows, heads, dim):
        raise RuntimeError(f"Internal error: KVCache: {name} has shape {tuple(t.shape)}, expected "
                           f"{(rows, heads, dim)}")
    if t.stride(2) != 1 or (heads > 1 and t.stride(1) != dim):
        raise ValueError(f"{name} must have packed [heads, dim] rows")
    if rows > 1 and t.stride(0) < heads * dim:
        raise ValueError(f"{name} rows overlap")
    return t.stride(0) if rows > 1 else heads * dim


def _counts(num_tokens, n: int):
    if isinstance(num_tokens, ctypes.Array):
        arr = num_tokens
    else:
        vals = [int(x) for x in num_tokens]
        arr = (ctypes.c_int32 * max(1, len(vals)))(*vals)
        if len(vals) != n:
            raise ValueError("num_tokens must hold one count per id")
    return arr


class KVCache:
    """kv_cache.rs:51-102.  One HBM slab holds every layer's K and V pool."""

    def __init__(self, num_blocks: int, block_size: int, num_layers: int, num_kv_heads: int,
                 head_dim: int, dtype=torch.float32, max_seqs: int = 256,
                 max_blocks_per_seq: int = 1024, stream=None):
        self._h = None
        if dtype not in _TORCH_TO_ZK:
            raise TypeError(f"unsupported KV dtype {dtype}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self._stream_obj = stream
        # bound now: at interpreter exit the module globals may already be gone
        self._destroy = _lib.lib().zk_cache_destroy
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().zk_cache_create(num_blocks, block_size, num_layers, num_kv_heads,
                                              head_dim, _TORCH_TO_ZK[dtype], max_seqs,
                                              max_blocks_per_seq, _stream(stream), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_h", None) and destroy is not None:
            destroy(self._h)
            self._h = None

    # -- sequence lifecycle (kv_cache.rs:104-166) --------------------------
    def register_seq(self, id: str, max_blocks: int) -> None:
        _lib.check(_lib.lib().zk_cache_register_seq(self._h, _id(id), max_blocks))

    def alloc_block(self, id: str, bm: BlockManager) -> int:
        out = ctypes.c_size_t()
        _lib.check(_lib.lib().zk_cache_alloc_block(self._h, _id(id), bm.handle, ctypes.byref(out)))
        return int(out.value)

    def release_seq(self, id: str) -> None:
        _lib.check(_lib.lib().zk_cache_release_seq(self._h, _id(id)))

    def fork_seq(self, parent: str, child: str) -> None:
        _lib.check(_lib.lib().zk_cache_fork_seq(self._h, _id(parent), _id(child)))

    def set_fp8_scales(self, id: str, k_scales, v_scales) -> None:
        ks = torch.as_tensor(k_scales, dtype=torch.float32).contiguous().cpu()
        vs = torch.as_tensor(v_scales, dtype=torch.float32).contiguous().cpu()
        n = self.num_layers * self.num_kv_heads
        if ks.numel() != n or vs.numel() != n:
            raise ValueError(f"scales must hold num_layers * num_kv_heads = {n} values")
        _lib.check(_lib.lib().zk_cache_set_fp8_scales(self._h, _id(id), ks.data_ptr(), vs.data_ptr()))

    # -- queries (kv_cache.rs:168-204) --------------------------------------
    def seq_state(self, id: str) -> SeqKvState:
        L = _lib.lib()
        ct, bo, nb = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(L.zk_cache_seq_state(self._h, _id(id), ctypes.byref(ct), ctypes.byref(bo),
                                        ctypes.byref(nb)))
        ids = (ctypes.c_int64 * max(1, nb.value))()
        n = ctypes.c_size_t(nb.value)
        _lib.check(L.zk_cache_block_ids(self._h, _id(id), ids, ctypes.byref(n)))
        return SeqKvState(block_table=self.block_table_ptr(id), block_ids=list(ids[:n.value]),
                          cached_tokens=ct.value, block_offset=bo.value,
                          max_blocks=self.max_blocks(id))

    def max_blocks(self, id: str) -> int:
        out = ctypes.c_size_t()
        _lib.check(_lib.lib().zk_cache_max_blocks(self._h, _id(id), ctypes.byref(out)))
        return int(out.value)

    def block_table_ptr(self, id: str) -> int:
        out = ctypes.c_void_p()
        _lib.check(_lib.lib().zk_cache_block_table_ptr(self._h, _id(id), ctypes.byref(out)))
        return int(out.value)

    def k_pool_ptr(self, layer: int) -> int:
        return int(_lib.lib().zk_cache_k_pool_ptr(self._h, layer) or 0)

    def v_pool_ptr(self, layer: int) -> int:
        return int(_lib.lib().zk_cache_v_pool_ptr(self._h, layer) or 0)

    # -- store / append (kv_cache.rs:206-356) -------------------------------
    def _kv(self, k, v, rows):
        for name, t in (("k", k), ("v", v)):
            _dev(t, name)
            if t.dtype not in (torch.float32, torch.bfloat16):
                raise TypeError(f"{name} must be float32 or bfloat16")
            if t.numel() != rows * self.num_kv_heads * self.head_dim:
                raise RuntimeError(f"Internal error: KVCache: {name} has {t.numel()} elements, expected "
                                   f"{rows * self.num_kv_heads * self.head_dim}")
        if k.dtype != v.dtype:
            raise TypeError("k and v must share a dtype")
        return zk_dtype(k)

    def store_kv(self, layer: int, id: str, k, v, start_token: int, n_tokens: int) -> None:
        dt = self._kv(k, v, n_tokens)
        _lib.check(_lib.lib().zk_cache_store_kv(self._h, layer, _id(id), k.data_ptr(), v.data_ptr(),
                                                dt, start_token, n_tokens))

    def append_kv(self, layer: int, id: str, k, v) -> None:
        dt = self._kv(k, v, 1)
        _lib.check(_lib.lib().zk_cache_append_kv(self._h, layer, _id(id), k.data_ptr(), v.data_ptr(),
                                                 dt))

    def append_kv_batch(self, layer: int, ids, k, v) -> None:
        """One decode token per sequence: k, v are [len(ids), Hkv, D]; ids is a
        list of ids or a SeqBatch."""
        b = _batch(ids)
        n = len(b)
        dt = self._kv(k, v, n)
        _lib.check(_lib.lib().zk_cache_append_kv_batch(self._h, layer, b.arr, n, k.data_ptr(),
                                                       v.data_ptr(), dt))

    def write_batch(self, layer: int, ids, num_tokens, k, v) -> None:
        """Mixed step write: sequence ids[i] receives num_tokens[i] tokens
        (packed in batch order in k, v [sum(num_tokens), Hkv, D]) at its
        cached_tokens position; the last layer advances every sequence.  k and
        v may be row-strided views (e.g. the K / V columns of a fused QKV
        projection output): only the token stride may differ from packed."""
        b = _batch(ids)
        nt = _counts(num_tokens, len(b))
        rows = int(sum(nt))
        stride = _token_stride(k, "k", rows, self.num_kv_heads, self.head_dim)
        if _token_stride(v, "v", rows, self.num_kv_heads, self.head_dim) != stride:
            raise ValueError("k and v must share a token stride")
        if k.dtype != v.dtype or k.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("k and v must both be float32 or bfloat16")
        _lib.check(_lib.lib().zk_cache_write_batch(self._h, layer, b.arr, ctypes.addressof(nt), len(b),
                                                   k.data_ptr(), v.data_ptr(), zk_dtype(k), stride))

    def write_batch_qkv(self, layer: int, ids, num_tokens, x, w_qkv, num_heads: int, out=None):
        """The fused q/k/v projection of x [T, hidden] (bf16) against w_qkv
        [(H + 2 Hkv) D, hidden] and write_batch of its K and V columns, in
        one call (zk_cache_write_batch_qkv): returns the projection buffer
        [T, (H + 2 Hkv) D], whose q columns are always written (its K / V
        columns only when the projection was not folded into the write)."""
        b = _batch(ids)
        nt = _counts(num_tokens, len(b))
        rows = int(sum(nt))
        cols = (num_heads + 2 * self.num_kv_heads) * self.head_dim
        if x.dtype != torch.bfloat16 or w_qkv.dtype != torch.bfloat16:
            raise TypeError("x and w_qkv must be bfloat16")
        if x.dim() != 2 or x.shape[0] != rows or tuple(w_qkv.shape) != (cols, x.shape[1]):
            raise ValueError("x must be [sum(num_tokens), hidden] and w_qkv [(H + 2 Hkv) D, hidden]")
        if out is None:
            out = torch.empty((rows, cols), dtype=torch.bfloat16, device=x.device)
        elif out.dtype != torch.bfloat16 or tuple(out.shape) != (rows, cols):
            raise ValueError("out must be a bfloat16 [sum(num_tokens), (H + 2 Hkv) D] tensor")
        _lib.check(_lib.lib().zk_cache_write_batch_qkv(self._h, layer, b.arr, ctypes.addressof(nt), len(b),
                                                       _dev(x, "x"), _dev(w_qkv, "w_qkv"), x.shape[1], num_heads,
                                                       _dev(out, "out")))
        return out

    # -- decode --------------------------------------------------------------
    def paged_decode(self, layer: int, ids, q, out=None, scale=None, mapping="grouped"):
        """Decode attention for registered sequences `ids` (batch order; a list
        or a SeqBatch), q [N, H, D]."""
        _dev(q, "q")
        b = _batch(ids)
        n, h, d = q.shape
        if n != len(b) or d != self.head_dim:
            raise ValueError("q must be [len(ids), H, head_dim]")
        if out is None:
            out = torch.empty_like(q)
        if scale is None:
            scale = 1.0 / math.sqrt(d)
        m = {"grouped": _lib.GQA_GROUPED, "modulo": _lib.GQA_MODULO}[mapping]
        _lib.check(_lib.lib().zk_cache_paged_decode(self._h, layer, b.arr, n, q.data_ptr(),
                                                    zk_dtype(q), _dev(out, "out"), h, float(scale), m))
        return out

    def decode_append(self, layer: int, ids, k, v, q, out=None, scale=None, mapping="grouped"):
        """append_kv_batch(layer, ids, k, v) then paged_decode(layer, ids, q),
        with the same results; one decode launch on bf16 MFMA shapes (the
        decode stores each sequence's new K / V row and attends it)."""
        _dev(q, "q")
        b = _batch(ids)
        n, h, d = q.shape
        if n != len(b) or d != self.head_dim:
            raise ValueError("q must be [len(ids), H, head_dim]")
        dt = self._kv(k, v, n)
        if out is None:
            out = torch.empty_like(q)
        if scale is None:
            scale = 1.0 / math.sqrt(d)
        m = {"grouped": _lib.GQA_GROUPED, "modulo": _lib.GQA_MODULO}[mapping]
        _lib.check(_lib.lib().zk_cache_decode_append(self._h, layer, b.arr, n, k.data_ptr(), v.data_ptr(), dt,
                                                     q.data_ptr(), zk_dtype(q), _dev(out, "out"), h, float(scale),
                                                     m))
        return out

    def attention_batch(self, layer: int, ids, num_tokens, q, out=None, scale=None, mapping="grouped"):
        """Mixed step attention after write_batch: the num_tokens[i] rows of
        sequence ids[i] (packed in batch order in q [sum(num_tokens), H, D])
        are its last num_tokens[i] tokens at this layer, attended causally.
        q may be a row-strided view (the Q columns of a fused QKV output);
        out is packed [rows, H, D]."""
        b = _batch(ids)
        nt = _counts(num_tokens, len(b))
        rows, h, d = q.shape
        if rows != sum(nt) or d != self.head_dim:
            raise ValueError("q must be [sum(num_tokens), H, head_dim]")
        qs = _token_stride(q, "q", rows, h, d)
        if out is None:
            out = torch.empty((rows, h, d), dtype=q.dtype, device=q.device)
        if scale is None:
            scale = 1.0 / math.sqrt(d)
        m = {"grouped": _lib.GQA_GROUPED, "modulo": _lib.GQA_MODULO}[mapping]
        _lib.check(_lib.lib().zk_cache_attention_batch(self._h, layer, b.arr, ctypes.addressof(nt), len(b),
                                                       q.data_ptr(), zk_dtype(q), qs, _dev(out, "out"), h,
                                                       float(scale), m))
        return out

    def decode_sharing(self):
        """(subgroups, shared pages) of the last paged_decode's prefix sharing."""
        sg, pages = ctypes.c_int(), ctypes.c_int64()
        _lib.check(_lib.lib().zk_cache_decode_sharing(self._h, ctypes.byref(sg), ctypes.byref(pages)))
        return sg.value, pages.value

    # -- swap (host <-> device block moves) -----------------------------------
    def enable_swap(self, num_host_blocks: int) -> None:
        """Pinned host space of num_host_blocks slots (one block of every pool)."""
        _lib.check(_lib.lib().zk_cache_enable_swap(self._h, num_host_blocks))

    def swap_space(self):
        """(total, free) host slots."""
        t, f = ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(_lib.lib().zk_cache_swap_space(self._h, ctypes.byref(t), ctypes.byref(f)))
        return t.value, f.value

    def swap_out(self, ids) -> None:
        b = _batch(ids)
        _lib.check(_lib.lib().zk_cache_swap_out(self._h, b.arr, len(b)))

    def swap_in(self, ids, bm: BlockManager | None = None) -> None:
        b = _batch(ids)
        _lib.check(_lib.lib().zk_cache_swap_in(self._h, b.arr, len(b), bm.handle if bm is not None else None))

    def is_swapped(self, id: str) -> bool:
        out = ctypes.c_int()
        _lib.check(_lib.lib().zk_cache_seq_swapped(self._h, _id(id), ctypes.byref(out)))
        return bool(out.value)

    # -- pool views ----------------------------------------------------------
    def _pool_view(self, ptr: int) -> torch.Tensor:
        """Device tensor aliasing a pool (shape [num_blocks, Hkv, bs, D])."""
        from ._devmem import tensor_from_device_ptr
        shape = (self.num_blocks, self.num_kv_heads, self.block_size, self.head_dim)
        dtype = self.dtype
        return tensor_from_device_ptr(ptr, shape, dtype, owner=self)

    def k_pool(self, layer: int) -> torch.Tensor:
        return self._pool_view(self.k_pool_ptr(layer))

    def v_pool(self, layer: int) -> torch.Tensor:
        return self._pool_view(self.v_pool_ptr(layer))
