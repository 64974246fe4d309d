"""HipAttention.paged_forward -- mirror of CudaAttention::paged_forward.

src/attention/cuda.rs:112-209 launches paged_attention[_gqa]_kernel on raw
device pointers with scale = 1/sqrt(head_dim) (cuda.rs:141) and the grouped
q-head -> kv-head mapping (paged_attention.cu:32).  This mirror takes the same
arguments (plus dtypes, defaulting to the reference's f32) and runs the
split-K gfx950 kernels in one batched launch sequence; the workspace is owned
by the HipAttention object and reused between calls (the role the reference's
BufferPool plays, buffer_pool.rs:23-61).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib


class HipAttention:
    def __init__(self, device=None):
        self.device = torch.device("cuda", 0) if device is None else torch.device(device)
        self._ws = None

    def _workspace(self, nbytes: int) -> torch.Tensor:
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._ws

    def paged_forward(self, q: int, k_pool: int, v_pool: int, block_tables: int, seq_lens: int,
                      o: int, num_seqs: int, num_heads: int, num_kv_heads: int, head_dim: int,
                      block_size: int, max_blocks_per_seq: int, num_blocks: int,
                      q_dtype: int = _lib.F32, kv_dtype: int = _lib.F32, mapping: int = _lib.GQA_GROUPED,
                      k_scales: int = 0, v_scales: int = 0, stream=None) -> None:
        """Arguments are device addresses (ints), as in cuda.rs:126-140."""
        if num_kv_heads <= 0 or num_heads % num_kv_heads != 0:
            raise RuntimeError("Internal error: paged_attention: num_heads must be a multiple of num_kv_heads")
        scale = 1.0 / math.sqrt(head_dim)
        need = int(_lib.lib().zk_paged_decode_workspace_size(num_seqs, num_heads, head_dim,
                                                              max_blocks_per_seq, block_size))
        ws = self._workspace(need)
        s = torch.cuda.current_stream(self.device) if stream is None else stream
        _lib.check(_lib.lib().zk_paged_decode(
            q, q_dtype, k_pool, v_pool, kv_dtype, o, block_tables, seq_lens, num_seqs, num_heads,
            num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_blocks, scale, mapping,
            k_scales or None, v_scales or None, ws.data_ptr(), ws.numel(),
            ctypes.c_void_p(s.cuda_stream)))
