"""KV side of a batched HIP ModelRunner: one bind, then one write launch and
one attention call per layer for the whole schedule() batch.

The reference runner (src/cuda_runner.rs:271-461) loops over the batch and,
per sequence and layer, calls store_kv / append_kv and paged_forward with
num_seqs=1 after a synchronous copy of the sequence length; its KV cache
never learns the scheduler's blocks (no caller of register_seq /
alloc_block).  Here the scheduler and the cache share one BlockManager:

    plan = runner.begin_step(sched.schedule())   # drop preempted, bind tables
    for layer in range(L):
        q, k, v = ...                              # the model's projections
        runner.write(layer, plan, k, v)            # zk_cache_write_batch
        out = runner.attention(layer, plan, q)     # zk_cache_attention_batch

Rows of q / k / v / out are the batch's step tokens packed in batch order
(entry i owns plan.num_tokens[i] rows).  drop_state (engine.rs:20-22) releases
the cache's view of a sequence; its blocks belong to the scheduler.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from .block_manager import BlockManager
from .kv_cache import KVCache, SeqBatch


@dataclass
class StepPlan:
    """The packed batch of one step."""
    ids: SeqBatch
    num_tokens: ctypes.Array      # int32 per entry
    tokens_before: list
    total_tokens: int


class PagedKVRunner:
    def __init__(self, cache: KVCache, block_manager: BlockManager):
        if block_manager.block_size != cache.block_size:
            raise ValueError("BlockManager and KVCache block sizes differ")
        self.cache = cache
        self.bm = block_manager
        self._bound = set()

    def begin_step(self, out) -> StepPlan:
        """Move the KV of sequences preempted by swap to host slots (before
        anything of this step can write their freed blocks), drop the state of
        those preempted by recompute, bind every entry's blocks
        (Sequence.blocks) as its block table -- checking that the cache holds
        exactly entry.tokens_before tokens of it -- and copy the KV of
        re-admitted swapped sequences back into their new blocks."""
        if out.swapped_out:
            self.cache.swap_out(out.swapped_out)
        for rid in out.preempted:
            self.drop_state(rid)
        batch = out.batch
        n = len(batch)
        ids = SeqBatch([s.request_id for s in batch])
        handles = [h for s in batch for h in s.blocks]
        harr = (_lib.BlockHandleC * max(1, len(handles)))(*[h._c() for h in handles])
        nb = (ctypes.c_size_t * max(1, n))(*[len(s.blocks) for s in batch])
        tb = (ctypes.c_size_t * max(1, n))(*[s.tokens_before for s in batch])
        _lib.check(_lib.lib().zk_cache_bind_blocks(self.cache._h, self.bm.handle, ids.arr, n, harr, nb, tb))
        self._bound.update(ids.ids)
        if out.swapped_in:
            self.cache.swap_in(out.swapped_in)
        nt = (ctypes.c_int32 * max(1, n))(*[s.num_tokens for s in batch])
        return StepPlan(ids, nt, [s.tokens_before for s in batch], sum(s.num_tokens for s in batch))

    def write(self, layer: int, plan: StepPlan, k, v) -> None:
        self.cache.write_batch(layer, plan.ids, plan.num_tokens, k, v)

    def write_qkv(self, layer: int, plan: StepPlan, x, w_qkv, num_heads: int, out=None):
        """The step's fused q/k/v projection and KV write for one layer; returns
        the projection buffer (its q columns feed attention)."""
        return self.cache.write_batch_qkv(layer, plan.ids, plan.num_tokens, x, w_qkv, num_heads, out=out)

    def attention(self, layer: int, plan: StepPlan, q, out=None, scale=None, mapping="grouped"):
        return self.cache.attention_batch(layer, plan.ids, plan.num_tokens, q, out=out, scale=scale,
                                          mapping=mapping)

    def drop_state(self, request_id: str) -> None:
        if request_id in self._bound:
            self._bound.discard(request_id)
            self.cache.release_seq(request_id)
