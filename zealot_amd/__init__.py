"""zealot_amd -- MI355X (gfx950) paged-KV hot path of the Zealot engine.

Host-side mirror of the reference interfaces over the C ABI in
include/zealot_kv.h (implemented by libzealot_kv.so, built from
zealot_amd/csrc with `python -m zealot_amd.build`):

  BlockManager, BlockHandle   src/block_manager.rs
  KVCache                     src/kv_cache.rs
  HipAttention.paged_forward  src/attention/cuda.rs (CudaAttention::paged_forward)
  Scheduler, SchedulerConfig  src/scheduler.rs (over a BlockManager shared
                              with the KVCache)
  PagedKVRunner               KV side of a batched ModelRunner step
                              (src/cuda_runner.rs:271-461)
  ops.append / gather / copy_blocks / paged_decode / paged_prefill / fp8_scales
                              stateless launches over caller-owned tensors
"""
from ._lib import ZealotError, lib  # noqa: F401
from .block_manager import BlockHandle, BlockManager  # noqa: F401
from .scheduler import CancelOutcome, Priority, Scheduler, SchedulerConfig  # noqa: F401

__all__ = ["BlockHandle", "BlockManager", "ZealotError", "lib", "ops", "KVCache", "SeqBatch",
           "HipAttention", "Scheduler", "SchedulerConfig", "Priority", "CancelOutcome", "PagedKVRunner"]


def __getattr__(name):
    # torch-dependent modules load lazily so BlockManager works without torch
    import importlib
    if name in ("KVCache", "SeqBatch"):
        return getattr(importlib.import_module(".kv_cache", __name__), name)
    if name == "PagedKVRunner":
        return importlib.import_module(".runner", __name__).PagedKVRunner
    if name == "HipAttention":
        return importlib.import_module(".attention", __name__).HipAttention
    if name == "ops":
        return importlib.import_module(".ops", __name__)
    raise AttributeError(name)
