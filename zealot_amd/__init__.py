"""zealot_amd -- MI355X (gfx950) paged-KV hot path of the Zealot engine.

Host-side mirror of the reference interfaces over the C ABI in
include/zealot_kv.h (implemented by libzealot_kv.so, built from
zealot_amd/csrc with `python -m zealot_amd.build`):

  BlockManager, BlockHandle   src/block_manager.rs
  KVCache                     src/kv_cache.rs
  HipAttention.paged_forward  src/attention/cuda.rs (CudaAttention::paged_forward)
  ops.append / gather / copy_blocks / paged_decode / fp8_scales
                              stateless launches over caller-owned tensors
"""
from ._lib import ZealotError, lib  # noqa: F401
from .block_manager import BlockHandle, BlockManager  # noqa: F401

__all__ = ["BlockHandle", "BlockManager", "ZealotError", "lib", "ops", "KVCache", "HipAttention"]


def __getattr__(name):
    # torch-dependent modules load lazily so BlockManager works without torch
    if name == "KVCache":
        from .kv_cache import KVCache
        return KVCache
    if name == "HipAttention":
        from .attention import HipAttention
        return HipAttention
    if name == "ops":
        from . import ops
        return ops
    raise AttributeError(name)
