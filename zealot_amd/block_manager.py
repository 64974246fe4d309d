"""BlockManager / BlockHandle over the C ABI.

Mirrors the Python surface of the reference's PyO3 classes
(src/block_manager.rs:16-84; exercised by tests/test_block_manager.py):
``BlockManager(num_gpu_blocks, block_size)`` with ``allocate()``, ``free(h)``,
``reference(h)`` and the ``free_blocks`` / ``num_gpu_blocks`` / ``block_size``
getters; ``BlockHandle(block_id, generation)`` with the same attributes and a
repr naming both.  Every failure is a RuntimeError whose text is the
reference's ZealotError message (src/error.rs:3-46, converted to RuntimeError
at error.rs:48-52).  The allocator itself is C++ (zealot_amd/csrc/block_manager.cpp).
"""
from __future__ import annotations

import ctypes

from . import _lib


class BlockHandle:
    """block_manager.rs:16-39."""

    __slots__ = ("_id", "_gen")

    def __init__(self, block_id: int, generation: int):
        self._id = int(block_id)
        self._gen = int(generation)

    @property
    def block_id(self) -> int:
        return self._id

    @property
    def generation(self) -> int:
        return self._gen

    def __repr__(self) -> str:
        return f"BlockHandle(id={self._id}, gen={self._gen})"

    def __eq__(self, other) -> bool:
        return isinstance(other, BlockHandle) and (self._id, self._gen) == (other._id, other._gen)

    def __hash__(self) -> int:
        return hash((self._id, self._gen))

    def _c(self) -> _lib.BlockHandleC:
        return _lib.BlockHandleC(self._id, self._gen)


class BlockManager:
    """block_manager.rs:41-165 (pymethods at :51-84, Rust-native try_* at :86-164)."""

    def __init__(self, num_gpu_blocks: int, block_size: int):
        L = _lib.lib()
        self._h = None
        # bound now: at interpreter exit the module globals may already be gone
        self._destroy = L.zk_bm_destroy
        if num_gpu_blocks < 0 or block_size < 0:
            raise OverflowError("can't convert negative int to unsigned")
        h = ctypes.c_void_p()
        _lib.check(L.zk_bm_create(num_gpu_blocks, block_size, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_h", None) and destroy is not None:
            destroy(self._h)
            self._h = None

    @property
    def handle(self) -> ctypes.c_void_p:
        """The zk_block_manager* for the C ABI."""
        return self._h

    # -- pymethods --------------------------------------------------------
    def allocate(self) -> BlockHandle:
        out = _lib.BlockHandleC()
        _lib.check(_lib.lib().zk_bm_allocate(self._h, ctypes.byref(out)))
        return BlockHandle(out.block_id, out.generation)

    def free(self, handle: BlockHandle) -> None:
        _lib.check(_lib.lib().zk_bm_free(self._h, handle._c()))

    def reference(self, handle: BlockHandle) -> None:
        _lib.check(_lib.lib().zk_bm_reference(self._h, handle._c()))

    @property
    def free_blocks(self) -> int:
        return int(_lib.lib().zk_bm_available(self._h))

    @property
    def num_gpu_blocks(self) -> int:
        return int(_lib.lib().zk_bm_num_gpu_blocks(self._h))

    @property
    def block_size(self) -> int:
        return int(_lib.lib().zk_bm_block_size(self._h))

    # -- Rust-native names --------------------------------------------------
    try_allocate = allocate
    try_free = free
    try_reference = reference

    def available(self) -> int:
        return self.free_blocks

    def refcount(self, block_id: int) -> int:
        return int(_lib.lib().zk_bm_refcount(self._h, block_id))
