"""Reference model of Zealot's BlockManager -- TEST INFRASTRUCTURE ONLY.

Restates the semantics of src/block_manager.rs:88-164 (create / try_allocate /
try_free / try_reference / check) in the shape of the model used by the
reference's property test (tests/block_manager_proptest.rs:43-137): a LIFO free
stack built as ``reversed(range(n))`` plus a per-block state that is either
``("free", generation)`` or ``("alloc", refcount, generation)``.  Generations
persist across free/allocate cycles and start at 1.

Used only by tests/ as the checker of the product's C++ BlockManager.
"""
from __future__ import annotations


class ModelError(Exception):
    def __init__(self, kind: str, **detail):
        super().__init__(kind)
        self.kind = kind
        self.detail = detail


class BlockManagerModel:
    def __init__(self, num_blocks: int, block_size: int = 16):
        if block_size == 0:  # block_manager.rs:89-91
            raise ModelError("InvalidBlockSize", block_size=block_size)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.free_stack = list(reversed(range(num_blocks)))  # block_manager.rs:93-95
        self.state = [("free", 1) for _ in range(num_blocks)]  # generation starts at 1

    def available(self) -> int:
        return len(self.free_stack)

    def allocated_count(self) -> int:
        return sum(1 for s in self.state if s[0] == "alloc")

    def _check(self, block_id: int, generation: int):
        # block_manager.rs:151-164: id range first, then generation.
        if block_id >= self.num_blocks:
            raise ModelError("BlockNotAllocated", block_id=block_id)
        cur = self.state[block_id][-1]
        if generation != cur:
            raise ModelError("StaleHandle", block_id=block_id, handle_gen=generation,
                             current_gen=cur)

    def allocate(self):
        # block_manager.rs:108-122
        if not self.free_stack:
            raise ModelError("OutOfBlocks", requested=1, available=0)
        bid = self.free_stack.pop()
        gen = self.state[bid][-1]
        self.state[bid] = ("alloc", 1, gen)
        return bid, gen

    def free(self, block_id: int, generation: int) -> bool:
        """Returns True when the block went back to the pool (block_manager.rs:125-135)."""
        self._check(block_id, generation)
        st = self.state[block_id]
        if st[0] != "alloc":
            # Only a forged handle (BlockHandle(id, gen) built by hand for a block
            # that is free) gets here.  The reference's fetch_sub would wrap the
            # refcount; the product rejects it as BlockNotAllocated instead.
            raise ModelError("BlockNotAllocated", block_id=block_id)
        rc, gen = st[1], st[2]
        if rc == 1:
            self.state[block_id] = ("free", gen + 1)
            self.free_stack.append(block_id)
            return True
        self.state[block_id] = ("alloc", rc - 1, gen)
        return False

    def reference(self, block_id: int, generation: int) -> None:
        # block_manager.rs:140-144
        self._check(block_id, generation)
        st = self.state[block_id]
        if st[0] != "alloc":
            raise ModelError("BlockNotAllocated", block_id=block_id)
        self.state[block_id] = ("alloc", st[1] + 1, st[2])

    def refcount(self, block_id: int) -> int:
        st = self.state[block_id]
        return st[1] if st[0] == "alloc" else 0
