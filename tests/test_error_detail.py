"""Typed error payloads at the C boundary (zk_last_error_detail).

The reference's ZealotError variants carry fields (src/error.rs:4-37):
StaleHandle{block_id, handle_gen, current_gen}, OutOfBlocks{requested,
available}, SequenceTooLong{required, capacity}, BlockNotAllocated(id),
InvalidBlockSize(size).  A Rust caller of the C ABI rebuilds each variant
from the status code and zk_last_error_detail's three fields; these tests
check the fields for every variant the path raises, on the CPU (BlockManager
and scheduler calls need no GPU)."""
import ctypes
import threading

import pytest

from zealot_amd import BlockManager, ZealotError, _lib
from zealot_amd.scheduler import Scheduler, SchedulerConfig


def detail():
    f = (ctypes.c_uint64 * 3)()
    code = _lib.lib().zk_last_error_detail(f)
    return code, tuple(int(x) for x in f)


def bm_c(n, bs):
    h = ctypes.c_void_p()
    assert _lib.lib().zk_bm_create(n, bs, ctypes.byref(h)) == 0
    return h


def handle(i, g):
    return _lib.BlockHandleC(i, g)


def test_stale_handle_fields():
    L = _lib.lib()
    bm = bm_c(4, 16)
    h = _lib.BlockHandleC()
    assert L.zk_bm_allocate(bm, ctypes.byref(h)) == 0
    assert L.zk_bm_free(bm, h) == 0                       # generation 1 -> 2
    assert L.zk_bm_reference(bm, h) == _lib.ERR_STALE_HANDLE
    assert detail() == (_lib.ERR_STALE_HANDLE, (h.block_id, 1, 2))
    assert L.zk_last_error().decode() == f"Stale handle: block {h.block_id} was freed (gen 1, current 2)"
    # reading the message does not consume the fields
    assert detail() == (_lib.ERR_STALE_HANDLE, (h.block_id, 1, 2))
    L.zk_bm_destroy(bm)


def test_out_of_blocks_fields():
    L = _lib.lib()
    bm = bm_c(1, 16)
    h = _lib.BlockHandleC()
    assert L.zk_bm_allocate(bm, ctypes.byref(h)) == 0
    assert L.zk_bm_allocate(bm, ctypes.byref(h)) == _lib.ERR_OUT_OF_BLOCKS
    assert detail() == (_lib.ERR_OUT_OF_BLOCKS, (1, 0, 0))  # block_manager.rs:113-116
    assert L.zk_last_error().decode() == "Out of blocks: requested 1, available 0"
    L.zk_bm_destroy(bm)


def test_block_not_allocated_fields():
    L = _lib.lib()
    bm = bm_c(4, 16)
    assert L.zk_bm_free(bm, handle(7, 1)) == _lib.ERR_BLOCK_NOT_ALLOCATED   # id >= n
    assert detail() == (_lib.ERR_BLOCK_NOT_ALLOCATED, (7, 0, 0))
    assert L.zk_last_error().decode() == "Block 7 is not allocated"
    assert L.zk_bm_check(bm, handle(2, 1)) == _lib.ERR_BLOCK_NOT_ALLOCATED  # live gen, free block
    assert detail() == (_lib.ERR_BLOCK_NOT_ALLOCATED, (2, 0, 0))
    L.zk_bm_destroy(bm)


def test_invalid_block_size_fields():
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.zk_bm_create(4, 0, ctypes.byref(h)) == _lib.ERR_INVALID_BLOCK_SIZE
    assert detail() == (_lib.ERR_INVALID_BLOCK_SIZE, (0, 0, 0))
    assert L.zk_last_error().decode() == "Invalid block size: 0"


def test_sequence_too_long_fields():
    # scheduler.rs:234-240: worst case = ceil((prompt + max_tokens) / block_size) blocks
    s = Scheduler(SchedulerConfig(block_size=16, num_gpu_blocks=8))
    with pytest.raises(ZealotError) as e:
        s.make_sequence("r", list(range(100)), 50)
    assert e.value.code == _lib.ERR_SEQUENCE_TOO_LONG
    assert e.value.fields == {"required": 10, "capacity": 8}
    assert str(e.value) == "Sequence too long: worst case needs 10 blocks, pool capacity is 8"
    assert detail() == (_lib.ERR_SEQUENCE_TOO_LONG, (10, 8, 0))


def test_untyped_errors_have_no_fields():
    L = _lib.lib()
    rc = L.zk_append(None, None, 7, None, None, _lib.BF16, None, 4, 8, 128, 16, 10, None, None, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert detail() == (_lib.ERR_INVALID_ARGUMENT, (0, 0, 0))
    assert "dtype" in L.zk_last_error().decode()


def test_python_error_carries_fields():
    bm = BlockManager(2, 16)
    h = bm.allocate()
    bm.free(h)
    with pytest.raises(ZealotError) as e:
        bm.free(h)
    assert e.value.code == _lib.ERR_STALE_HANDLE
    assert e.value.fields == {"block_id": h.block_id, "handle_gen": 1, "current_gen": 2}
    bm2 = BlockManager(1, 16)
    bm2.allocate()
    with pytest.raises(RuntimeError) as e:  # still a RuntimeError, as error.rs:48-52
        bm2.allocate()
    assert e.value.fields == {"requested": 1, "available": 0}


def test_last_error_survives_success_and_is_per_thread():
    L = _lib.lib()
    bm = bm_c(2, 16)
    assert L.zk_bm_free(bm, handle(9, 1)) == _lib.ERR_BLOCK_NOT_ALLOCATED
    h = _lib.BlockHandleC()
    assert L.zk_bm_allocate(bm, ctypes.byref(h)) == 0       # a success leaves the last failure
    assert detail() == (_lib.ERR_BLOCK_NOT_ALLOCATED, (9, 0, 0))
    seen = {}

    def other():
        seen["before"] = detail()
        L.zk_bm_reference(bm, handle(h.block_id, 5))        # stale on this thread only
        seen["after"] = detail()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == (_lib.OK, (0, 0, 0))
    assert seen["after"] == (_lib.ERR_STALE_HANDLE, (h.block_id, 5, 1))
    assert detail() == (_lib.ERR_BLOCK_NOT_ALLOCATED, (9, 0, 0))
    L.zk_bm_destroy(bm)


def test_null_fields_pointer():
    L = _lib.lib()
    L.zk_bm_create(4, 0, ctypes.byref(ctypes.c_void_p()))
    assert L.zk_last_error_detail(None) == _lib.ERR_INVALID_BLOCK_SIZE
