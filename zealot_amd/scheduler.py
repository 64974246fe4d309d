"""Continuous-batching scheduler over the C ABI (include/zealot_sched.h) -- the
host mirror of src/scheduler.rs:15-478.

Names and argument meaning follow the reference: SchedulerConfig, Priority,
Scheduler.make_sequence / add / schedule / finish / promote_to_decoding /
advance_prefill / cancel / is_idle, and batch entries with is_prefill(),
is_final_chunk(), step_input(), len().  The queues and block bookkeeping live
in C++ (zealot_amd/csrc/scheduler.cpp).  The BlockManager may be shared with a
KVCache (Scheduler(cfg, block_manager=bm)), in which case each batch entry's
`blocks` are the handles the KV cache binds as the sequence's block table.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass

from . import _lib
from .block_manager import BlockHandle, BlockManager


class Priority(enum.IntEnum):
    """scheduler.rs:15-21."""
    Lowest = 0
    Medium = 1
    High = 2
    Highest = 3


@dataclass
class SchedulerConfig:
    """scheduler.rs:156-178 (defaults of impl Default)."""
    max_num_seqs: int = 8
    block_size: int = 16
    num_gpu_blocks: int = 1024
    max_prefill_tokens: int = 2048
    prefill_chunk_size: int = 512
    swap_blocks: int = 0  # host swap space (0: recompute only, the reference's policy)

    def _c(self) -> _lib.SchedConfigC:
        return _lib.SchedConfigC(self.max_num_seqs, self.block_size, self.num_gpu_blocks,
                                 self.max_prefill_tokens, self.prefill_chunk_size, self.swap_blocks)


class CancelOutcome(enum.IntEnum):
    """scheduler.rs:191-197."""
    NotFound = 0
    WasWaiting = 1
    WasRunning = 2


class PendingSequence:
    """A Sequence made by make_sequence and not yet added (scheduler.rs:225-253)."""

    def __init__(self, ptr: ctypes.c_void_p, request_id: str):
        # bound now: at interpreter exit the module globals may already be gone
        self._destroy = _lib.lib().zk_sequence_destroy
        self._p = ptr
        self.request_id = request_id

    def __del__(self):
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_p", None) and destroy is not None:
            destroy(self._p)
            self._p = None


class Sequence:
    """A batch entry of schedule(): a snapshot of the sequence at that step
    (scheduler.rs:51-153); the write-backs go to the scheduler by id."""

    def __init__(self, sched: "Scheduler", e: _lib.SchedEntryC):
        self._s = sched
        self.request_id = e.request_id.decode()
        self._prefill = bool(e.is_prefill)
        self._final = bool(e.is_final_chunk)
        self.num_tokens = int(e.num_tokens)        # tokens fed this step
        self.tokens_before = int(e.tokens_before)  # KV tokens held before this step
        self._len = int(e.len)
        self.blocks = [BlockHandle(e.blocks[i].block_id, e.blocks[i].generation) for i in range(e.num_blocks)]

    def is_prefill(self) -> bool:
        return self._prefill

    def is_final_chunk(self) -> bool:
        return self._final

    def len(self) -> int:
        return self._len

    def __len__(self) -> int:
        return self._len

    def step_input(self) -> list:
        return self._s.step_input(self.request_id)

    def push_token(self, token: int) -> None:
        """output_tokens.push (engine.rs write-back)."""
        _lib.check(_lib.lib().zk_sched_push_token(self._s._h, self.request_id.encode(), int(token)))

    def mark_prefilled(self) -> None:
        _lib.check(_lib.lib().zk_sched_mark_prefilled(self._s._h, self.request_id.encode()))


@dataclass
class ScheduleOutput:
    """scheduler.rs:185-189, plus the sequences preempted by swap this step
    and those re-admitted from swap."""
    batch: list
    preempted: list
    swapped_out: list = None
    swapped_in: list = None


class Scheduler:
    """scheduler.rs:199-478 over a private or shared BlockManager."""

    def __init__(self, cfg: SchedulerConfig | None = None, block_manager: BlockManager | None = None):
        self._h = None
        self.cfg = cfg or SchedulerConfig()
        self._bm = block_manager  # keeps a shared manager alive
        self._destroy = _lib.lib().zk_sched_destroy  # bound now, for __del__ at interpreter exit
        h = ctypes.c_void_p()
        c = self.cfg._c()
        _lib.check(_lib.lib().zk_sched_create(ctypes.byref(c), block_manager.handle if block_manager else None,
                                              ctypes.byref(h)))
        self._h = h

    def __del__(self):
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_h", None) and destroy is not None:
            destroy(self._h)
            self._h = None

    def make_sequence(self, request_id: str, prompt_tokens, max_tokens: int,
                      priority: Priority = Priority.Medium) -> PendingSequence:
        toks = [int(t) for t in prompt_tokens]
        arr = (ctypes.c_int64 * max(1, len(toks)))(*toks)
        out = ctypes.c_void_p()
        _lib.check(_lib.lib().zk_sched_make_sequence(self._h, request_id.encode(), arr, len(toks), int(max_tokens),
                                                     int(priority), ctypes.byref(out)))
        return PendingSequence(out, request_id)

    def add(self, seq: PendingSequence) -> None:
        if not seq._p:
            raise ValueError("sequence was already added")
        _lib.check(_lib.lib().zk_sched_add(self._h, seq._p))
        seq._p = None  # owned by the scheduler now

    def submit(self, request_id: str, prompt_tokens, max_tokens: int, priority: Priority = Priority.Medium):
        self.add(self.make_sequence(request_id, prompt_tokens, max_tokens, priority))

    def schedule(self) -> ScheduleOutput:
        out = _lib.SchedOutputC()
        _lib.check(_lib.lib().zk_sched_schedule(self._h, ctypes.byref(out)))
        batch = [Sequence(self, out.batch[i]) for i in range(out.batch_len)]
        pre = [out.preempted[i].decode() for i in range(out.num_preempted)]
        so = [out.swapped_out[i].decode() for i in range(out.num_swapped_out)]
        si = [out.swapped_in[i].decode() for i in range(out.num_swapped_in)]
        return ScheduleOutput(batch, pre, so, si)

    def finish(self, request_id: str):
        p, o = ctypes.c_size_t(), ctypes.c_size_t()
        if _lib.lib().zk_sched_finish(self._h, request_id.encode(), ctypes.byref(p), ctypes.byref(o)):
            return p.value, o.value
        return None

    def promote_to_decoding(self, request_id: str) -> None:
        _lib.lib().zk_sched_promote_to_decoding(self._h, request_id.encode())

    def advance_prefill(self, request_id: str) -> None:
        _lib.lib().zk_sched_advance_prefill(self._h, request_id.encode())

    def cancel(self, request_id: str):
        """(CancelOutcome, prompt_len, output_len)."""
        p, o = ctypes.c_size_t(), ctypes.c_size_t()
        r = CancelOutcome(_lib.lib().zk_sched_cancel(self._h, request_id.encode(), ctypes.byref(p), ctypes.byref(o)))
        if r == CancelOutcome.NotFound:
            return r, 0, 0
        return r, p.value, o.value

    def is_idle(self) -> bool:
        return bool(_lib.lib().zk_sched_is_idle(self._h))

    def free_blocks(self) -> int:
        return int(_lib.lib().zk_bm_available(_lib.lib().zk_sched_block_manager(self._h)))

    def step_input(self, request_id: str) -> list:
        n = ctypes.c_size_t(0)
        L = _lib.lib()
        rc = L.zk_sched_step_input(self._h, request_id.encode(), None, ctypes.byref(n))
        if rc != _lib.OK and n.value == 0:
            _lib.check(rc)
        buf = (ctypes.c_int64 * max(1, n.value))()
        _lib.check(L.zk_sched_step_input(self._h, request_id.encode(), buf, ctypes.byref(n)))
        return list(buf[:n.value])

    def seq_info(self, request_id: str) -> dict:
        info = _lib.SchedSeqInfoC()
        _lib.check(_lib.lib().zk_sched_seq_info(self._h, request_id.encode(), ctypes.byref(info)))
        return {f: getattr(info, f) for f, _ in info._fields_}
