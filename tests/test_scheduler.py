"""The scheduler (src/scheduler.rs) through the C ABI, host only.

The first group restates the reference's own unit tests
(scheduler.rs:484-806) case by case; the rest cover what this build adds:
a BlockManager shared with the KV cache, the per-entry step geometry the
runner binds (num_tokens, tokens_before, blocks), step_input of a multi-chunk
recompute, and rejected duplicate ids."""
import pytest

from zealot_amd import BlockManager, CancelOutcome, Priority, Scheduler, SchedulerConfig, ZealotError
from zealot_amd import _lib


def cfg(max_num_seqs, block_size, num_gpu_blocks):  # scheduler.rs:484-492
    return SchedulerConfig(max_num_seqs, block_size, num_gpu_blocks, max_prefill_tokens=1024,
                           prefill_chunk_size=512)


def submit(s, rid, prompt_len, max_tokens, priority=Priority.Medium):
    s.add(s.make_sequence(rid, [1] * prompt_len, max_tokens, priority))


def ids(out):
    return [e.request_id for e in out.batch]


# ---------------------------------------------------------------- reference tests
def test_promotion_respects_max_num_seqs():  # scheduler.rs:515-524
    s = Scheduler(cfg(1, 2, 16))
    submit(s, "a", 2, 2)
    submit(s, "b", 2, 2)
    out = s.schedule()
    assert ids(out) == ["a"]


def test_priority_jumps_queue():  # scheduler.rs:526-534
    s = Scheduler(cfg(1, 2, 16))
    submit(s, "low", 2, 2, Priority.Lowest)
    submit(s, "top", 2, 2, Priority.Highest)
    assert ids(s.schedule()) == ["top"]


def test_waiting_when_blocks_exhausted():  # scheduler.rs:536-547
    s = Scheduler(cfg(8, 2, 2))
    for r in "abc":
        submit(s, r, 2, 2)
    assert ids(s.schedule()) == ["a", "b"]


def test_admission_control_rejects_oversized_sequence():  # scheduler.rs:549-564
    s = Scheduler(cfg(8, 2, 2))
    with pytest.raises(ZealotError) as e:
        s.make_sequence("huge", [1] * 2, 8, Priority.Medium)
    assert e.value.code == _lib.ERR_SEQUENCE_TOO_LONG


def test_preemption_frees_blocks_and_resumes():  # scheduler.rs:566-611
    s = Scheduler(cfg(2, 2, 4))
    submit(s, "a", 4, 4)
    submit(s, "b", 2, 2)
    out = s.schedule()
    assert len(out.batch) == 2
    assert s.free_blocks() == 1
    out = s.schedule()
    a = next(e for e in out.batch if e.request_id == "a")
    a.push_token(10)
    a.push_token(11)
    a.mark_prefilled()
    s.schedule()
    assert s.free_blocks() == 0
    out = s.schedule()
    b = next(e for e in out.batch if e.request_id == "b")
    b.push_token(20)
    b.mark_prefilled()
    out = s.schedule()
    assert out.preempted == ["a"]
    assert s.free_blocks() == 2
    s.finish("b")
    out = s.schedule()
    a = next(e for e in out.batch if e.request_id == "a")
    assert a.is_prefill(), "preempted seq must re-prefill (recompute)"
    assert len(a.step_input()) == 6, "prompt 4 + preserved output 2"


def test_cancel_waiting_and_running():  # scheduler.rs:613-625
    s = Scheduler(cfg(1, 2, 16))
    submit(s, "a", 2, 2)
    submit(s, "b", 2, 2)
    s.schedule()
    assert s.cancel("b") == (CancelOutcome.WasWaiting, 2, 0)
    assert s.cancel("a") == (CancelOutcome.WasRunning, 2, 0)
    assert s.cancel("ghost")[0] == CancelOutcome.NotFound
    assert s.is_idle()
    assert s.free_blocks() == 16


def test_finish_releases_all_blocks():  # scheduler.rs:627-638
    s = Scheduler(cfg(8, 2, 4))
    submit(s, "a", 4, 2)
    s.schedule()
    assert s.free_blocks() == 2
    assert s.finish("a") == (4, 0)
    assert s.free_blocks() == 4
    assert s.is_idle()


def _chunk_cfg(chunk):
    return SchedulerConfig(max_num_seqs=8, block_size=2, num_gpu_blocks=1024, max_prefill_tokens=512,
                           prefill_chunk_size=chunk)


def test_chunked_prefill_splits_long_prompt():  # scheduler.rs:640-688
    s = Scheduler(_chunk_cfg(256))
    submit(s, "a", 1024, 4)
    for final in (False, False, False, True):
        out = s.schedule()
        assert len(out.batch) == 1
        assert out.batch[0].is_prefill()
        assert out.batch[0].is_final_chunk() == final
        s.advance_prefill("a")
    out = s.schedule()
    assert len(out.batch) == 1 and not out.batch[0].is_prefill()


def test_chunked_prefill_short_prompt_still_one_step():  # scheduler.rs:690-713
    s = Scheduler(_chunk_cfg(256))
    submit(s, "a", 128, 4)
    out = s.schedule()
    assert len(out.batch) == 1 and out.batch[0].is_final_chunk()


def test_chunked_prefill_interleaves_with_decode():  # scheduler.rs:715-769
    s = Scheduler(_chunk_cfg(256))
    submit(s, "a", 512, 4)
    submit(s, "b", 128, 4)
    out = s.schedule()
    assert len(out.batch) == 2
    a, b = (next(e for e in out.batch if e.request_id == r) for r in "ab")
    assert a.is_prefill() and not a.is_final_chunk()
    assert b.is_prefill() and b.is_final_chunk()
    s.advance_prefill("a")
    s.advance_prefill("b")
    out = s.schedule()
    assert len(out.batch) == 2
    a, b = (next(e for e in out.batch if e.request_id == r) for r in "ab")
    assert a.is_prefill() and a.is_final_chunk()
    assert not b.is_prefill()


def test_advance_prefill_tracks_position():  # scheduler.rs:771-805
    s = Scheduler(_chunk_cfg(100))
    submit(s, "a", 300, 4)
    for _ in range(3):
        s.schedule()
        s.advance_prefill("a")
    out = s.schedule()
    assert len(out.batch) == 1
    assert not out.batch[0].is_prefill(), "should be in decoding after 3 chunks complete"


# ---------------------------------------------------------------- additions
def test_shared_block_manager_sees_the_schedulers_blocks():
    bm = BlockManager(16, 4)
    s = Scheduler(SchedulerConfig(4, 4, 16, 64, 8), block_manager=bm)
    submit(s, "a", 10, 4)  # chunk 8 -> 2 blocks
    out = s.schedule()
    assert bm.free_blocks == 14
    (e,) = out.batch
    assert [bm.refcount(h.block_id) for h in e.blocks] == [1, 1]
    # a handle the scheduler frees goes stale for everyone
    s.finish("a")
    assert bm.free_blocks == 16
    with pytest.raises(ZealotError) as err:
        bm.free(e.blocks[0])
    assert err.value.code == _lib.ERR_STALE_HANDLE


def test_shared_block_manager_must_match_config():
    bm = BlockManager(16, 4)
    with pytest.raises(ZealotError) as e:
        Scheduler(SchedulerConfig(4, 8, 16, 64, 8), block_manager=bm)
    assert e.value.code == _lib.ERR_FAILED_PRECONDITION


def test_destroy_returns_blocks_to_a_shared_manager():
    bm = BlockManager(16, 4)
    s = Scheduler(SchedulerConfig(4, 4, 16, 64, 8), block_manager=bm)
    submit(s, "a", 10, 4)
    submit(s, "b", 3, 4)
    s.schedule()
    assert bm.free_blocks < 16
    del s
    assert bm.free_blocks == 16


def test_step_geometry_of_chunks_and_decodes():
    """num_tokens / tokens_before / len / blocks per entry over a chunked
    prompt and its decode steps."""
    s = Scheduler(SchedulerConfig(max_num_seqs=4, block_size=4, num_gpu_blocks=64, max_prefill_tokens=64,
                                  prefill_chunk_size=8))
    submit(s, "a", 19, 8)
    seen = []
    for step in range(3):  # chunks 8, 8, 3
        (e,) = s.schedule().batch
        seen.append((e.num_tokens, e.tokens_before, e.len(), len(e.blocks), e.is_final_chunk()))
        if e.is_final_chunk():
            e.push_token(100 + step)
            e.mark_prefilled()
        s.advance_prefill("a")
    assert seen == [(8, 0, 8, 2, False), (8, 8, 16, 4, False), (3, 16, 19, 5, True)]
    for t in range(3):  # decodes at positions 19, 20, 21
        (e,) = s.schedule().batch
        assert (e.num_tokens, e.tokens_before, e.len(), e.is_prefill()) == (1, 19 + t, 20 + t, False)
        assert len(e.blocks) == (20 + t + 3) // 4
        assert e.step_input() == [100 + 2 + t]
        e.push_token(103 + t)


def _engine_write_back(e, token):
    """engine.rs:229-291 for one entry: a token on decodes and final chunks."""
    if not e.is_prefill() or e.is_final_chunk():
        e.push_token(token())
    if e.is_prefill() and e.is_final_chunk():
        e.mark_prefilled()


def _recompute_case():
    """b (High) and a (Lowest) decode until b's growth preempts a; pool of 6
    blocks of 2 tokens, chunks of 4."""
    s = Scheduler(SchedulerConfig(max_num_seqs=2, block_size=2, num_gpu_blocks=6, max_prefill_tokens=64,
                                  prefill_chunk_size=4))
    s.add(s.make_sequence("b", [9, 9], 4, Priority.High))
    s.add(s.make_sequence("a", list(range(6)), 2, Priority.Lowest))
    tok = iter(range(50, 100))
    for step in range(4):
        out = s.schedule()
        for e in out.batch:
            _engine_write_back(e, (lambda: next(tok)) if e.request_id == "a" else (lambda: 20 + step))
        for e in out.batch:
            if e.is_prefill():
                s.advance_prefill(e.request_id)
    return s, out


def test_multi_chunk_recompute_feeds_outputs_after_the_prompt():
    s, out = _recompute_case()
    assert out.preempted == ["a"]
    assert s.seq_info("a")["output_len"] == 2 and s.seq_info("a")["state"] == 0
    out = s.schedule()  # a re-admitted: first chunk of its recompute
    (e,) = [x for x in out.batch if x.request_id == "a"]
    assert e.is_prefill() and not e.is_final_chunk()
    assert e.step_input() == [0, 1, 2, 3] and (e.num_tokens, e.tokens_before) == (4, 0)
    s.advance_prefill("a")
    s.finish("b")
    (e,) = [x for x in s.schedule().batch if x.request_id == "a"]
    assert e.is_final_chunk()
    # the reference would give [4, 5, 50, 51] here too, and [0, 1, 2, 3, 50, 51] above
    assert e.step_input() == [4, 5, 50, 51] and (e.num_tokens, e.tokens_before) == (4, 4)
    assert len(e.blocks) == 4


def test_sequence_short_of_blocks_waits():
    """With no victim left the top-up stops (scheduler.rs:386); the sequence
    then stays out of the batch instead of running without its blocks."""
    s, out = _recompute_case()
    s.schedule()  # a re-admitted with the 3 free blocks
    s.advance_prefill("a")
    out = s.schedule()  # a's final chunk needs a 4th block; b is in the other queue
    assert [e.request_id for e in out.batch] == ["b"]
    assert s.seq_info("a")["num_blocks"] == 3
    s.finish("b")
    out = s.schedule()
    (e,) = out.batch
    assert e.request_id == "a" and e.is_final_chunk() and len(e.blocks) == 4


def test_duplicate_ids_are_rejected():
    s = Scheduler(cfg(4, 2, 16))
    submit(s, "a", 2, 2)
    seq = s.make_sequence("a", [1, 2], 2)
    with pytest.raises(ZealotError) as e:
        s.add(seq)
    assert e.value.code == _lib.ERR_ALREADY_EXISTS
    s.schedule()
    with pytest.raises(ZealotError):
        s.add(s.make_sequence("a", [1], 1))


# ---------------------------------------------------------------- swap preemption
def _swap_case(swap_blocks):
    """_recompute_case's pool (6 blocks of 2 tokens) with host swap space."""
    s = Scheduler(SchedulerConfig(max_num_seqs=2, block_size=2, num_gpu_blocks=6, max_prefill_tokens=64,
                                  prefill_chunk_size=4, swap_blocks=swap_blocks))
    s.add(s.make_sequence("b", [9, 9], 4, Priority.High))
    s.add(s.make_sequence("a", list(range(6)), 2, Priority.Lowest))
    tok = iter(range(50, 100))
    for step in range(4):
        out = s.schedule()
        for e in out.batch:
            _engine_write_back(e, (lambda: next(tok)) if e.request_id == "a" else (lambda: 20 + step))
        for e in out.batch:
            if e.is_prefill():
                s.advance_prefill(e.request_id)
    return s, out


def test_swap_preemption_keeps_progress():
    s, out = _swap_case(swap_blocks=8)
    assert out.preempted == [] and out.swapped_out == ["a"]
    info = s.seq_info("a")
    assert info["swapped"] == 1 and info["state"] == 0 and not info["is_prefill"] and info["output_len"] == 2
    assert s.free_blocks() == 3  # a's 4 blocks went back; b took one more
    s.finish("b")
    out = s.schedule()
    assert out.swapped_in == ["a"] and out.swapped_out == []
    (e,) = out.batch
    # straight back to decoding: prompt 6 + outputs 2, the last output is the input
    assert (e.request_id, e.is_prefill(), e.num_tokens, e.tokens_before, e.len()) == ("a", False, 1, 7, 8)
    assert e.step_input() == [51] and len(e.blocks) == 4


def test_swap_space_full_falls_back_to_recompute():
    s, out = _swap_case(swap_blocks=3)  # a's KV (7 tokens) needs 4 host blocks
    assert out.swapped_out == [] and out.preempted == ["a"]
    assert s.seq_info("a")["swapped"] == 0 and s.seq_info("a")["is_prefill"]


def test_swap_mid_prefill_resumes_at_its_position():
    """A sequence swapped while its prompt is half done resumes the prompt
    where it stopped (the reference restarts it from token 0).  Two 24-token
    prompts in chunks of 8 over 8 blocks of 4: the high-priority one's third
    chunk needs the low one's blocks."""
    s = Scheduler(SchedulerConfig(max_num_seqs=2, block_size=4, num_gpu_blocks=8, max_prefill_tokens=64,
                                  prefill_chunk_size=8, swap_blocks=16))
    s.add(s.make_sequence("lo", list(range(100, 124)), 2, Priority.Lowest))
    s.add(s.make_sequence("hi", list(range(24)), 2, Priority.High))
    for _ in range(2):
        out = s.schedule()
        assert sorted(e.request_id for e in out.batch) == ["hi", "lo"]
        for e in out.batch:
            s.advance_prefill(e.request_id)
    out = s.schedule()
    assert out.swapped_out == ["lo"] and out.preempted == []
    info = s.seq_info("lo")
    assert info["swapped"] == 1 and info["is_prefill"] and info["prefill_pos"] == 16
    s.finish("hi")
    out = s.schedule()
    assert out.swapped_in == ["lo"]
    (e,) = out.batch
    assert e.is_prefill() and e.is_final_chunk() and e.tokens_before == 16
    assert e.step_input() == list(range(116, 124)) and len(e.blocks) == 6


def test_cancel_of_a_swapped_sequence_returns_its_host_space():
    s, out = _swap_case(swap_blocks=4)
    assert out.swapped_out == ["a"]
    assert s.cancel("a")[0] == CancelOutcome.WasWaiting
    # the host space is free again: the same preemption swaps instead of recomputing
    s.add(s.make_sequence("c", list(range(6)), 2, Priority.Lowest))
    s.finish("b")
    assert s.seq_info("c")["swapped"] == 0
