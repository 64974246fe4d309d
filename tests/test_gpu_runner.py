"""Scheduler -> KV wiring on the MI355X: the scheduler (src/scheduler.rs) and
the KV cache share one BlockManager, and a PagedKVRunner turns each
schedule() batch into one bind, one write and one attention call per layer.

An engine loop in the shape of engine.rs:127-291 runs six requests through a
pool small enough to force preemptions (recompute) and chunked prefills
mixed with decodes.  Every layer of every step is checked against the
oracle's chunked prefill over the cache's pools, with each entry's block
table taken from the scheduler's handles and its chunk starting at
tokens_before; the pool bytes of every sequence in the batch equal the
tokens written since its last admission.  At the end every block is back in
the manager and the cache holds no sequence.  Tolerance 2e-2 (bf16)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, normal, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_scheduler_runner_engine_loop():
    import zealot_amd as ze
    from zealot_amd import KVCache, PagedKVRunner, Priority, Scheduler, SchedulerConfig
    rng = np.random.default_rng(77)
    L, H, Hkv, D, BS, NB, MB = 2, 16, 4, 128, 16, 28, 32
    bm = ze.BlockManager(NB, BS)
    sched = Scheduler(SchedulerConfig(max_num_seqs=4, block_size=BS, num_gpu_blocks=NB, max_prefill_tokens=256,
                                      prefill_chunk_size=96), block_manager=bm)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=8, max_blocks_per_seq=MB)
    runner = PagedKVRunner(cache, bm)
    prompts, max_tokens = [40, 150, 200, 17, 300, 90], [6, 10, 8, 12, 5, 9]
    prios = [Priority.Medium, Priority.High, Priority.Lowest, Priority.Medium, Priority.Highest, Priority.Lowest]
    for i, (p, m, pr) in enumerate(zip(prompts, max_tokens, prios)):
        sched.add(sched.make_sequence(f"r{i}", list(rng.integers(0, 1000, p)), m, pr))
    written = {}  # rid -> layer -> list of (k, v) rows since the last admission
    scale = np.float32(1 / math.sqrt(D))
    preemptions = mixed = steps = 0
    finished = []
    while not sched.is_idle():
        steps += 1
        assert steps < 200
        out = sched.schedule()
        for rid in out.preempted:
            written.pop(rid, None)
        preemptions += len(out.preempted)
        plan = runner.begin_step(out)
        batch = out.batch
        if not batch:
            continue
        kinds = {e.is_prefill() for e in batch}
        mixed += len(kinds) == 2
        nt = [e.num_tokens for e in batch]
        cu = np.concatenate([[0], np.cumsum(nt)]).astype(np.int64)
        bt = -np.ones((len(batch), MB), np.int32)
        for i, e in enumerate(batch):
            bt[i, :len(e.blocks)] = [h.block_id for h in e.blocks]
            if e.tokens_before == 0:
                written[e.request_id] = {l: [] for l in range(L)}
        announce(f"runner step {steps}: {[(e.request_id, e.num_tokens, e.tokens_before) for e in batch]}")
        for layer in range(L):
            k = normal(rng, (plan.total_tokens, Hkv, D), oracle.BF16)
            v = normal(rng, (plan.total_tokens, Hkv, D), oracle.BF16)
            q = normal(rng, (plan.total_tokens, H, D), oracle.BF16)
            runner.write(layer, plan, to_dev(k), to_dev(v))
            o = to_host(runner.attention(layer, plan, to_dev(q)))
            for i, e in enumerate(batch):
                written[e.request_id][layer].append((k[cu[i]:cu[i + 1]], v[cu[i]:cu[i + 1]]))
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            ref = oracle.paged_prefill(as_f32(q, oracle.BF16), kp, vp, oracle.BF16, bt, cu,
                                       [e.tokens_before for e in batch], Hkv, D, BS, scale, True)
            assert max_abs_err(as_f32(o, oracle.BF16), ref) <= 2e-2, (steps, layer)
            for i, e in enumerate(batch):  # pool bytes of the sequence == its writes
                T = e.tokens_before + e.num_tokens
                kk = np.concatenate([a for a, _ in written[e.request_id][layer]])
                vv = np.concatenate([b for _, b in written[e.request_id][layer]])
                assert kk.shape[0] == T, (e.request_id, T)
                gk = oracle.gather(kp, oracle.BF16, bt[i], T, Hkv, D, BS, np.uint16)
                gv = oracle.gather(vp, oracle.BF16, bt[i], T, Hkv, D, BS, np.uint16)
                assert np.array_equal(gk, kk) and np.array_equal(gv, vv), (steps, layer, e.request_id)
        # engine write-back (engine.rs:229-291)
        for e in batch:
            if not e.is_prefill() or e.is_final_chunk():
                e.push_token(int(rng.integers(0, 1000)))
                if e.is_prefill():
                    e.mark_prefilled()
        for e in batch:
            if e.is_prefill():
                sched.advance_prefill(e.request_id)
        for e in batch:
            info = sched.seq_info(e.request_id)
            if info["state"] == 1 and info["output_len"] >= max_tokens[int(e.request_id[1:])]:
                runner.drop_state(e.request_id)
                assert sched.finish(e.request_id) is not None
                finished.append(e.request_id)
    torch.cuda.synchronize()
    assert sorted(finished) == sorted(f"r{i}" for i in range(6))
    assert preemptions >= 1 and mixed >= 1
    assert bm.free_blocks == NB
    for rid in finished:
        with pytest.raises(RuntimeError):
            cache.seq_state(rid)


def test_bind_rejects_stale_and_foreign_handles():
    """Binding checks every handle against the shared manager and the cache's
    own sequences before changing anything."""
    import zealot_amd as ze
    from zealot_amd import KVCache, _lib
    bm = ze.BlockManager(8, 16)
    cache = KVCache(8, 16, 1, 2, 64, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=4)
    announce("bind checks")
    h1, h2 = bm.allocate(), bm.allocate()

    def bind(ids, blocks, tokens_before=None):
        import ctypes
        from zealot_amd.kv_cache import SeqBatch
        b = SeqBatch(ids)
        flat = [h for hs in blocks for h in hs]
        harr = (_lib.BlockHandleC * max(1, len(flat)))(*[h._c() for h in flat])
        nb = (ctypes.c_size_t * len(ids))(*[len(x) for x in blocks])
        tb = None if tokens_before is None else (ctypes.c_size_t * len(ids))(*tokens_before)
        _lib.check(_lib.lib().zk_cache_bind_blocks(cache._h, bm.handle, b.arr, len(ids), harr, nb, tb))

    bind(["s"], [[h1]])
    assert cache.seq_state("s").block_ids == [h1.block_id]
    bm.free(h2)
    with pytest.raises(RuntimeError, match="Stale handle"):
        bind(["s", "t"], [[h1], [h2]])
    with pytest.raises(RuntimeError):  # t was not registered by the failed call
        cache.seq_state("t")
    with pytest.raises(RuntimeError, match="holds 0 tokens"):
        bind(["s"], [[h1]], tokens_before=[5])
    cache.register_seq("own", 4)
    cache.alloc_block("own", bm)
    with pytest.raises(RuntimeError, match="owns its blocks"):
        bind(["own"], [[h1]])
    with pytest.raises(RuntimeError, match="caller"):
        cache.fork_seq("s", "s2")
    cache.release_seq("s")  # a bound sequence's handle stays the caller's
    assert bm.refcount(h1.block_id) == 1
    bm.free(h1)
    torch.cuda.synchronize()
