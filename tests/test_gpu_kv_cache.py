"""KVCache (src/kv_cache.rs) end to end on the MI355X: register / alloc_block /
store_kv / append_kv / paged_decode through the C ABI, the C1 plumbing case,
and prefix sharing with copy-on-write (BlockManager reference/free semantics,
stale handles rejected)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, normal, to_dev, to_host

pytestmark = pytest.mark.gpu


def _ctx(cache, layer, sid, L):
    """Token-major K, V of a sequence, read back through the pool views."""
    st = cache.seq_state(sid)
    kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
    bt = np.asarray(st.block_ids, np.int32)
    H, D, BS = cache.num_kv_heads, cache.head_dim, cache.block_size
    dt = oracle.F32 if kp.dtype == np.float32 else oracle.BF16
    k = oracle.gather(kp, dt, bt, L, H, D, BS, kp.dtype)
    v = oracle.gather(vp, dt, bt, L, H, D, BS, vp.dtype)
    return k, v


def test_c1_plumbing_through_kvcache():
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(40)
    L, H, D, BS, NB = 2, 4, 32, 16, 256
    prompts = {"s0": 17, "s1": 40, "s2": 77, "s3": 130}
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, H, D, dtype=torch.float32, max_seqs=8, max_blocks_per_seq=16)
    written = {sid: {l: ([], []) for l in range(L)} for sid in prompts}
    announce("kvcache C1 plumbing")
    for sid, p in prompts.items():
        cache.register_seq(sid, 16)
        for _ in range((p + 8 + BS - 1) // BS):
            cache.alloc_block(sid, bm)
        for layer in range(L):
            k = normal(rng, (p, H, D), oracle.F32)
            v = normal(rng, (p, H, D), oracle.F32)
            cache.store_kv(layer, sid, to_dev(k), to_dev(v), 0, p)
            written[sid][layer][0].append(k)
            written[sid][layer][1].append(v)
        assert cache.seq_state(sid).cached_tokens == p
    for step in range(8):
        for sid, p in prompts.items():
            for layer in range(L):
                k = normal(rng, (1, H, D), oracle.F32)
                v = normal(rng, (1, H, D), oracle.F32)
                cache.append_kv(layer, sid, to_dev(k[0]), to_dev(v[0]))
                written[sid][layer][0].append(k)
                written[sid][layer][1].append(v)
            st = cache.seq_state(sid)
            assert st.cached_tokens == p + step + 1 and st.block_offset == (p + step + 1) % BS
    torch.cuda.synchronize()
    ids = list(prompts)
    for layer in range(L):
        for sid, p in prompts.items():
            k, v = _ctx(cache, layer, sid, p + 8)
            assert np.array_equal(k, np.concatenate(written[sid][layer][0]))
            assert np.array_equal(v, np.concatenate(written[sid][layer][1]))
        q = normal(rng, (4, H, D), oracle.F32)
        out = to_host(cache.paged_decode(layer, ids, to_dev(q)))
        kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
        bt = -np.ones((4, 16), np.int32)
        for i, sid in enumerate(ids):
            b = cache.seq_state(sid).block_ids
            bt[i, :len(b)] = b
        ref = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [prompts[s] + 8 for s in ids], H, D, BS,
                                  np.float32(1 / math.sqrt(D)))
        assert max_abs_err(out, ref) <= 1e-5
    # errors follow kv_cache.rs
    with pytest.raises(RuntimeError, match="unknown seq nope"):
        cache.seq_state("nope")
    one = to_dev(normal(rng, (1, H, D), oracle.F32))
    with pytest.raises(RuntimeError, match=r"block_idx 9 OOB \(have 9 blocks\)"):
        cache.store_kv(0, "s3", one, one, 9 * 16, 1)
    for sid in ids:
        cache.release_seq(sid)
    assert bm.free_blocks == NB


def test_prefix_fork_copy_on_write():
    """C4 in miniature: forks share prefix pages; the first write into the shared,
    partially filled tail block copies it (all layers, K and V) into a fresh block."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(41)
    L, H, D, BS, NB = 3, 8, 128, 16, 128
    prefix = 16 * 5 + 7  # partially filled tail block
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, H, D, dtype=torch.bfloat16, max_seqs=8, max_blocks_per_seq=16)
    cache.register_seq("p", 16)
    for _ in range(6):
        cache.alloc_block("p", bm)
    pref = {}
    for layer in range(L):
        k = normal(rng, (prefix, H, D), oracle.BF16)
        v = normal(rng, (prefix, H, D), oracle.BF16)
        cache.store_kv(layer, "p", to_dev(k), to_dev(v), 0, prefix)
        pref[layer] = (k, v)
    announce("kvcache fork/CoW")
    for c in ("c0", "c1", "c2"):
        cache.fork_seq("p", c)
    parent_ids = cache.seq_state("p").block_ids
    for b in parent_ids:
        assert bm.refcount(b) == 4
    # child c0 appends one token -> CoW of the tail block only
    new = {}
    for layer in range(L):
        k = normal(rng, (1, H, D), oracle.BF16)
        v = normal(rng, (1, H, D), oracle.BF16)
        cache.append_kv(layer, "c0", to_dev(k[0]), to_dev(v[0]))
        new[layer] = (k, v)
    torch.cuda.synchronize()
    c0 = cache.seq_state("c0").block_ids
    assert c0[:5] == parent_ids[:5] and c0[5] != parent_ids[5]
    assert bm.refcount(parent_ids[5]) == 3 and bm.refcount(c0[5]) == 1
    for layer in range(L):
        pk, pv = _ctx(cache, layer, "p", prefix)
        assert np.array_equal(pk, pref[layer][0]) and np.array_equal(pv, pref[layer][1])
        ck, cv = _ctx(cache, layer, "c0", prefix + 1)
        assert np.array_equal(ck[:prefix], pref[layer][0]) and np.array_equal(ck[prefix:], new[layer][0])
        assert np.array_equal(cv[:prefix], pref[layer][1]) and np.array_equal(cv[prefix:], new[layer][1])
        # the untouched forks still read the parent's tail
        k1, _ = _ctx(cache, layer, "c1", prefix)
        assert np.array_equal(k1, pref[layer][0])
    # releasing everything returns every block; old handles are stale afterwards
    h_old = ze.BlockHandle(parent_ids[0], 1)
    for s in ("c0", "c1", "c2", "p"):
        cache.release_seq(s)
    assert bm.free_blocks == NB
    with pytest.raises(RuntimeError, match="Stale handle"):
        bm.reference(h_old)
