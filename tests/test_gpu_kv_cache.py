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


def _decode_vs_oracle(cache, layer, ids, lens, rng, H, D, BS):
    """One decode of every sequence at `layer` through the KVCache, within 1e-5
    of the fp32 oracle (src/attention/mod.rs:64-98) over the pages as they are."""
    q = normal(rng, (len(ids), H, D), oracle.F32)
    out = to_host(cache.paged_decode(layer, ids, to_dev(q)))
    kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
    bt = -np.ones((len(ids), 16), np.int32)
    for i, sid in enumerate(ids):
        b = cache.seq_state(sid).block_ids
        bt[i, :len(b)] = b
    ref = oracle.paged_decode(q, kp, vp, oracle.F32, bt, lens, H, D, BS, np.float32(1 / math.sqrt(D)))
    assert max_abs_err(out, ref) <= 1e-5, (layer, lens)


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
    ids = list(prompts)
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
        # the decode of every layer after each step (model_runner_cpu.rs:241-250
        # attends the last row over the context so far)
        for layer in range(L):
            _decode_vs_oracle(cache, layer, ids, [prompts[s] + step + 1 for s in ids], rng, H, D, BS)
    torch.cuda.synchronize()
    for layer in range(L):
        for sid, p in prompts.items():
            k, v = _ctx(cache, layer, sid, p + 8)
            assert np.array_equal(k, np.concatenate(written[sid][layer][0]))
            assert np.array_equal(v, np.concatenate(written[sid][layer][1]))
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


def _expected_bytes(tokens_k, tokens_v, src, H, D, BS, ks=None, vs=None):
    """Pool-format bytes [T, H, D] of a token sequence, written by the oracle
    into a contiguous scratch pool (fp8: quantised with scale row 0)."""
    T = tokens_k.shape[0]
    nb = (T + BS - 1) // BS
    fp8 = ks is not None
    dt = oracle.FP8 if fp8 else oracle.BF16
    pool_dtype = np.uint8 if fp8 else np.uint16
    kp = np.zeros((nb, H, BS, D), pool_dtype)
    vp = np.zeros((nb, H, BS, D), pool_dtype)
    rows = np.zeros(T, np.int32) if fp8 else None
    oracle.append_slots(kp, vp, dt, tokens_k, tokens_v, src, np.arange(T), H, D, BS, nb,
                        ks, vs, rows)
    bt = np.arange(nb, dtype=np.int32)
    return (oracle.gather(kp, dt, bt, T, H, D, BS, pool_dtype),
            oracle.gather(vp, dt, bt, T, H, D, BS, pool_dtype))


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_append_kv_batch_forks_layerwise_decode(kv):
    """Batched decode append over forked sequences: the first append copies each
    fork's shared tail (one batched copy), every layer's decode sees the token
    appended at that layer, and the pool bytes equal the oracle's."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(42 if kv == "bf16" else 43)
    L, H, Hkv, D, BS, NB = 2, 8, 2, 128, 16, 64
    fp8 = kv == "fp8"
    cdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    kvdt = oracle.FP8 if fp8 else oracle.BF16
    prefixes = {"pa": 16 * 3 + 5, "pb": 16 * 2 + 9}
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=cdt, max_seqs=16, max_blocks_per_seq=8)
    toks = {}  # seq -> layer -> (k list, v list) of bf16 bit arrays [1, Hkv, D]
    scales = {}
    for pid, p in prefixes.items():
        cache.register_seq(pid, 8)
        for _ in range((p + BS - 1) // BS):
            cache.alloc_block(pid, bm)
        kl = [normal(rng, (p, Hkv, D), oracle.BF16) for _ in range(L)]
        vl = [normal(rng, (p, Hkv, D), oracle.BF16) for _ in range(L)]
        if fp8:
            ks = np.stack([np.abs(as_f32(x, oracle.BF16)).max(axis=(0, 2)) / 448 for x in kl]).astype(np.float32)
            vs = np.stack([np.abs(as_f32(x, oracle.BF16)).max(axis=(0, 2)) / 448 for x in vl]).astype(np.float32)
            cache.set_fp8_scales(pid, ks.ravel(), vs.ravel())
            scales[pid] = (ks, vs)
        for layer in range(L):
            cache.store_kv(layer, pid, to_dev(kl[layer]), to_dev(vl[layer]), 0, p)
        toks[pid] = {l: ([kl[l]], [vl[l]]) for l in range(L)}
    children = []
    for pid in prefixes:
        for j in range(3):
            cid = f"{pid}.{j}"
            cache.fork_seq(pid, cid)
            children.append(cid)
            toks[cid] = {l: (list(toks[pid][l][0]), list(toks[pid][l][1])) for l in range(L)}
            scales[cid] = scales.get(pid)
    parent_of = {c: c.split(".")[0] for c in children}
    announce(f"kvcache append_kv_batch forks kv={kv}")
    n = len(children)
    scale = np.float32(1 / math.sqrt(D))
    for step in range(12):
        for cid in children:
            st = cache.seq_state(cid)
            if st.cached_tokens == len(st.block_ids) * BS:
                cache.alloc_block(cid, bm)
        for layer in range(L):
            k = normal(rng, (n, Hkv, D), oracle.BF16)
            v = normal(rng, (n, Hkv, D), oracle.BF16)
            cache.append_kv_batch(layer, children, to_dev(k), to_dev(v))
            for i, cid in enumerate(children):
                toks[cid][layer][0].append(k[i:i + 1])
                toks[cid][layer][1].append(v[i:i + 1])
            q = normal(rng, (n, H, D), oracle.BF16)
            out = to_host(cache.paged_decode(layer, children, to_dev(q)))
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            lens = [prefixes[parent_of[c]] + step + 1 for c in children]
            bt = -np.ones((n, 8), np.int32)
            for i, cid in enumerate(children):
                b = cache.seq_state(cid).block_ids
                bt[i, :len(b)] = b
            kw = {}
            if fp8:
                kw = dict(k_scales=np.stack([scales[c][0][layer] for c in children]),
                          v_scales=np.stack([scales[c][1][layer] for c in children]))
            ref = oracle.paged_decode(as_f32(q, oracle.BF16), kp, vp, kvdt, bt, lens, Hkv, D, BS,
                                      scale, **kw)
            assert max_abs_err(as_f32(out, oracle.BF16), ref) <= 2e-2, (step, layer)
        for cid in children:
            assert cache.seq_state(cid).cached_tokens == prefixes[parent_of[cid]] + step + 1
    torch.cuda.synchronize()
    # every fork copied its tail once; parents keep their blocks and bytes
    for pid, p in prefixes.items():
        pb = cache.seq_state(pid).block_ids
        full = p // BS
        for b in pb[:full]:
            assert bm.refcount(b) == 4
        assert bm.refcount(pb[full]) == 1
        for j in range(3):
            cb = cache.seq_state(f"{pid}.{j}").block_ids
            assert cb[:full] == pb[:full] and cb[full] != pb[full]
    for sid in list(prefixes) + children:
        T = cache.seq_state(sid).cached_tokens
        for layer in range(L):
            kk = np.concatenate(toks[sid][layer][0])
            vv = np.concatenate(toks[sid][layer][1])
            sc = (scales[sid][0][layer][None], scales[sid][1][layer][None]) if fp8 else (None, None)
            ek, ev = _expected_bytes(kk, vv, oracle.BF16, Hkv, D, BS, *sc)
            pdt = np.uint8 if fp8 else np.uint16
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            bt = np.asarray(cache.seq_state(sid).block_ids, np.int32)
            gk = oracle.gather(kp, kvdt, bt, T, Hkv, D, BS, pdt)
            gv = oracle.gather(vp, kvdt, bt, T, Hkv, D, BS, pdt)
            assert np.array_equal(gk, ek) and np.array_equal(gv, ev), (sid, layer)
    # batch errors: duplicate ids, unknown ids, and missing blocks fail before any write
    one = to_dev(normal(rng, (2, Hkv, D), oracle.BF16))
    with pytest.raises(RuntimeError, match="twice"):
        cache.append_kv_batch(0, [children[0], children[0]], one, one)
    with pytest.raises(RuntimeError, match="unknown seq nope"):
        cache.append_kv_batch(0, [children[0], "nope"], one, one)
    for sid in children + list(prefixes):
        cache.release_seq(sid)
    assert bm.free_blocks == NB


@pytest.mark.parametrize("G,D,qdt,mapping", [(4, 128, "bf16", "grouped"), (1, 128, "bf16", "grouped"),
                                             (2, 64, "bf16", "grouped"), (8, 128, "bf16", "grouped"),
                                             (4, 64, "f32", "grouped"), (4, 128, "bf16", "modulo")])
def test_forked_prefix_decode_shares_pages(G, D, qdt, mapping):
    """Forks of one prefix are decoded in subgroups that read the shared pages
    once for up to 32 query rows (QK and PV on MFMA), then merged with each
    fork's own pages; the result matches the oracle over every sequence's
    full table, and the expected subgroups were formed."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(1000 + 10 * G + D)
    Hkv, BS, NB, MB = 2, 16, 512, 32
    H = G * Hkv
    prefixes = {"pa": 16 * 17 + 3, "pb": 16 * 20, "solo": 16 * 18 + 1}
    nforks = {"pa": 9, "pb": 3, "solo": 0}
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, 1, Hkv, D, dtype=torch.bfloat16, max_seqs=32, max_blocks_per_seq=MB)
    for pid, p in prefixes.items():
        cache.register_seq(pid, MB)
        for _ in range((p + BS - 1) // BS):
            cache.alloc_block(pid, bm)
        cache.store_kv(0, pid, to_dev(normal(rng, (p, Hkv, D), oracle.BF16)),
                       to_dev(normal(rng, (p, Hkv, D), oracle.BF16)), 0, p)
    ids = list(prefixes)
    for pid, nf in nforks.items():
        for j in range(nf):
            cid = f"{pid}.{j}"
            cache.fork_seq(pid, cid)
            ids.append(cid)
            for _ in range(1 + j % 4):  # fork-private tokens (copy-on-write of a partial tail)
                st = cache.seq_state(cid)
                if st.cached_tokens == len(st.block_ids) * BS:
                    cache.alloc_block(cid, bm)
                cache.append_kv(0, cid, to_dev(normal(rng, (1, Hkv, D), oracle.BF16)[0]),
                                to_dev(normal(rng, (1, Hkv, D), oracle.BF16)[0]))
    ids = [ids[i] for i in rng.permutation(len(ids))]
    n = len(ids)
    q = normal(rng, (n, H, D), oracle.BF16 if qdt == "bf16" else oracle.F32)
    announce(f"shared-prefix decode G={G} D={D} q={qdt} mapping={mapping}")
    out = to_host(cache.paged_decode(0, ids, to_dev(q), mapping=mapping))
    cap = 32 // G

    def chunks(m):
        return m // cap + (1 if m % cap >= 2 else 0)
    sg, pages = cache.decode_sharing()
    assert sg == chunks(1 + nforks["pa"]) + chunks(1 + nforks["pb"])
    kp, vp = to_host(cache.k_pool(0)), to_host(cache.v_pool(0))
    bt = -np.ones((n, MB), np.int32)
    lens = []
    for i, sid in enumerate(ids):
        st = cache.seq_state(sid)
        bt[i, :len(st.block_ids)] = st.block_ids
        lens.append(st.cached_tokens)
    qf = as_f32(q, oracle.BF16) if qdt == "bf16" else q
    ref = oracle.paged_decode(qf, kp, vp, oracle.BF16, bt, lens, Hkv, D, BS, np.float32(1 / math.sqrt(D)),
                              mapping=oracle.GROUPED if mapping == "grouped" else oracle.MODULO)
    got = as_f32(out, oracle.BF16) if qdt == "bf16" else out
    assert max_abs_err(got, ref) <= 2e-2
    for sid in ids:
        cache.release_seq(sid)
    assert bm.free_blocks == NB


@pytest.mark.parametrize("seed", range(8))
def test_random_fork_trees_decode_append_against_oracle(seed):
    """Seeded random prefix trees through the KVCache: prefixes of random
    length (some too short to share), forks of them and forks of forks
    (taken after the parent wrote a few tokens of its own), decoded in a
    random order by decode_append (the new token stored and attended in one
    launch) over two layers for three steps, with blocks allocated as
    sequences cross block edges and first writes into shared tails copied.
    Every layer of every step against the fp32 oracle over each sequence's
    pages as they are (src/kv_cache.rs:281-356, src/attention/mod.rs:64-98)."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(3000 + seed)
    G = (1, 2, 4, 8)[seed % 4]
    D = (128, 64)[seed // 4]
    Hkv = int(rng.choice([1, 2]))
    H, L, BS, MB, NB = G * Hkv, 2, 16, 64, 2048
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=128, max_blocks_per_seq=MB)

    def grow(sid, n):  # n more tokens at every layer, allocating as needed
        st = cache.seq_state(sid)
        start = st.cached_tokens
        while len(cache.seq_state(sid).block_ids) * BS < start + n:
            cache.alloc_block(sid, bm)
        for layer in range(L):
            k = normal(rng, (n, Hkv, D), oracle.BF16)
            v = normal(rng, (n, Hkv, D), oracle.BF16)
            cache.store_kv(layer, sid, to_dev(k), to_dev(v), start, n)

    ids = []
    can_share = False  # some prefix has 16 full pages and a fork: a subgroup must form
    for pi in range(int(rng.integers(1, 5))):
        pid = f"p{pi}"
        cache.register_seq(pid, MB)
        plen = int(rng.integers(1, 700)) if pi else int(rng.integers(16 * BS, 700))  # the first can share
        grow(pid, plen)
        ids.append(pid)
        nf = int(rng.integers(0, 13)) if pi else int(rng.integers(1, 13))
        can_share |= plen >= 16 * BS and nf > 0
        for fi in range(nf):
            cid = f"{pid}.{fi}"
            cache.fork_seq(pid, cid)
            ids.append(cid)
            if rng.random() < 0.6:
                grow(cid, int(rng.integers(1, 40)))
            if rng.random() < 0.3:  # a fork of the fork, after its own tokens
                gid = f"{cid}.g"
                cache.fork_seq(cid, gid)
                ids.append(gid)
    order = [ids[i] for i in rng.permutation(len(ids))]
    n = len(order)
    announce(f"random fork tree {seed}: G={G} Hkv={Hkv} D={D} seqs={n}")
    scale = np.float32(1 / math.sqrt(D))
    for step in range(3):
        for sid in order:
            st = cache.seq_state(sid)
            if st.cached_tokens == len(st.block_ids) * BS:
                cache.alloc_block(sid, bm)
        lens = [cache.seq_state(sid).cached_tokens + 1 for sid in order]
        for layer in range(L):
            k = normal(rng, (n, Hkv, D), oracle.BF16)
            v = normal(rng, (n, Hkv, D), oracle.BF16)
            q = normal(rng, (n, H, D), oracle.BF16)
            out = to_host(cache.decode_append(layer, order, to_dev(k), to_dev(v), to_dev(q)))
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            bt = -np.ones((n, MB), np.int32)
            for i, sid in enumerate(order):
                b = cache.seq_state(sid).block_ids
                bt[i, :len(b)] = b
                pos = lens[i] - 1  # the appended row sits where its sequence's table says
                blk, off = b[pos // BS], pos % BS
                assert np.array_equal(kp[blk, :, off], k[i]) and np.array_equal(vp[blk, :, off], v[i]), (sid, layer)
            ref = oracle.paged_decode(as_f32(q, oracle.BF16), kp, vp, oracle.BF16, bt, lens, Hkv, D, BS, scale)
            assert max_abs_err(as_f32(out, oracle.BF16), ref) <= 2e-2, (step, layer)
            sg, _ = cache.decode_sharing()
            assert (sg > 0) == can_share, (sg, can_share)
    for sid in order:
        cache.release_seq(sid)
    assert bm.free_blocks == NB


def test_decode_plan_reuse_across_layers_and_batches():
    """The cache plans a decode once and reuses the plan while the shapes,
    lengths, prefix groups and tables stay the same (the layers of a step);
    the work items carry the block ids of their first pages, so another batch
    with the same lengths but other tables, or a length that changes in one
    layer, makes a new plan.  Every call is checked against the oracle."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng(77)
    L, H, Hkv, D, BS, NB = 3, 8, 2, 128, 16, 160
    lens = {"a": 300, "b": 40, "c": 300, "d": 40}
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=8, max_blocks_per_seq=24)
    for sid, T in lens.items():
        cache.register_seq(sid, 24)
        for _ in range((T + 1 + BS - 1) // BS):
            cache.alloc_block(sid, bm)
        for layer in range(L):
            cache.store_kv(layer, sid, to_dev(normal(rng, (T, Hkv, D), oracle.BF16)),
                           to_dev(normal(rng, (T, Hkv, D), oracle.BF16)), 0, T)
    scale = np.float32(1 / math.sqrt(D))

    def check(layer, ids, seq_lens):
        q = normal(rng, (len(ids), H, D), oracle.BF16)
        out = to_host(cache.paged_decode(layer, ids, to_dev(q)))
        kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
        bt = -np.ones((len(ids), 24), np.int32)
        for i, sid in enumerate(ids):
            b = cache.seq_state(sid).block_ids
            bt[i, :len(b)] = b
        exp = oracle.paged_decode(as_f32(q, oracle.BF16), kp, vp, oracle.BF16, bt, seq_lens, Hkv, D, BS, scale)
        assert max_abs_err(as_f32(out, oracle.BF16), exp) <= 2e-2, (layer, ids)

    announce("decode plan reuse")
    check(0, ["a", "b"], [300, 40])
    check(1, ["a", "b"], [300, 40])  # the next layer: same plan
    check(1, ["c", "d"], [300, 40])  # other sequences, same lengths: other tables, a new plan
    # one more token in layer 2 only: a new plan there, and again for layer 0
    cache.store_kv(2, "a", to_dev(normal(rng, (1, Hkv, D), oracle.BF16)),
                   to_dev(normal(rng, (1, Hkv, D), oracle.BF16)), 300, 1)
    check(2, ["a", "b"], [301, 40])
    check(0, ["a", "b"], [300, 40])
    check(2, ["b", "a"], [40, 301])  # order matters: sequence indices change
    torch.cuda.synchronize()


def test_cow_out_of_blocks_keeps_typed_error():
    """A BlockManager rejection raised inside a KVCache call (the copy-on-write
    allocation) reaches the caller with its code and fields unchanged
    (OutOfBlocks{requested: 1, available: 0}, src/error.rs:11-12), and nothing
    is written."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    L, H, D, BS, NB = 2, 8, 128, 16, 3
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, H, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=4)
    cache.register_seq("p", 4)
    for _ in range(3):
        cache.alloc_block("p", bm)        # the pool is now empty
    x = torch.ones((20, H, D), dtype=torch.bfloat16, device="cuda")
    for layer in range(L):
        cache.store_kv(layer, "p", x, x, 0, 20)
    cache.fork_seq("p", "c")
    one = torch.zeros((1, H, D), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ze.ZealotError) as e:
        cache.append_kv(0, "c", one[0], one[0])  # needs a fresh block for the copy
    assert e.value.code == ze._lib.ERR_OUT_OF_BLOCKS
    assert e.value.fields == {"requested": 1, "available": 0}
    assert str(e.value) == "Out of blocks: requested 1, available 0"
    assert cache.seq_state("c").cached_tokens == 20
    cache.release_seq("c")
    cache.release_seq("p")
    assert bm.free_blocks == NB


@pytest.mark.parametrize("dtype,H,Hkv,D", [("bf16", 32, 8, 128), ("bf16", 8, 8, 64), ("f32", 4, 4, 32),
                                           ("fp8", 32, 8, 128)])
def test_decode_append_is_append_then_decode(dtype, H, Hkv, D):
    """zk_cache_decode_append (one launch on bf16 MFMA shapes: the decode
    stores each sequence's new K / V row and attends it) against
    append_kv_batch + paged_decode on a twin cache with the same history:
    outputs and every pool byte equal after each of 40 steps over 2 layers,
    with forks whose first write copies a shared tail block and sequences
    crossing block boundaries (src/kv_cache.rs:281-356,
    src/attention/mod.rs:64-98); the f32 and fp8 caches take the two-call
    path (bf16 rows quantised by the append)."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    from zealot_amd.kv_cache import SeqBatch
    cdt = {"bf16": torch.bfloat16, "f32": torch.float32, "fp8": torch.float8_e4m3fn}[dtype]
    odt = oracle.F32 if dtype == "f32" else oracle.BF16
    L, BS, NB, STEPS = 2, 16, 600, 40
    rng = np.random.default_rng(46 + D)
    base = {f"s{i}": int(rng.integers(1, 700)) for i in range(12)}
    base["par"] = 16 * 20 + 5  # forked: its children's first append copies the partial tail
    kids = [f"k{i}" for i in range(6)]
    caches = []
    init = {s: [normal(rng, (t, Hkv, D), odt) for _ in range(2 * L)] for s, t in base.items()}
    for _ in range(2):
        bm = ze.BlockManager(NB, BS)
        cache = KVCache(NB, BS, L, Hkv, D, dtype=cdt, max_seqs=32, max_blocks_per_seq=64)
        for sid, t in base.items():
            cache.register_seq(sid, 64)
            for _ in range((t + STEPS + BS - 1) // BS):
                cache.alloc_block(sid, bm)
            if dtype == "fp8":  # N(0,1) rows: |x| < 448 * 0.05 at these sizes
                cache.set_fp8_scales(sid, np.full(L * Hkv, 0.05, np.float32), np.full(L * Hkv, 0.05, np.float32))
            for layer in range(L):
                cache.store_kv(layer, sid, to_dev(init[sid][2 * layer]), to_dev(init[sid][2 * layer + 1]), 0, t)
        for k in kids:
            cache.fork_seq("par", k)
        caches.append((cache, bm))
    ids = [s for s in base if s != "par"] + kids
    batch = SeqBatch(ids)
    pos = {s: base[s] for s in base}
    for k in kids:
        pos[k] = base["par"]
    announce(f"decode_append {dtype} H{H}/Hkv{Hkv}/D{D}: {len(ids)} seqs x {STEPS} steps")
    for step in range(STEPS):  # the forks share the parent's later blocks too: each is copied on first write
        for layer in range(L):
            k = to_dev(normal(rng, (len(ids), Hkv, D), odt))
            v = to_dev(normal(rng, (len(ids), Hkv, D), odt))
            q = to_dev(normal(rng, (len(ids), H, D), odt))
            (ca, _), (cb, _) = caches
            got = ca.decode_append(layer, batch, k, v, q)
            cb.append_kv_batch(layer, batch, k, v)
            want = cb.paged_decode(layer, batch, q)
            torch.cuda.synchronize()
            assert np.array_equal(to_host(got), to_host(want)), (step, layer)
            for pa, pb in ((ca.k_pool(layer), cb.k_pool(layer)), (ca.v_pool(layer), cb.v_pool(layer))):
                assert np.array_equal(to_host(pa), to_host(pb)), (step, layer)
        for sid in ids:
            pos[sid] += 1
            assert ca.seq_state(sid).cached_tokens == cb.seq_state(sid).cached_tokens == pos[sid]
    (ca, _), _ = caches
    par = ca.seq_state("par").block_ids
    for k in kids:  # the forks copied the partial tail, the full blocks before it stay shared
        ids_k = ca.seq_state(k).block_ids
        assert ids_k[:20] == par[:20] and ids_k[20] != par[20]
    if dtype == "fp8":  # fp8 decode parity with the oracle: tests/test_gpu_decode.py, test_gpu_full_size.py
        return
    # and the last step against the oracle on the pages as they are
    last = L - 1
    kp, vp = to_host(ca.k_pool(last)), to_host(ca.v_pool(last))
    bt = -np.ones((len(ids), 64), np.int32)
    for i, sid in enumerate(ids):
        b = ca.seq_state(sid).block_ids
        bt[i, :len(b)] = b
    ref = oracle.paged_decode(as_f32(to_host(q), odt), kp, vp, odt, bt, [pos[s] for s in ids], Hkv, D, BS,
                              np.float32(1 / math.sqrt(D)), threads=8)
    assert max_abs_err(as_f32(to_host(got), odt), ref) <= (2e-2 if dtype == "bf16" else 1e-5)


def test_device_table_rows_follow_queued_allocations():
    """`alloc_block` queues its table write; the device rows
    (`block_table_ptr`, kv_cache.rs:188-190) still read as the handles say:
    after the pointer call, after a batched write that flushes the queue, in a
    fork's copied row, and in a row reset by release / register."""
    import ctypes
    import zealot_amd as ze
    from zealot_amd import KVCache, _lib
    L, H, D, BS, NB, MB = 2, 2, 32, 16, 64, 8
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, H, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=MB)
    lib = _lib.lib()

    def row(ptr):  # the device row as it is, without the pointer call's flush
        dst = torch.empty(MB, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        _lib.check(lib.zk_stream_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(ptr), MB * 4, None))
        torch.cuda.synchronize()
        return dst.cpu().tolist()

    def want(sid):
        b = cache.seq_state(sid).block_ids
        return b + [-1] * (MB - len(b))

    announce("device table rows after queued allocations")
    cache.register_seq("a", MB)
    cache.register_seq("b", MB)
    for sid in ("a", "b", "a", "a", "b"):
        cache.alloc_block(sid, bm)
    assert row(cache.block_table_ptr("a")) == want("a")
    assert row(cache.block_table_ptr("b")) == want("b")
    pa = cache.block_table_ptr("a")
    cache.alloc_block("a", bm)                      # queued
    x = torch.ones((3, H, D), dtype=torch.bfloat16, device="cuda")
    cache.store_kv(0, "a", x, x, 0, 3)              # a batched write flushes the queue
    assert row(pa) == want("a") and want("a")[3] >= 0
    cache.alloc_block("a", bm)                      # queued, then copied by the fork
    cache.fork_seq("a", "c")
    assert row(cache.block_table_ptr("c")) == want("a") == want("c")
    pb = cache.block_table_ptr("b")
    cache.alloc_block("b", bm)                      # queued, then the row is reset
    cache.release_seq("b")
    cache.register_seq("d", MB)
    assert row(cache.block_table_ptr("d")) == [-1] * MB
    assert row(pb) == [-1] * MB or cache.block_table_ptr("d") != pb
    for sid in ("a", "c", "d"):
        cache.release_seq(sid)
    assert bm.free_blocks == NB


def test_device_rows_take_the_last_queued_write():
    """An entry queued twice before a flush (allocations, then a swap-out that
    clears the row) ends with the later value on the device, every time: the
    one-launch table update applies only the last write to each entry."""
    import ctypes
    import zealot_amd as ze
    from zealot_amd import KVCache, _lib
    L, H, D, BS, NB, MB = 2, 2, 32, 16, 256, 64
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, H, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=MB)
    cache.enable_swap(MB)
    lib = _lib.lib()

    def row(ptr):
        dst = torch.empty(MB, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        _lib.check(lib.zk_stream_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(ptr), MB * 4, None))
        torch.cuda.synchronize()
        return dst.cpu().tolist()

    announce("device rows: allocation then swap-out queued together")
    cache.register_seq("s", MB)
    for rep, (nw, extra) in enumerate(((4, 60), (1, 16), (2, 1), (3, 37))):
        ptr = cache.block_table_ptr("s")
        for _ in range(nw):
            cache.alloc_block("s", bm)
        x = torch.ones((nw * BS, H, D), dtype=torch.bfloat16, device="cuda")
        cache.store_kv(0, "s", x, x, 0, nw * BS)   # written blocks (the write flushes the queue)
        for _ in range(extra):
            cache.alloc_block("s", bm)          # queued, not flushed
        cache.swap_out(["s"])                   # queues -1 over every entry, the queued ones too
        assert cache.is_swapped("s")
        assert row(ptr) == [-1] * MB, rep
        cache.swap_in(["s"], bm)                # fresh blocks for the written ones: the row follows them
        want = cache.seq_state("s").block_ids
        assert len(want) == nw and row(ptr) == want + [-1] * (MB - nw), rep
        cache.release_seq("s")
        cache.register_seq("s", MB)
        assert row(cache.block_table_ptr("s")) == [-1] * MB, rep
    cache.release_seq("s")
    assert bm.free_blocks == NB
