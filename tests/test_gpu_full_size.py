"""C4 and C5 at their full BASELINE sizes on the MI355X, checked against the
CPU oracle on sampled sequences.

C5: 512 sequences, context U[1024, 16384], Llama-3-8B heads, K/V drawn in
bf16, quantised to fp8-e4m3 on append with per-(sequence, kv-head) amax
scales; the batched decode of all 512 is checked on 8 sampled sequences
against the fp32 oracle on the unquantised bf16 inputs (5e-2) and against the
oracle on the dequantised fp8 pages (2e-2), their pages bit-exact with the
oracle's quantiser, and on all 512 against a plain PyTorch fp32 decode of
the dequantised pages (2e-2; that decode matches the oracle on the sampled
ones to 1e-4).

C4: 16 prefixes of 2048 + r tokens (r in [1, 15]: the tail block is partial)
over 32 bf16 layers, 8 forks each, through the stateful KVCache, for all 64
decode steps of append + paged attention (even steps through the fused
decode_append launch, odd ones through append_kv_batch + paged_decode):
fork refcounts, the copy-on-write
of all 128 tails in all 64 pools (bit-exact), the 16 prefix subgroups of the
shared decode, every block a fork gains on the way (a fresh private block
with one reference whenever its position crosses a block boundary, about
four per fork), sampled (fork, layer, step) decodes spread over the 64 steps
against the oracle (2e-2) with their pages bit-exact, the decode of all 128
forks at the first and last layer on steps 0, 15, 31, 47 and 63 against a
plain PyTorch fp32 decode of their pages (2e-2), and every block back in the
BlockManager at the end with old handles stale (src/block_manager.rs:108-164,
src/kv_cache.rs:281-356)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, paged_tables, to_dev, to_host, torch_decode_ref

pytestmark = pytest.mark.gpu


def _bf16_bits(t):
    return to_host(t)


def test_c5_fp8_full_size_sampled_against_oracle():
    from zealot_amd import ops
    N, H, Hkv, D, BS = 512, 32, 8, 128, 16
    rng = np.random.default_rng(55)
    lens = rng.integers(1024, 16385, N)
    bt, nb = paged_tables(rng, lens, BS)
    pick = set(int(x) for x in rng.choice(N, 8, replace=False))
    announce(f"C5 full size: N={N} sum_ctx={int(lens.sum())} blocks={nb} sampled={sorted(pick)}")
    g = torch.Generator(device="cuda").manual_seed(55)
    kp = torch.zeros((nb, Hkv, BS, D), dtype=torch.uint8, device="cuda")
    vp = torch.zeros_like(kp)
    ks = torch.empty((N, Hkv), dtype=torch.float32, device="cuda")
    vs = torch.empty_like(ks)
    src = {}  # sampled sequence -> (k bf16 bits, v bf16 bits) of its context
    for n0 in range(0, N, 32):
        n1 = min(N, n0 + 32)
        L = lens[n0:n1]
        T = int(L.sum())
        k = torch.randn((T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        cu = np.concatenate([[0], np.cumsum(L)]).astype(np.int64)
        ks[n0:n1] = ops.fp8_scales(k, to_dev(cu))
        vs[n0:n1] = ops.fp8_scales(v, to_dev(cu))
        slots = np.concatenate([bt[n, np.arange(l) // BS].astype(np.int64) * BS + np.arange(l) % BS
                                for n, l in zip(range(n0, n1), L)])
        rows = np.repeat(np.arange(n0, n1), L).astype(np.int32)
        ops.append(kp, vp, k, v, to_dev(slots), k_scales=ks, v_scales=vs, token_row=to_dev(rows))
        for n in range(n0, n1):
            if n in pick:
                a, b = int(cu[n - n0]), int(cu[n - n0 + 1])
                src[n] = (_bf16_bits(k[a:b]), _bf16_bits(v[a:b]))
        del k, v
    q = torch.randn((N, H, D), generator=g, device="cuda").to(torch.bfloat16)
    out = ops.paged_decode(q, kp, vp, to_dev(bt), to_dev(lens.astype(np.int32)), k_scales=ks, v_scales=vs)
    torch.cuda.synchronize()
    got = as_f32(to_host(out), oracle.BF16)
    assert np.all(np.isfinite(got))
    # all 512 against a plain PyTorch fp32 decode of the dequantised pages
    tref = torch_decode_ref(q, kp, vp, bt, lens, BS, k_scales=ks, v_scales=vs, fp8=True).cpu().numpy()
    assert max_abs_err(got, tref) <= 2e-2
    qh = to_host(q)
    ks_h, vs_h = to_host(ks), to_host(vs)
    scale = np.float32(1 / math.sqrt(D))
    for n in sorted(pick):
        Ln = int(lens[n])
        k_src, v_src = src[n]
        # scales and quantised pages of this sequence, bit-exact with the oracle
        cu1 = np.array([0, Ln], np.int64)
        ks_ref = oracle.fp8_scales(k_src, oracle.BF16, cu1, Hkv, D)
        vs_ref = oracle.fp8_scales(v_src, oracle.BF16, cu1, Hkv, D)
        assert np.array_equal(ks_ref[0], ks_h[n]) and np.array_equal(vs_ref[0], vs_h[n]), n
        npg = (Ln + BS - 1) // BS
        idx = torch.from_numpy(bt[n, :npg].astype(np.int64)).cuda()
        kpg, vpg = to_host(kp.index_select(0, idx)), to_host(vp.index_select(0, idx))
        k8 = np.zeros((npg, Hkv, BS, D), np.uint8)
        v8 = np.zeros_like(k8)
        oracle.append_slots(k8, v8, oracle.FP8, k_src, v_src, oracle.BF16, np.arange(Ln, dtype=np.int64), Hkv, D,
                            BS, npg, ks_ref, vs_ref, np.zeros(Ln, np.int32))
        assert np.array_equal(kpg, k8) and np.array_equal(vpg, v8), n
        bt1 = np.arange(npg, dtype=np.int32)[None, :]
        q1 = as_f32(qh[n:n + 1], oracle.BF16)
        # the bar: the fp32 oracle on the unquantised bf16 inputs
        kf = np.zeros((npg, Hkv, BS, D), np.float32)
        vf = np.zeros_like(kf)
        oracle.append_slots(kf, vf, oracle.F32, as_f32(k_src, oracle.BF16), as_f32(v_src, oracle.BF16),
                            oracle.F32, np.arange(Ln, dtype=np.int64), Hkv, D, BS, npg)
        ref = oracle.paged_decode(q1, kf, vf, oracle.F32, bt1, [Ln], Hkv, D, BS, scale, threads=8)
        assert max_abs_err(got[n:n + 1], ref) <= 5e-2, n
        # and tightly against the dequantised fp8 pages
        ref8 = oracle.paged_decode(q1, k8, v8, oracle.FP8, bt1, [Ln], Hkv, D, BS, scale, oracle.GROUPED,
                                   ks_ref, vs_ref, threads=8)
        assert max_abs_err(got[n:n + 1], ref8) <= 2e-2, n
        assert max_abs_err(tref[n:n + 1], ref8) <= 1e-4, n  # the torch decode is the oracle's


def test_c4_prefix_cow_full_size():
    import zealot_amd as ze
    from zealot_amd import KVCache
    from zealot_amd.kv_cache import SeqBatch
    P, F, L, H, Hkv, D, BS = 16, 8, 32, 32, 8, 128, 16
    STEPS = 64
    WHOLE = (0, 15, 31, 47, 63)  # steps whose whole batch is checked at the first and last layer
    rng = np.random.default_rng(44)
    plen = 2048 + rng.integers(1, BS, P)
    MB = (int(plen.max()) + STEPS + BS - 1) // BS + 1
    grown = (STEPS + BS - 1) // BS + 1  # blocks a fork may gain: its tail copy and the steps' new blocks
    NB = sum((int(x) + BS - 1) // BS for x in plen) + P * F * grown + 64
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=P * (F + 1), max_blocks_per_seq=MB)
    announce(f"C4 full size: {P} prefixes x {int(plen.min())}..{int(plen.max())} tokens, {L} layers, "
             f"{P * F} forks, {NB} blocks")
    g = torch.Generator(device="cuda").manual_seed(44)
    pk = [[None] * L for _ in range(P)]
    pv = [[None] * L for _ in range(P)]
    for p in range(P):
        cache.register_seq(f"p{p}", MB)
        for _ in range((int(plen[p]) + BS - 1) // BS):
            cache.alloc_block(f"p{p}", bm)
        for layer in range(L):
            pk[p][layer] = torch.randn((int(plen[p]), Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
            pv[p][layer] = torch.randn((int(plen[p]), Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
            cache.store_kv(layer, f"p{p}", pk[p][layer], pv[p][layer], 0, int(plen[p]))
    children = [f"p{p}.f{j}" for p in range(P) for j in range(F)]
    parent = [p for p in range(P) for _ in range(F)]
    for cid, p in zip(children, parent):
        cache.fork_seq(f"p{p}", cid)
    pblocks = [cache.seq_state(f"p{p}").block_ids for p in range(P)]
    for p in range(P):
        assert all(bm.refcount(b) == 1 + F for b in pblocks[p])  # parent + 8 forks (try_reference)
    batch = SeqBatch(children)
    n = len(children)
    kin = [[torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16) for _ in range(L)]
           for _ in range(STEPS)]
    vin = [[torch.randn((n, Hkv, D), generator=g, device="cuda").to(torch.bfloat16) for _ in range(L)]
           for _ in range(STEPS)]
    qin = [[torch.randn((n, H, D), generator=g, device="cuda").to(torch.bfloat16) for _ in range(L)]
           for _ in range(STEPS)]
    # sampled decodes spread over the steps, late ones included (step >= 40:
    # every fork has crossed at least two block boundaries by then)
    sample = [(int(rng.integers(0, n)), layer, step) for step, layer in
              ((0, 0), (0, 31), (3, 7), (12, 20), (17, 0), (29, 31), (40, 5), (46, 31), (55, 0), (63, 17),
               (63, 31))]
    outs, whole = {}, {}
    out = torch.empty((n, H, D), dtype=torch.bfloat16, device="cuda")
    pos = [int(plen[p]) for p in parent]
    private = [set() for _ in children]  # blocks each fork gained by alloc_block
    for step in range(STEPS):
        for i, cid in enumerate(children):  # a block for the token if the tail is full
            if pos[i] % BS == 0:
                before = cache.seq_state(cid).block_ids
                cache.alloc_block(cid, bm)
                ids = cache.seq_state(cid).block_ids
                # kv_cache.rs:107-130 / block_manager.rs:108-122: one fresh block
                # at the table's end, one reference, the earlier entries unchanged
                assert ids[:-1] == before and len(ids) == pos[i] // BS + 1, (cid, step)
                assert bm.refcount(ids[-1]) == 1 and ids[-1] not in private[i], (cid, step)
                private[i].add(ids[-1])
        for layer in range(L):
            if step % 2 == 0:  # even steps: the fused append + decode launch
                cache.decode_append(layer, batch, kin[step][layer], vin[step][layer], qin[step][layer], out=out)
            else:
                cache.append_kv_batch(layer, batch, kin[step][layer], vin[step][layer])
                cache.paged_decode(layer, batch, qin[step][layer], out=out)
            if step == 0 and layer == 0:
                torch.cuda.synchronize()
                _check_cow(cache, bm, pblocks, plen, parent, children, kin[0][0], vin[0][0], F, L, BS)
            for i, sl, ss in sample:
                if (sl, ss) == (layer, step):
                    outs[(i, sl, ss)] = out[i].clone()
            if step in WHOLE and layer in (0, L - 1):  # every fork, checked below
                whole[(step, layer)] = out.clone()
        if step == 0:
            sg, pages = cache.decode_sharing()
            assert sg == P and pages == P * 128, (sg, pages)  # every subgroup shares its 128 full prefix pages
        pos = [x + 1 for x in pos]
        for i, cid in enumerate(children):
            st = cache.seq_state(cid)
            assert st.cached_tokens == pos[i] and st.block_offset == pos[i] % BS, (cid, step)
    torch.cuda.synchronize()
    # every fork: the shared full prefix blocks, its copied tail, then the
    # blocks it gained, all private and distinct across forks
    for i, cid in enumerate(children):
        ids = cache.seq_state(cid).block_ids
        t = int(plen[parent[i]]) // BS
        assert ids[:t] == pblocks[parent[i]][:t]
        assert len(ids) == (pos[i] + BS - 1) // BS and set(ids[t + 1:]) == private[i], cid
        assert len(private[i]) == (pos[i] - 1) // BS - t, cid  # (pos - 1) // BS - t boundaries crossed
        assert all(bm.refcount(b) == 1 for b in ids[t:]), cid
    gained = [b for s_ in private for b in s_] + [cache.seq_state(c).block_ids[int(plen[parent[i]]) // BS]
                                                   for i, c in enumerate(children)]
    assert len(set(gained)) == len(gained)
    # positions 2048 + r .. 2111 + r (r in [1, 15]) cross 2064, 2080, 2096 and 2112: four blocks per fork
    assert sum(len(s_) for s_ in private) == 4 * n
    scale = np.float32(1 / math.sqrt(D))
    for (i, layer, step), o in outs.items():
        p = parent[i]
        ctx = int(plen[p]) + step + 1
        k_exp = np.concatenate([to_host(pk[p][layer])] + [to_host(kin[s][layer][i:i + 1]) for s in range(step + 1)])
        v_exp = np.concatenate([to_host(pv[p][layer])] + [to_host(vin[s][layer][i:i + 1]) for s in range(step + 1)])
        ids = cache.seq_state(children[i]).block_ids
        npg = (ctx + BS - 1) // BS
        idx = torch.tensor(ids[:npg], dtype=torch.int64, device="cuda")
        kpg = to_host(cache.k_pool(layer).index_select(0, idx))
        vpg = to_host(cache.v_pool(layer).index_select(0, idx))
        bt1 = np.arange(npg, dtype=np.int32)
        # pages written at this layer up to this step are the inputs, bit for bit
        assert np.array_equal(oracle.gather(kpg, oracle.BF16, bt1, ctx, Hkv, D, BS, np.uint16), k_exp)
        assert np.array_equal(oracle.gather(vpg, oracle.BF16, bt1, ctx, Hkv, D, BS, np.uint16), v_exp)
        # later steps overwrote nothing this decode read, so the final pages give its reference
        ref = oracle.paged_decode(as_f32(to_host(qin[step][layer][i:i + 1]), oracle.BF16), kpg, vpg, oracle.BF16,
                                  bt1[None, :], [ctx], Hkv, D, BS, scale, threads=8)
        assert max_abs_err(as_f32(to_host(o)[None], oracle.BF16), ref) <= 2e-2, (i, layer, step)
        # pins the torch decode used for the whole batch
        tref = torch_decode_ref(qin[step][layer][i:i + 1], cache.k_pool(layer), cache.v_pool(layer),
                                np.asarray(ids[:npg], np.int64)[None, :], [ctx], BS).cpu().numpy()
        assert max_abs_err(tref, ref) <= 1e-4, (i, layer, step)
    # the decode of every fork at the first and last layer on the WHOLE steps
    # against a plain PyTorch fp32 decode over the forks' final pages (shared
    # prefix pages, copied tails, the gained blocks and the appended tokens):
    # later steps only wrote positions past that step's context
    bt_all = np.full((n, MB), -1, np.int64)
    for i, cid in enumerate(children):
        ids = cache.seq_state(cid).block_ids
        bt_all[i, :len(ids)] = ids
    for (step, layer), o in sorted(whole.items()):
        ctxs = [int(plen[p]) + step + 1 for p in parent]
        tref = torch_decode_ref(qin[step][layer], cache.k_pool(layer), cache.v_pool(layer), bt_all, ctxs,
                                BS).cpu().numpy()
        assert max_abs_err(as_f32(to_host(o), oracle.BF16), tref) <= 2e-2, (step, layer)
    # release: the forks' references go, then the parents' last one bumps the generations
    for cid in children:
        cache.release_seq(cid)
    for p in range(P):
        assert all(bm.refcount(b) == 1 for b in pblocks[p])
    for p in range(P):
        cache.release_seq(f"p{p}")
    assert bm.free_blocks == NB
    with pytest.raises(RuntimeError, match="Stale handle") as e:
        bm.reference(ze.BlockHandle(pblocks[0][0], 1))
    assert e.value.fields == {"block_id": pblocks[0][0], "handle_gen": 1, "current_gen": 2}


def _check_cow(cache, bm, pblocks, plen, parent, children, k0, v0, F, L, BS):
    """After the first append at layer 0: each fork's partial tail block was
    copied into a fresh block in every pool, the shared tail lost one
    reference per fork, the full prefix blocks are still shared."""
    tails_c, tails_p, rows = [], [], []
    for i, cid in enumerate(children):
        p = parent[i]
        ids = cache.seq_state(cid).block_ids
        t = int(plen[p]) // BS
        assert ids[:t] == pblocks[p][:t] and ids[t] != pblocks[p][t]
        assert bm.refcount(ids[t]) == 1
        tails_c.append(ids[t])
        tails_p.append(pblocks[p][t])
        rows.append(int(plen[p]) % BS)
    for p in range(len(pblocks)):
        t = int(plen[p]) // BS
        assert bm.refcount(pblocks[p][t]) == 1                 # 1 + F references, F freed by the copies
        assert all(bm.refcount(b) == 1 + F for b in pblocks[p][:t])
    ic = torch.tensor(tails_c, dtype=torch.int64, device="cuda")
    ip = torch.tensor(tails_p, dtype=torch.int64, device="cuda")
    r = torch.tensor(rows, dtype=torch.int64, device="cuda")
    ar = torch.arange(len(children), device="cuda")
    for layer in range(L):
        for pool, new in ((cache.k_pool(layer), k0), (cache.v_pool(layer), v0)):
            got = pool.index_select(0, ic)    # [forks, Hkv, BS, D]
            want = pool.index_select(0, ip).clone()
            if layer == 0:                    # the appended token sits in row r of the copy
                want[ar, :, r, :] = new
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), layer
