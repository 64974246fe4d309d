"""A runner's mixed prefill / decode step through the KVCache (write_batch +
attention_batch) on the MI355X: the per-sequence store_kv / append_kv /
paged_forward loop of cuda_runner.rs:274-461 done as one write launch and one
attention call per layer for the whole batch.

Every layer of every step is checked against the oracle's chunked prefill
(or_paged_prefill, causal) over the cache's own pools, with each entry's
chunk starting at the sequence's cached_tokens before the step; pool bytes
are checked against the oracle's writes at the end.  Covered: prompt chunks,
decodes, empty entries, forks with copy-on-write and shared-prefix decode
inside mixed steps, fp8 pools with per-(seq, head) scales, and an f32 pool
(no MFMA prefill kernel: every chunk row runs as a decode).
Tolerance: 2e-2 absolute for bf16 / fp8 pools, 1e-5 for f32."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, normal, to_dev, to_host
from tests.test_gpu_kv_cache import _expected_bytes

pytestmark = pytest.mark.gpu

# step -> {seq: tokens}; "fork" entries fork the parent before the step
SCHEDULE = [
    {"a": 64, "b": 20, "p": 128},
    {"a": 36, "b": 1, "p": 128, "d": 5},
    {"a": 1, "b": 1, "p": 44, "d": 40},
    {"fork": ("p", ["p0", "p1", "p2"]), "a": 1, "b": 17, "p0": 1, "p1": 1, "p2": 1, "d": 1, "p": 0},
    {"a": 1, "b": 1, "p0": 1, "p1": 1, "p2": 1, "d": 1},
    {"p0": 1, "a": 30, "p1": 1, "p2": 1},
    {"p": 1, "d": 3, "b": 1},
]


@pytest.mark.parametrize("kv", ["bf16", "fp8", "f32"])
def test_mixed_steps_match_oracle(kv):
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng({"bf16": 61, "fp8": 62, "f32": 63}[kv])
    L, H, Hkv, D, BS, NB, MB = 2, 16, 4, 128, 16, 96, 32
    fp8, f32 = kv == "fp8", kv == "f32"
    cdt = {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "f32": torch.float32}[kv]
    kvdt = {"bf16": oracle.BF16, "fp8": oracle.FP8, "f32": oracle.F32}[kv]
    src = oracle.F32 if f32 else oracle.BF16
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=cdt, max_seqs=16, max_blocks_per_seq=MB)
    toks, scales, cached = {}, {}, {}
    scale = np.float32(1 / math.sqrt(D))
    tol = 1e-5 if f32 else 2e-2
    for step, plan in enumerate(SCHEDULE):
        plan = dict(plan)
        if "fork" in plan:
            parent, kids = plan.pop("fork")
            for kid in kids:
                cache.fork_seq(parent, kid)
                toks[kid] = {l: (list(toks[parent][l][0]), list(toks[parent][l][1])) for l in range(L)}
                scales[kid] = scales.get(parent)
                cached[kid] = cached[parent]
        ids = list(plan)
        nt = [plan[s] for s in ids]
        for sid, n in zip(ids, nt):
            if sid not in cached:
                cache.register_seq(sid, MB)
                cached[sid] = 0
                toks[sid] = {l: ([], []) for l in range(L)}
                if fp8:
                    ks = (4.5 / 448 * (1 + rng.random((L, Hkv)))).astype(np.float32)
                    vs = (4.5 / 448 * (1 + rng.random((L, Hkv)))).astype(np.float32)
                    cache.set_fp8_scales(sid, ks.ravel(), vs.ravel())
                    scales[sid] = (ks, vs)
            while len(cache.seq_state(sid).block_ids) * BS < cached[sid] + n:
                cache.alloc_block(sid, bm)
        T = sum(nt)
        cu = np.concatenate([[0], np.cumsum(nt)]).astype(np.int64)
        batch = ze.SeqBatch(ids)
        announce(f"mixed step {step} kv={kv} counts={nt}")
        for layer in range(L):
            k = normal(rng, (T, Hkv, D), src)
            v = normal(rng, (T, Hkv, D), src)
            cache.write_batch(layer, batch, nt, to_dev(k), to_dev(v))
            for i, sid in enumerate(ids):
                toks[sid][layer][0].append(k[cu[i]:cu[i + 1]])
                toks[sid][layer][1].append(v[cu[i]:cu[i + 1]])
            q = normal(rng, (T, H, D), src)
            out = to_host(cache.attention_batch(layer, batch, nt, to_dev(q)))
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            bt = -np.ones((len(ids), MB), np.int32)
            for i, sid in enumerate(ids):
                b = cache.seq_state(sid).block_ids
                bt[i, :len(b)] = b
            kw = {}
            if fp8:
                kw = dict(k_scales=np.stack([scales[s][0][layer] for s in ids]),
                          v_scales=np.stack([scales[s][1][layer] for s in ids]))
            qf = q if f32 else as_f32(q, oracle.BF16)
            ref = oracle.paged_prefill(qf, kp, vp, kvdt, bt, cu, [cached[s] for s in ids], Hkv, D, BS, scale,
                                       True, **kw)
            got = out if f32 else as_f32(out, oracle.BF16)
            assert max_abs_err(got, ref) <= tol, (step, layer)
            if kv == "bf16" and step in (4, 5):
                sg, pages = cache.decode_sharing()
                assert sg >= 1 and pages >= 16, (step, sg, pages)  # p0..p2 share p's 18 full pages
        for sid, n in zip(ids, nt):
            cached[sid] += n
            assert cache.seq_state(sid).cached_tokens == cached[sid]
    torch.cuda.synchronize()
    for sid in cached:
        Tn = cached[sid]
        for layer in range(L):
            kk = np.concatenate(toks[sid][layer][0])
            vv = np.concatenate(toks[sid][layer][1])
            assert kk.shape[0] == Tn
            bt = np.asarray(cache.seq_state(sid).block_ids, np.int32)
            kp, vp = to_host(cache.k_pool(layer)), to_host(cache.v_pool(layer))
            if f32:
                gk = oracle.gather(kp, oracle.F32, bt, Tn, Hkv, D, BS, np.float32)
                gv = oracle.gather(vp, oracle.F32, bt, Tn, Hkv, D, BS, np.float32)
                assert np.array_equal(gk, kk) and np.array_equal(gv, vv), (sid, layer)
                continue
            sc = (scales[sid][0][layer][None], scales[sid][1][layer][None]) if fp8 else (None, None)
            ek, ev = _expected_bytes(kk, vv, oracle.BF16, Hkv, D, BS, *sc)
            pdt = np.uint8 if fp8 else np.uint16
            gk = oracle.gather(kp, kvdt, bt, Tn, Hkv, D, BS, pdt)
            gv = oracle.gather(vp, kvdt, bt, Tn, Hkv, D, BS, pdt)
            assert np.array_equal(gk, ek) and np.array_equal(gv, ev), (sid, layer)


def test_mixed_step_errors_write_nothing():
    """write_batch rejects a repeated id and a position without a block before
    writing anything; attention_batch rejects rows the layer does not hold."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    Hkv, D, BS = 2, 64, 16
    bm = ze.BlockManager(16, BS)
    cache = KVCache(16, BS, 2, Hkv, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=4)
    for sid in ("x", "y"):
        cache.register_seq(sid, 4)
        cache.alloc_block(sid, bm)
    announce("mixed step errors")
    k = torch.zeros(20, Hkv, D, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="twice"):
        cache.write_batch(0, ["x", "x"], [1, 1], k[:2], k[:2])
    with pytest.raises(RuntimeError, match="OOB"):
        cache.write_batch(0, ["x", "y"], [3, 17], k, k)  # y needs a second block
    for sid in ("x", "y"):
        assert cache.seq_state(sid).cached_tokens == 0
    q = torch.zeros(2, 8, D, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="fewer tokens"):
        cache.attention_batch(0, ["x", "y"], [1, 1], q)
    cache.write_batch(0, ["x", "y"], [1, 1], k[:2], k[:2])
    cache.attention_batch(0, ["x", "y"], [1, 1], q)  # layer 0 now holds one token each
    with pytest.raises(RuntimeError, match="fewer tokens"):
        cache.attention_batch(1, ["x", "y"], [1, 1], q)
    torch.cuda.synchronize()


def test_mixed_step_at_bench_shape_every_row():
    """The bench's runner step at its full shape (252 decodes with contexts
    U[512, 8192] and 4 prompt chunks of 512 tokens after U[0, 4096) cached
    ones, 32/8 heads of 128, bf16): one write_batch + attention_batch, every
    decode row against a plain PyTorch fp32 decode and every chunk row against
    a plain PyTorch fp32 causal prefill over the cache's pages (2e-2); both
    references pinned to the oracle on sampled rows (1e-4)."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    from zealot_amd.kv_cache import SeqBatch
    from tests.gpu_util import torch_decode_ref, torch_prefill_ref
    ND, NC, C, H, Hkv, D, BS = 252, 4, 512, 32, 8, 128, 16
    rng = np.random.default_rng(64)
    dec_ctx = rng.integers(512, 8193, ND)
    starts = rng.integers(0, 4096, NC)
    total = [int(x) for x in dec_ctx] + [int(s) + C for s in starts]
    pages = [(t + BS - 1) // BS for t in total]
    nb = sum(pages) + 16
    announce(f"mixed step at bench shape: {ND} decodes + {NC} chunks of {C}, {nb} blocks")
    bm = ze.BlockManager(nb, BS)
    cache = KVCache(nb, BS, 1, Hkv, D, dtype=torch.bfloat16, max_seqs=ND + NC, max_blocks_per_seq=max(pages))
    ids = [f"d{i}" for i in range(ND)] + [f"c{i}" for i in range(NC)]
    for sid, p in zip(ids, pages):
        cache.register_seq(sid, p)
        for _ in range(p):
            cache.alloc_block(sid, bm)
    before = [int(x) - 1 for x in dec_ctx] + [int(s) for s in starts]
    g = torch.Generator(device="cuda").manual_seed(64)
    allb = SeqBatch(ids)
    T0 = sum(before)
    k0 = torch.randn((T0, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    v0 = torch.randn((T0, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    cache.write_batch(0, allb, before, k0, v0)
    del k0, v0
    nt = [1] * ND + [C] * NC
    T = sum(nt)
    k = torch.randn((T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn((T, H, D), generator=g, device="cuda").to(torch.bfloat16)
    cache.write_batch(0, allb, nt, k, v)
    out = cache.attention_batch(0, allb, nt, q)
    torch.cuda.synchronize()
    got = as_f32(to_host(out), oracle.BF16)
    assert np.all(np.isfinite(got))
    blocks = [cache.seq_state(s).block_ids for s in ids]
    bt = np.full((ND, max(pages)), -1, np.int64)
    for i in range(ND):
        bt[i, :pages[i]] = blocks[i][:pages[i]]
    dref = torch_decode_ref(q[:ND], cache.k_pool(0), cache.v_pool(0), bt, dec_ctx, BS).cpu().numpy()
    assert max_abs_err(got[:ND], dref) <= 2e-2
    scale = np.float32(1 / math.sqrt(D))
    for i in rng.choice(ND, 3, replace=False):  # the torch decode is the oracle's
        L = int(dec_ctx[i])
        idx = torch.tensor(bt[i, :pages[i]], dtype=torch.int64, device="cuda")
        kp, vp = to_host(cache.k_pool(0).index_select(0, idx)), to_host(cache.v_pool(0).index_select(0, idx))
        ref = oracle.paged_decode(as_f32(to_host(q[i:i + 1]), oracle.BF16), kp, vp, oracle.BF16,
                                  np.arange(pages[i], dtype=np.int32)[None, :], [L], Hkv, D, BS, scale, threads=8)
        assert max_abs_err(dref[i:i + 1], ref) <= 1e-4, int(i)
    row = ND
    for c in range(NC):
        sid, st = ND + c, int(starts[c])
        pref = torch_prefill_ref(q[row:row + C], cache.k_pool(0), cache.v_pool(0), blocks[sid], st, BS).cpu().numpy()
        assert max_abs_err(got[row:row + C], pref) <= 2e-2, c
        if c == 0:  # the torch prefill is the oracle's, on the chunk's first 8 rows
            npg = (st + 8 + BS - 1) // BS
            idx = torch.tensor(blocks[sid][:npg], dtype=torch.int64, device="cuda")
            kp, vp = to_host(cache.k_pool(0).index_select(0, idx)), to_host(cache.v_pool(0).index_select(0, idx))
            ref = oracle.paged_prefill(as_f32(to_host(q[row:row + 8]), oracle.BF16), kp, vp, oracle.BF16,
                                       np.arange(npg, dtype=np.int32)[None, :], np.array([0, 8], np.int64), [st],
                                       Hkv, D, BS, scale, True, oracle.GROUPED)
            assert max_abs_err(pref[:8], ref) <= 1e-4
        row += C
