"""KV swap (zk_cache_swap_out / zk_cache_swap_in) on the MI355X: host <->
device block moves for preemption (docs/architecture.md:452-469, no
reference code).

Pool bytes of every swapped sequence come back bit-exact in freshly allocated
blocks after the old blocks were handed to another sequence and overwritten;
attention after swap-in matches the oracle; the BlockManager and the host
space return to their starting counts; swapped sequences refuse writes and
attention; staging in several chunks (more than 512 MiB of blocks) moves the
same bytes; a scheduler-driven model loop with swap preemption is in
test_gpu_model.py."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, normal, to_dev, to_host

pytestmark = pytest.mark.gpu


def _pools(cache, L):
    return [(to_host(cache.k_pool(l)), to_host(cache.v_pool(l))) for l in range(L)]


def _seq_bytes(pools, blocks, T, Hkv, D, BS, dt, pdt):
    bt = np.asarray(blocks, np.int32)
    return [(oracle.gather(kp, dt, bt, T, Hkv, D, BS, pdt), oracle.gather(vp, dt, bt, T, Hkv, D, BS, pdt))
            for kp, vp in pools]


@pytest.mark.parametrize("kv", ["bf16", "fp8", "f32"])
def test_swap_round_trip_bit_exact(kv):
    import zealot_amd as ze
    from zealot_amd import KVCache
    rng = np.random.default_rng({"bf16": 81, "fp8": 82, "f32": 83}[kv])
    L, H, Hkv, D, BS, NB = 3, 8, 2, 128, 16, 48
    cdt = {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "f32": torch.float32}[kv]
    dt = {"bf16": oracle.BF16, "fp8": oracle.FP8, "f32": oracle.F32}[kv]
    pdt = {"bf16": np.uint16, "fp8": np.uint8, "f32": np.float32}[kv]
    src = oracle.F32 if kv == "f32" else oracle.BF16
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=cdt, max_seqs=8, max_blocks_per_seq=16)
    cache.enable_swap(20)
    lens = {"x": 37, "y": 16, "z": 100}
    scales = {}
    for sid, T in lens.items():
        cache.register_seq(sid, 16)
        for _ in range((T + BS - 1) // BS + 1):  # one spare block beyond the written ones
            cache.alloc_block(sid, bm)
        if kv == "fp8":
            scales[sid] = (rng.random((L, Hkv)).astype(np.float32) / 100 + 0.01,
                           rng.random((L, Hkv)).astype(np.float32) / 100 + 0.01)
            cache.set_fp8_scales(sid, scales[sid][0].ravel(), scales[sid][1].ravel())
        for l in range(L):
            cache.store_kv(l, sid, to_dev(normal(rng, (T, Hkv, D), src)), to_dev(normal(rng, (T, Hkv, D), src)), 0, T)
    announce(f"swap round trip {kv}")
    before = _pools(cache, L)
    ref = {sid: _seq_bytes(before, cache.seq_state(sid).block_ids, T, Hkv, D, BS, dt, pdt) for sid, T in lens.items()}
    free0 = bm.free_blocks
    cache.swap_out(["x", "z"])
    assert cache.is_swapped("x") and cache.is_swapped("z") and not cache.is_swapped("y")
    assert cache.seq_state("x").block_ids == [] and cache.seq_state("x").cached_tokens == 37
    assert bm.free_blocks == free0 + 4 + 8  # every block, the spare ones included
    assert cache.swap_space() == (20, 20 - 3 - 7)  # written blocks only
    # hand the freed blocks to someone else and overwrite them
    cache.register_seq("w", 16)
    for _ in range(12):
        cache.alloc_block("w", bm)
    if kv == "fp8":
        cache.set_fp8_scales("w", np.ones(L * Hkv, np.float32), np.ones(L * Hkv, np.float32))
    for l in range(L):
        cache.store_kv(l, "w", to_dev(normal(rng, (192, Hkv, D), src)), to_dev(normal(rng, (192, Hkv, D), src)), 0, 192)
    with pytest.raises(RuntimeError, match="swapped out"):
        cache.store_kv(0, "x", to_dev(normal(rng, (1, Hkv, D), src)), to_dev(normal(rng, (1, Hkv, D), src)), 37, 1)
    with pytest.raises(RuntimeError, match="swapped out"):
        cache.paged_decode(0, ["z"], to_dev(normal(rng, (1, H, D), oracle.BF16)))
    cache.release_seq("w")
    cache.swap_in(["z", "x"], bm)
    assert cache.swap_space() == (20, 20)
    assert not cache.is_swapped("x")
    after = _pools(cache, L)
    for sid, T in lens.items():
        got = _seq_bytes(after, cache.seq_state(sid).block_ids, T, Hkv, D, BS, dt, pdt)
        for l in range(L):
            assert np.array_equal(got[l][0], ref[sid][l][0]) and np.array_equal(got[l][1], ref[sid][l][1]), (sid, l)
    # attention over the restored pages
    ids = list(lens)
    qdt = oracle.F32 if kv == "f32" else oracle.BF16
    q = normal(rng, (3, H, D), qdt)
    out = to_host(cache.paged_decode(1, ids, to_dev(q)))
    kp, vp = after[1]
    bt = -np.ones((3, 16), np.int32)
    for i, sid in enumerate(ids):
        b = cache.seq_state(sid).block_ids
        bt[i, :len(b)] = b
    kw = {}
    if kv == "fp8":
        kw = dict(k_scales=np.stack([scales[s][0][1] for s in ids]), v_scales=np.stack([scales[s][1][1] for s in ids]))
    exp = oracle.paged_decode(as_f32(q, qdt), kp, vp, dt, bt, [lens[s] for s in ids], Hkv, D, BS,
                              np.float32(1 / math.sqrt(D)), **kw)
    assert max_abs_err(as_f32(out, qdt), exp) <= (1e-5 if kv == "f32" else 2e-2)
    # a release of a swapped sequence frees its host slots
    cache.swap_out(["y"])
    assert cache.swap_space()[1] == 19
    cache.release_seq("y")
    assert cache.swap_space()[1] == 20
    torch.cuda.synchronize()


def test_swap_errors_leave_state_unchanged():
    import zealot_amd as ze
    from zealot_amd import KVCache
    bm = ze.BlockManager(8, 16)
    cache = KVCache(8, 16, 1, 2, 64, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=4)
    announce("swap errors")
    cache.register_seq("a", 4)
    for _ in range(3):
        cache.alloc_block("a", bm)
    k = torch.zeros(40, 2, 64, dtype=torch.bfloat16, device="cuda")
    cache.store_kv(0, "a", k, k, 0, 40)
    with pytest.raises(RuntimeError, match="no swap space"):
        cache.swap_out(["a"])
    cache.enable_swap(2)
    with pytest.raises(RuntimeError, match="Out of blocks"):  # 3 written blocks, 2 host slots
        cache.swap_out(["a"])
    assert not cache.is_swapped("a") and len(cache.seq_state("a").block_ids) == 3
    with pytest.raises(RuntimeError, match="not swapped"):
        cache.swap_in(["a"], bm)
    torch.cuda.synchronize()


def test_swap_in_chunks_beyond_the_staging_size():
    """More than 512 MiB of blocks: staged in several chunks, bytes compared on
    the device."""
    import zealot_amd as ze
    from zealot_amd import KVCache
    L, Hkv, D, BS = 4, 8, 128, 16  # 256 KiB per host slot -> 2048 slots per chunk
    T = 40000
    nblk = (T + BS - 1) // BS
    NB = nblk * 2 + 8
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=4, max_blocks_per_seq=nblk)
    cache.enable_swap(nblk)
    cache.register_seq("big", nblk)
    for _ in range(nblk):
        cache.alloc_block("big", bm)
    g = torch.Generator(device="cuda").manual_seed(5)
    for l in range(L):
        x = torch.randn((T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        cache.store_kv(l, "big", x, x * 2, 0, T)
    announce("swap chunked")
    old = torch.tensor(cache.seq_state("big").block_ids, device="cuda")
    want = [(cache.k_pool(l).index_select(0, old).clone(), cache.v_pool(l).index_select(0, old).clone())
            for l in range(L)]
    # occupy the low block ids so the swap-in lands elsewhere
    cache.register_seq("pad", nblk)
    cache.swap_out(["big"])
    for _ in range(min(nblk, NB - nblk)):
        cache.alloc_block("pad", bm)
    cache.swap_in(["big"], bm)
    new = torch.tensor(cache.seq_state("big").block_ids, device="cuda")
    assert not torch.equal(new, old)
    for l in range(L):
        assert torch.equal(cache.k_pool(l).index_select(0, new), want[l][0])
        assert torch.equal(cache.v_pool(l).index_select(0, new), want[l][1])
    torch.cuda.synchronize()
