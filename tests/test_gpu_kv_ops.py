"""KV append, block-table gather and copy-on-write block copy on the MI355X:
bit-exact against the CPU oracle, with canary fills proving nothing outside
the written slots changes."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, normal, paged_tables, to_dev, to_host

pytestmark = pytest.mark.gpu

CANARY16 = np.uint16(0x7FBF)  # a bf16 NaN pattern no append writes


def _slots_for(bt, starts, counts, BS):
    out = []
    for n, (s, c) in enumerate(zip(starts, counts)):
        g = s + np.arange(c)
        out.append(bt[n, g // BS].astype(np.int64) * BS + g % BS)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def _append_both(kp0, vp0, k, v, slots, cache_dt, src_dt, Hkv, D, BS, nb):
    from zealot_amd import ops
    kpd, vpd = to_dev(kp0), to_dev(vp0)
    ops.append(kpd, vpd, to_dev(k), to_dev(v), to_dev(slots))
    torch.cuda.synchronize()
    kr, vr = kp0.copy(), vp0.copy()
    oracle.append_slots(kr, vr, cache_dt, k, v, src_dt, slots, Hkv, D, BS, nb)
    return to_host(kpd), to_host(vpd), kr, vr


def test_c1_plumbing_append_fp32():
    """C1: 2 layers, 4 MHA heads, D=32, fp32, pool 256 x 16; prompts 17/40/77/130 then
    8 single-token decode appends per sequence; tables are a seeded permutation."""
    rng = np.random.default_rng(30)
    H, D, BS, NB, L = 4, 32, 16, 256, 2
    prompts = [17, 40, 77, 130]
    total = [p + 8 for p in prompts]
    perm = rng.permutation(NB).astype(np.int32)
    pages = [(t + BS - 1) // BS for t in total]
    bt = -np.ones((4, max(pages)), np.int32)
    o = 0
    for n, p in enumerate(pages):
        bt[n, :p] = perm[o:o + p]
        o += p
    announce("append C1 fp32")
    for layer in range(L):
        kp = np.zeros((NB, H, BS, D), np.float32)
        vp = np.zeros_like(kp)
        # prefill: one launch for all four prompts
        slots = _slots_for(bt, [0] * 4, prompts, BS)
        k = normal(rng, (len(slots), H, D), oracle.F32)
        v = normal(rng, (len(slots), H, D), oracle.F32)
        gk, gv, rk, rv = _append_both(kp, vp, k, v, slots, oracle.F32, oracle.F32, H, D, BS, NB)
        assert np.array_equal(gk, rk) and np.array_equal(gv, rv)
        kp, vp = rk, rv
        for step in range(8):  # decode steps, one token per sequence
            slots = _slots_for(bt, [p + step for p in prompts], [1] * 4, BS)
            k = normal(rng, (4, H, D), oracle.F32)
            v = normal(rng, (4, H, D), oracle.F32)
            gk, gv, rk, rv = _append_both(kp, vp, k, v, slots, oracle.F32, oracle.F32, H, D, BS, NB)
            assert np.array_equal(gk, rk) and np.array_equal(gv, rv)
            kp, vp = rk, rv


def test_c3_chunked_prefill_append_full_size_bitexact():
    """C3: 64 sequences x 512 new tokens at non-16-aligned offsets, bf16, Hkv=8, D=128."""
    rng = np.random.default_rng(31)
    N, C, H, D, BS = 64, 512, 8, 128, 16
    starts = rng.integers(0, 2048, N)
    starts[starts % BS == 0] += 1
    bt, nb = paged_tables(rng, starts + C, BS)
    slots = _slots_for(bt, starts, [C] * N, BS)
    announce(f"append C3 full size tokens={len(slots)} blocks={nb}")
    k = normal(rng, (len(slots), H, D), oracle.BF16)
    v = normal(rng, (len(slots), H, D), oracle.BF16)
    kp0 = np.full((nb, H, BS, D), CANARY16, np.uint16)
    vp0 = kp0.copy()
    gk, gv, rk, rv = _append_both(kp0, vp0, k, v, slots, oracle.BF16, oracle.BF16, H, D, BS, nb)
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)
    # canary: exactly the written slots changed
    written = np.zeros((nb, BS), bool)
    written[slots // BS, slots % BS] = True
    assert np.all(gk.transpose(0, 2, 1, 3)[~written] == CANARY16)


def test_append_skips_negative_slots_and_converts_dtypes():
    rng = np.random.default_rng(32)
    H, D, BS, NB = 8, 128, 16, 64
    slots = rng.permutation(NB * BS)[:300].astype(np.int64)
    slots[::7] = -1
    k = normal(rng, (300, H, D), oracle.F32)
    v = normal(rng, (300, H, D), oracle.F32)
    # f32 source into a bf16 pool (element kernel, RNE conversion)
    kp0 = np.full((NB, H, BS, D), CANARY16, np.uint16)
    gk, gv, rk, rv = _append_both(kp0, kp0.copy(), k, v, slots, oracle.BF16, oracle.F32, H, D, BS, NB)
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)
    # odd head_dim (row bytes not a multiple of 16) takes the element path too
    D2 = 20
    k2 = normal(rng, (300, H, D2), oracle.BF16)
    kp2 = np.zeros((NB, H, BS, D2), np.uint16)
    gk, gv, rk, rv = _append_both(kp2, kp2.copy(), k2, k2, slots, oracle.BF16, oracle.BF16, H, D2, BS, NB)
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)


@pytest.mark.parametrize("H,D,BS", [(8, 128, 16), (6, 96, 16), (8, 64, 32), (4, 128, 8), (3, 64, 16)])
def test_append_copy_shapes_bitexact(H, D, BS):
    """Same-dtype appends: power-of-two heads, rows and blocks take the
    shift-and-mask kernel, the others the general one; both bit-exact,
    slots of -1 skipped."""
    rng = np.random.default_rng(H * 1000 + D + BS)
    NB, T = 40, 250
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    slots[::9] = -1
    k = normal(rng, (T, H, D), oracle.BF16)
    v = normal(rng, (T, H, D), oracle.BF16)
    kp0 = np.full((NB, H, BS, D), CANARY16, np.uint16)
    announce(f"append copy H={H} D={D} BS={BS}")
    gk, gv, rk, rv = _append_both(kp0, kp0.copy(), k, v, slots, oracle.BF16, oracle.BF16, H, D, BS, NB)
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)


def test_fp8_append_bitexact_including_saturation_and_nan():
    from zealot_amd import ops
    rng = np.random.default_rng(33)
    H, D, BS, NB, T = 8, 128, 16, 32, 100
    k = (rng.standard_normal((T, H, D)) * 50).astype(np.float32)
    k[0, 0, :4] = [np.nan, -np.nan, np.inf, -1e30]
    v = (rng.standard_normal((T, H, D)) * 0.01).astype(np.float32)
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    rows = (np.arange(T) % 3).astype(np.int32)
    ks = np.abs(rng.standard_normal((3, H))).astype(np.float32) / 4 + 0.01
    vs = np.abs(rng.standard_normal((3, H))).astype(np.float32) / 400 + 1e-4
    for src in (oracle.F32, oracle.BF16):
        kk = k if src == oracle.F32 else oracle.bf16_bits_from_f32(k).reshape(k.shape)
        vv = v if src == oracle.F32 else oracle.bf16_bits_from_f32(v).reshape(v.shape)
        kp = torch.zeros((NB, H, BS, D), dtype=torch.uint8, device="cuda")
        vp = torch.zeros_like(kp)
        ops.append(kp, vp, to_dev(kk), to_dev(vv), to_dev(slots), k_scales=to_dev(ks),
                   v_scales=to_dev(vs), token_row=to_dev(rows))
        torch.cuda.synchronize()
        rk = np.zeros((NB, H, BS, D), np.uint8)
        rv = np.zeros_like(rk)
        oracle.append_slots(rk, rv, oracle.FP8, kk, vv, src, slots, H, D, BS, NB, ks, vs, rows)
        assert np.array_equal(to_host(kp), rk), src
        assert np.array_equal(to_host(vp), rv), src


def test_gather_bitexact_roundtrip_and_sentinel():
    from zealot_amd import ops
    rng = np.random.default_rng(34)
    H, D, BS = 8, 128, 16
    lens = np.array([1, 16, 17, 500, 1234, 0, 77])
    bt, nb = paged_tables(rng, lens, BS)
    kp = normal(rng, (nb, H, BS, D), oracle.BF16)
    vp = normal(rng, (nb, H, BS, D), oracle.BF16)
    bt = bt.copy()
    bt[4, 10] = -1  # seq 4 stops after 160 tokens
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    T = int(lens.sum())
    ko = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    vo = torch.full_like(ko, float("nan"))
    announce("gather bf16")
    ops.gather(to_dev(kp), to_dev(vp), to_dev(bt), to_dev(lens.astype(np.int32)), to_dev(offs), ko, vo)
    torch.cuda.synchronize()
    gk, gv = to_host(ko), to_host(vo)
    for n, L in enumerate(lens):
        rk = oracle.gather(kp, oracle.BF16, bt[n], int(L), H, D, BS, np.uint16)
        rv = oracle.gather(vp, oracle.BF16, bt[n], int(L), H, D, BS, np.uint16)
        got_k = gk[offs[n]: offs[n] + len(rk)]
        assert np.array_equal(got_k, rk) and np.array_equal(gv[offs[n]: offs[n] + len(rv)], rv)
        # rows past a sentinel are untouched (still NaN)
        tail = gk[offs[n] + len(rk): offs[n] + L]
        assert np.all(np.isnan(oracle.f32_from_bf16_bits(tail.ravel())))


def test_copy_blocks_all_layers_bitexact():
    from zealot_amd import ops
    rng = np.random.default_rng(35)
    H, D, BS, NB, L = 8, 128, 16, 40, 40  # 80 pools > 64 per launch
    pools_h = [rng.integers(0, 65535, (NB, H, BS, D), dtype=np.uint16) for _ in range(2 * L)]
    pools = [to_dev(p) for p in pools_h]
    src = np.array([3, 7, 11, 20], np.int32)
    dst = np.array([30, 31, 0, 39], np.int32)
    announce("copy_blocks 80 pools")
    ops.copy_blocks(pools, to_dev(src), to_dev(dst))
    torch.cuda.synchronize()
    ref = [p.copy() for p in pools_h]
    oracle.copy_blocks(ref, H * BS * D * 2, src, dst)
    for g, r in zip(pools, ref):
        assert np.array_equal(to_host(g), r)


@pytest.mark.parametrize("H,D,BS", [(8, 128, 16), (1, 64, 16), (3, 96, 16), (2, 128, 8)])
def test_copy_blocks_block_sizes_bitexact(H, D, BS):
    """Blocks of whole 4 KiB pieces (32 KiB, 4 KiB) take the one-chunk-per-
    thread kernel, the rest (2 KiB, 9 KiB) the per-block loop; ids outside
    the pool skip their pair in both."""
    from zealot_amd import ops
    rng = np.random.default_rng(H * 1000 + D + BS)
    NB = 24
    pools_h = [rng.integers(0, 65535, (NB, H, BS, D), dtype=np.uint16) for _ in range(6)]
    pools = [to_dev(p) for p in pools_h]
    src = np.array([3, 7, -1, 20, 5, 40], np.int32)
    dst = np.array([10, 11, 12, 23, NB, 0], np.int32)
    announce(f"copy_blocks block {H}x{BS}x{D} bf16")
    ops.copy_blocks(pools, to_dev(src), to_dev(dst))
    torch.cuda.synchronize()
    ref = [p.copy() for p in pools_h]
    keep = (src >= 0) & (src < NB) & (dst >= 0) & (dst < NB)
    oracle.copy_blocks(ref, H * BS * D * 2, src[keep], dst[keep])
    for g, r in zip(pools, ref):
        assert np.array_equal(to_host(g), r)


@pytest.mark.parametrize("H,D,BS", [(8, 128, 16), (2, 128, 8)])
def test_copy_blocks_runs_of_one_source_bitexact(H, D, BS):
    """Forks copying one shared block give many pairs with the same source
    (the copy-on-write of a forked prefix's tail): runs of 1, 3, 16, 17 and
    40 pairs, a source repeated in two separate runs, an invalid source and
    invalid destinations inside runs, bit-exact against the oracle's
    pair-by-pair copy, for the piece kernel and the per-block kernel."""
    from zealot_amd import ops
    rng = np.random.default_rng(36 + H)
    NB = 200
    lengths = [1, 3, 16, 17, 40, 5, 2]
    sources = [5, 9, 13, 17, 21, 9, -1]  # 9 appears in two runs; -1 is skipped
    src = np.concatenate([np.full(n, s_, np.int32) for n, s_ in zip(lengths, sources)])
    dst = (np.arange(len(src), dtype=np.int32) + 60)  # distinct, none a source
    dst[[4, 30, 70]] = [NB, -3, NB + 1]              # skipped destinations inside runs
    pools_h = [rng.integers(0, 65535, (NB, H, BS, D), dtype=np.uint16) for _ in range(4)]
    pools = [to_dev(p) for p in pools_h]
    announce(f"copy_blocks runs {lengths} block {H}x{BS}x{D}")
    ops.copy_blocks(pools, to_dev(src), to_dev(dst))
    torch.cuda.synchronize()
    ref = [p.copy() for p in pools_h]
    keep = (src >= 0) & (src < NB) & (dst >= 0) & (dst < NB)
    oracle.copy_blocks(ref, H * BS * D * 2, src[keep], dst[keep])
    for g, r in zip(pools, ref):
        assert np.array_equal(to_host(g), r)


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, (10 << 20) + 48])
def test_stream_yardsticks(nbytes):
    """The bandwidth yardsticks: the copy is bit-exact, the read leaves its
    sink alone for an all-zero buffer (its fold is zero)."""
    import ctypes
    from zealot_amd import _lib
    lib = _lib.lib()
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda")
    dst = torch.zeros_like(src)
    announce(f"stream copy/read {nbytes} bytes")
    _lib.check(lib.zk_stream_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), nbytes, None))
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    zeros = torch.zeros_like(src)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    _lib.check(lib.zk_stream_read(ctypes.c_void_p(zeros.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()), None))
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def test_gather_is_invariant_to_moving_blocks():
    """Moving every block to another physical id (pool rows permuted, tables
    renumbered the same way) leaves the gathered contexts bit for bit the
    same: the gather depends on the tables' contents, not on where blocks
    sit (paged_attention.cu:63-83)."""
    from zealot_amd import ops
    rng = np.random.default_rng(71)
    H, D, BS = 8, 128, 16
    lens = np.array([1, 16, 17, 300, 999])
    bt, nb = paged_tables(rng, lens, BS)
    kp = normal(rng, (nb, H, BS, D), oracle.BF16)
    vp = normal(rng, (nb, H, BS, D), oracle.BF16)
    move = rng.permutation(nb)  # block b now lives at move[b]
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[move], vp2[move] = kp, vp
    bt2 = np.where(bt >= 0, move[np.maximum(bt, 0)], -1).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    T = int(lens.sum())
    outs = []
    announce("gather after moving every block")
    for k_, v_, t_ in ((kp, vp, bt), (kp2, vp2, bt2)):
        ko = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
        vo = torch.full_like(ko, float("nan"))
        ops.gather(to_dev(k_), to_dev(v_), to_dev(t_), to_dev(lens.astype(np.int32)), to_dev(offs), ko, vo)
        torch.cuda.synchronize()
        outs.append((to_host(ko), to_host(vo)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert not np.any(np.isnan(oracle.f32_from_bf16_bits(outs[0][0].ravel())))
