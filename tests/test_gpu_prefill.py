"""Chunked-prefill attention over pages (zk_paged_prefill) on the MI355X against
the oracle's or_paged_prefill on the same seeded inputs: causal (row t of a
chunk after `start` cached tokens sees positions [0, start + t],
attention.cu:117-121) and non-causal (CpuAttention::forward), both GQA
mappings, bf16 and fp8 pools, f32 and bf16 queries, ragged and empty chunks,
sentinel-cut tables, and C3's chunks at full size (every row against a
PyTorch fp32 causal prefill pinned to the oracle, sampled rows against the
oracle).
Tolerance: 2e-2 absolute (bf16 products / bf16 outputs)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, max_abs_err, normal, paged_tables, to_dev, to_host

pytestmark = pytest.mark.gpu


def _case(seed, H, Hkv, D, starts, chunks, kv="bf16", qdt="bf16"):
    rng = np.random.default_rng(seed)
    lens = [s + c for s, c in zip(starts, chunks)]
    bt, nb = paged_tables(rng, lens, 16)
    src = oracle.BF16
    kx = normal(rng, (nb, Hkv, 16, D), src)
    vx = normal(rng, (nb, Hkv, 16, D), src)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int64)
    q = normal(rng, (int(cu[-1]), H, D), oracle.BF16 if qdt == "bf16" else oracle.F32)
    ks = vs = None
    if kv == "fp8":
        # quantise whole pools with per-(seq, head) scales (the decode tests' policy)
        ks = (np.abs(as_f32(kx, src)).max() / 448 * (1 + rng.random((len(lens), Hkv)))).astype(np.float32)
        vs = (np.abs(as_f32(vx, src)).max() / 448 * (1 + rng.random((len(lens), Hkv)))).astype(np.float32)
        kp = np.zeros((nb, Hkv, 16, D), np.uint8)
        vp = np.zeros_like(kp)
        for n, L in enumerate(lens):
            pos = np.arange(L)
            slots = bt[n, pos // 16].astype(np.int64) * 16 + pos % 16
            kt = np.stack([kx[bt[n, p // 16], :, p % 16] for p in pos]) if L else np.zeros((0, Hkv, D), np.uint16)
            vt = np.stack([vx[bt[n, p // 16], :, p % 16] for p in pos]) if L else np.zeros((0, Hkv, D), np.uint16)
            oracle.append_slots(kp, vp, oracle.FP8, kt, vt, src, slots, Hkv, D, 16, nb, ks[n:n + 1], vs[n:n + 1],
                                np.zeros(L, np.int32))
        kvdt = oracle.FP8
    else:
        kp, vp, kvdt = kx, vx, oracle.BF16
    return q, kp, vp, kvdt, bt, cu, ks, vs


def _run(q, kp, vp, bt, cu, starts, causal, mapping, ks, vs):
    from zealot_amd import ops
    fp8 = kp.dtype == np.uint8
    kd = to_dev(kp).view(torch.float8_e4m3fn) if fp8 else to_dev(kp)
    vd = to_dev(vp).view(torch.float8_e4m3fn) if fp8 else to_dev(vp)
    out = ops.paged_prefill(to_dev(q), kd, vd, to_dev(bt), to_dev(cu), to_dev(np.asarray(starts, np.int32)),
                            causal=causal, mapping=mapping,
                            k_scales=None if ks is None else to_dev(ks), v_scales=None if vs is None else to_dev(vs))
    torch.cuda.synchronize()
    return to_host(out)


@pytest.mark.parametrize("G,D,kv,qdt,causal,mapping", [
    (4, 128, "bf16", "bf16", True, "grouped"),
    (4, 128, "bf16", "bf16", False, "grouped"),
    (1, 128, "bf16", "bf16", True, "grouped"),
    (2, 64, "bf16", "f32", True, "grouped"),
    (8, 128, "bf16", "bf16", True, "modulo"),
    (8, 64, "bf16", "bf16", False, "modulo"),
    (4, 128, "fp8", "bf16", True, "grouped"),
    (4, 64, "fp8", "f32", False, "grouped"),
])
def test_prefill_matches_oracle(G, D, kv, qdt, causal, mapping):
    Hkv = 2
    H = G * Hkv
    starts = [0, 0, 5, 16, 33, 100, 7, 250]
    chunks = [1, 70, 12, 16, 40, 129, 0, 65]  # ragged, a one-row chunk, an empty chunk
    q, kp, vp, kvdt, bt, cu, ks, vs = _case(100 + G + D + int(causal), H, Hkv, D, starts, chunks, kv, qdt)
    announce(f"prefill G={G} D={D} kv={kv} q={qdt} causal={causal} {mapping}")
    out = _run(q, kp, vp, bt, cu, starts, causal, mapping, ks, vs)
    ref = oracle.paged_prefill(as_f32(q, oracle.BF16) if qdt == "bf16" else q, kp, vp, kvdt, bt, cu, starts, Hkv,
                               D, 16, np.float32(1 / math.sqrt(D)), causal,
                               oracle.GROUPED if mapping == "grouped" else oracle.MODULO, ks, vs)
    got = as_f32(out, oracle.BF16) if qdt == "bf16" else out
    assert max_abs_err(got, ref) <= 2e-2


def test_prefill_sentinel_cuts_context():
    """A table entry < 0 or >= num_blocks inside the context ends the page walk
    for every row of the chunk (the decode's rule)."""
    H, Hkv, D = 8, 2, 128
    starts, chunks = [40, 0, 64], [30, 50, 20]
    q, kp, vp, kvdt, bt, cu, ks, vs = _case(7, H, Hkv, D, starts, chunks)
    bt = bt.copy()
    bt[0, 3] = -1              # context cut at 48 tokens
    bt[2, 2] = kp.shape[0] + 5  # out of range: cut at 32
    announce("prefill sentinels")
    out = _run(q, kp, vp, bt, cu, starts, True, "grouped", None, None)
    bt_ref = np.where(bt >= kp.shape[0], -1, bt).astype(np.int32)  # the same walk for the oracle's rule
    ref = oracle.paged_prefill(as_f32(q, oracle.BF16), kp, vp, kvdt, bt_ref, cu, starts, Hkv, D, 16,
                               np.float32(1 / math.sqrt(D)), True)
    assert max_abs_err(as_f32(out, oracle.BF16), ref) <= 2e-2


def test_prefill_c3_shape_sampled_rows():
    """C3's chunks at full size (64 sequences, 512 tokens at unaligned offsets
    < 4096, 32/8 heads, D = 128, bf16) in one call; 4 sequences x 3 x 16 rows
    are checked against the oracle (a causal sub-chunk of rows t0.. is the
    chunk that starts at start + t0), and every row of every chunk against a
    plain PyTorch fp32 causal prefill, itself within 1e-4 of the oracle on
    those rows."""
    from tests.gpu_util import torch_prefill_ref
    rng = np.random.default_rng(12)
    H, Hkv, D, N, C = 32, 8, 128, 64, 512
    starts = rng.integers(0, 4096, N)
    starts[starts % 16 == 0] += 1
    chunks = [C] * N
    q, kp, vp, kvdt, bt, cu, ks, vs = _case(13, H, Hkv, D, list(starts), chunks)
    announce("prefill C3 shape")
    out = _run(q, kp, vp, bt, cu, list(starts), True, "grouped", None, None)
    got = as_f32(out, oracle.BF16)
    qd, kd, vd = to_dev(q), to_dev(kp), to_dev(vp)
    tref = {}
    for n in range(N):
        a, b = int(cu[n]), int(cu[n + 1])
        tref[n] = torch_prefill_ref(qd[a:b], kd, vd, bt[n], int(starts[n]), 16).cpu().numpy()
        assert max_abs_err(got[a:b], tref[n]) <= 2e-2, n
    scale = np.float32(1 / math.sqrt(D))
    for n in (0, 21, 42, 63):
        for t0 in (0, 255, 496):
            rows = slice(int(cu[n]) + t0, int(cu[n]) + t0 + 16)
            ref = oracle.paged_prefill(as_f32(q[rows], oracle.BF16), kp, vp, kvdt, bt[n:n + 1],
                                       np.array([0, 16], np.int64), [int(starts[n]) + t0], Hkv, D, 16, scale, True)
            assert max_abs_err(got[rows], ref) <= 2e-2, (n, t0)
            assert max_abs_err(tref[n][t0:t0 + 16], ref) <= 1e-4, (n, t0)  # the torch prefill is the oracle's


def test_prefill_one_row_chunks_equal_decode():
    """One-row chunks at position p are decodes of p + 1 tokens: the prefill
    and decode kernels agree on the same pages."""
    from zealot_amd import ops
    H, Hkv, D = 32, 8, 128
    starts = [0, 15, 16, 200, 1000]
    q, kp, vp, kvdt, bt, cu, ks, vs = _case(14, H, Hkv, D, starts, [1] * 5)
    announce("prefill vs decode")
    out = _run(q, kp, vp, bt, cu, starts, True, "grouped", None, None)
    dec = ops.paged_decode(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt),
                           to_dev(np.asarray([s + 1 for s in starts], np.int32)))
    torch.cuda.synchronize()
    assert max_abs_err(as_f32(out, oracle.BF16), as_f32(to_host(dec), oracle.BF16)) <= 2e-2
