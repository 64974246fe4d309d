"""Paged decode attention on the MI355X against the CPU oracle.

Tolerances (absolute, on the output): 1e-5 for fp32 KV, 2e-2 for bf16 KV,
5e-2 for fp8 KV against the fp32 oracle on the bf16 inputs the fp8 pool was
quantised from.  The oracle computes in fp32 from the very same pool bytes.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, decode_case, max_abs_err, to_dev, to_host

pytestmark = pytest.mark.gpu

TOL = {oracle.F32: 1e-5, oracle.BF16: 2e-2}
ORACLE_DT = {oracle.F32: oracle.F32, oracle.BF16: oracle.BF16}


def _run(q, kp, vp, bt, lens, kv_dtype, mapping="grouped", **kw):
    from zealot_amd import ops
    out = ops.paged_decode(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt),
                           to_dev(np.asarray(lens, np.int32)), mapping=mapping, **kw)
    torch.cuda.synchronize()
    return as_f32(to_host(out), oracle.BF16 if out.dtype == torch.bfloat16 else oracle.F32)


def _oracle(q, kp, vp, bt, lens, kv_dtype, q_dtype, mapping):
    Hkv, D = kp.shape[1], kp.shape[3]
    qf = as_f32(q, q_dtype)
    m = oracle.GROUPED if mapping == "grouped" else oracle.MODULO
    return oracle.paged_decode(qf, kp, vp, kv_dtype, bt, lens, Hkv, D, kp.shape[2],
                               np.float32(1.0 / math.sqrt(D)), m, threads=8)


C2_LENS = [1, 15, 16, 17, 100, 511, 512, 513, 1000, 2048, 4097, 8192]


@pytest.mark.parametrize("mapping", ["grouped", "modulo"])
def test_c2_shape_bf16_small_batch(mapping):
    announce(f"decode bf16 H32/Hkv8/D128 lens={C2_LENS} mapping={mapping}")
    q, kp, vp, bt, nb = decode_case(20, 32, 8, 128, C2_LENS, oracle.BF16)
    got = _run(q, kp, vp, bt, C2_LENS, oracle.BF16, mapping)
    ref = _oracle(q, kp, vp, bt, C2_LENS, oracle.BF16, oracle.BF16, mapping)
    assert max_abs_err(got, ref) <= 2e-2


def test_c1_fp32_mha_d32():
    # C1: 2 layers, 4 heads MHA, D=32, fp32; contexts after prompt + 8 decode steps
    lens = [17 + 8, 40 + 8, 77 + 8, 130 + 8]
    announce(f"decode fp32 H4/Hkv4/D32 lens={lens}")
    q, kp, vp, bt, nb = decode_case(21, 4, 4, 32, lens, oracle.F32)
    got = _run(q, kp, vp, bt, lens, oracle.F32)
    ref = _oracle(q, kp, vp, bt, lens, oracle.F32, oracle.F32, "grouped")
    assert max_abs_err(got, ref) <= 1e-5


@pytest.mark.parametrize("H,Hkv,D,dt", [
    (8, 8, 128, oracle.BF16),    # G=1 (MHA) on MFMA
    (16, 8, 128, oracle.BF16),   # G=2
    (64, 8, 128, oracle.BF16),   # G=8
    (32, 8, 64, oracle.BF16),    # D=64
    (24, 8, 96, oracle.BF16),    # D=96 -> generic kernel
    (48, 4, 128, oracle.BF16),   # G=12 -> generic kernel
    (32, 8, 128, oracle.F32),    # fp32 GQA -> generic kernel
    (4, 4, 256, oracle.F32),     # D=256
])
def test_head_shapes(H, Hkv, D, dt):
    lens = [3, 16, 33, 700, 1500]
    announce(f"decode H{H}/Hkv{Hkv}/D{D} dt={dt} lens={lens}")
    q, kp, vp, bt, nb = decode_case(22 + H + D, H, Hkv, D, lens, dt)
    for mapping in ("grouped", "modulo"):
        got = _run(q, kp, vp, bt, lens, dt, mapping)
        ref = _oracle(q, kp, vp, bt, lens, dt, dt, mapping)
        assert max_abs_err(got, ref) <= TOL[dt], mapping


def test_f32_queries_on_bf16_pool():
    lens = [5, 300, 2100]
    q, kp, vp, bt, nb = decode_case(23, 32, 8, 128, lens, oracle.BF16, q_dtype=oracle.F32)
    got = _run(q, kp, vp, bt, lens, oracle.BF16)
    ref = _oracle(q, kp, vp, bt, lens, oracle.BF16, oracle.F32, "grouped")
    assert max_abs_err(got, ref) <= 2e-2


def test_empty_context_sentinel_and_out_of_range_ids():
    lens = [0, 40, 64, 50]
    q, kp, vp, bt, nb = decode_case(24, 32, 8, 128, lens, oracle.BF16)
    bt = bt.copy()
    bt[2, 2] = -1           # walk of seq 2 stops after 2 pages (32 tokens)
    bt[3, 1] = nb + 5       # an id outside the pool ends the walk too
    got = _run(q, kp, vp, bt, lens, oracle.BF16)
    assert np.all(got[0] == 0)
    ref_lens = [0, 40, 32, 16]
    ref = _oracle(q, kp, vp, bt, ref_lens, oracle.BF16, oracle.BF16, "grouped")
    assert max_abs_err(got, ref) <= 2e-2


@pytest.mark.parametrize("seed", range(10))
def test_random_batches_against_oracle(seed):
    """Seeded random batches: head counts and grouping (G in 1, 2, 4, 8), head
    size, KV dtype, mapping and batch size drawn per case; context lengths mix
    page and partition edges (0, 1, 15-17, multiples of 16 +- 1) with random
    ones; some tables carry spare columns, some a sentinel that ends the walk
    early (src/kernels/paged_attention.cu:63-83: the context is then the
    pages before it).  Every row against the fp32 oracle."""
    from tests.gpu_util import normal, paged_tables
    rng = np.random.default_rng(700 + seed)
    G = int(rng.choice([1, 2, 4, 8]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    H = G * Hkv
    D = int(rng.choice([64, 128]))
    dt = oracle.F32 if seed % 4 == 3 else oracle.BF16  # fp32 pools take the generic kernel
    mapping = "grouped" if rng.random() < 0.7 else "modulo"
    N = int(rng.integers(1, 49))
    edges = [0, 1, 15, 16, 17, 255, 256, 257, 767, 768, 769]
    lens = [int(rng.choice(edges)) if rng.random() < 0.4 else int(rng.integers(1, 3001)) for _ in range(N)]
    bt, nb = paged_tables(rng, lens, 16)
    if rng.random() < 0.5:  # spare columns past every sequence's pages
        bt = np.concatenate([bt, -np.ones((N, int(rng.integers(1, 9))), np.int32)], axis=1)
    ref_lens = list(lens)
    for i in range(N):
        pages = (lens[i] + 15) // 16
        if pages > 1 and rng.random() < 0.2:
            j = int(rng.integers(0, pages))
            bt[i, j] = -1 if rng.random() < 0.5 else nb + int(rng.integers(0, 100))
            ref_lens[i] = min(lens[i], 16 * j)
    kp = normal(rng, (nb, Hkv, 16, D), dt)
    vp = normal(rng, (nb, Hkv, 16, D), dt)
    q = normal(rng, (N, H, D), dt)
    announce(f"decode random case {seed}: H{H}/Hkv{Hkv}/D{D} dt={dt} {mapping} N={N} lens={lens}")
    got = _run(q, kp, vp, bt, lens, dt, mapping)
    ref = _oracle(q, kp, vp, bt, ref_lens, dt, dt, mapping)
    for i in range(N):
        if ref_lens[i] == 0:
            assert np.all(got[i] == 0), i
    assert max_abs_err(got, ref) <= TOL[dt]


def test_decode_is_deterministic():
    lens = [700, 4000]
    q, kp, vp, bt, nb = decode_case(25, 32, 8, 128, lens, oracle.BF16)
    a = _run(q, kp, vp, bt, lens, oracle.BF16)
    b = _run(q, kp, vp, bt, lens, oracle.BF16)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("src,lens", [
    (oracle.BF16, [1024, 3000, 5000, 16384]),  # C5 context range: the 5e-2 bar applies
    (oracle.F32, [1100, 2500, 9000]),
    (oracle.BF16, [1, 17, 200]),                # short contexts: fp8-oracle check only
])
def test_fp8_kv_decode(src, lens):
    """fp8 pools quantised on append (per-(seq, head) amax scales), decoded with
    fp32 accumulation.  For C5-range contexts (>= 1024 tokens) the output is
    within 5e-2 of the fp32 oracle on the unquantised inputs; for any context it
    is within 2e-2 of the oracle on the dequantised fp8 pages.  (At ctx = 1 the
    output is one dequantised V row, whose e4m3 rounding error -- up to 2^-4
    relative -- is not averaged away, so the 5e-2 bar is a long-context bar.)"""
    from zealot_amd import ops
    rng = np.random.default_rng(26)
    H, Hkv, D, BS = 32, 8, 128, 16
    from tests.gpu_util import normal, paged_tables
    bt, nb = paged_tables(rng, lens, BS)
    T = sum(lens)
    k = normal(rng, (T, Hkv, D), src)
    v = normal(rng, (T, Hkv, D), src)
    q = normal(rng, (len(lens), H, D), oracle.BF16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    slots = np.concatenate([bt[n, np.arange(L) // BS].astype(np.int64) * BS + np.arange(L) % BS
                            for n, L in enumerate(lens)])
    rows = np.repeat(np.arange(len(lens)), lens).astype(np.int32)
    announce(f"fp8 decode src={src} lens={lens}")
    kd, vd = to_dev(k), to_dev(v)
    ks = ops.fp8_scales(kd, to_dev(cu))
    vs = ops.fp8_scales(vd, to_dev(cu))
    kpool = torch.zeros((nb, Hkv, BS, D), dtype=torch.uint8, device="cuda")
    vpool = torch.zeros_like(kpool)
    ops.append(kpool, vpool, kd, vd, to_dev(slots), k_scales=ks, v_scales=vs, token_row=to_dev(rows))
    torch.cuda.synchronize()
    # scales and quantised pages are bit-exact against the oracle
    ks_ref = oracle.fp8_scales(k, src, cu, Hkv, D)
    vs_ref = oracle.fp8_scales(v, src, cu, Hkv, D)
    assert np.array_equal(to_host(ks), ks_ref) and np.array_equal(to_host(vs), vs_ref)
    kp_ref = np.zeros((nb, Hkv, BS, D), np.uint8)
    vp_ref = np.zeros_like(kp_ref)
    oracle.append_slots(kp_ref, vp_ref, oracle.FP8, k, v, src, slots, Hkv, D, BS, nb, ks_ref,
                        vs_ref, rows)
    assert np.array_equal(to_host(kpool), kp_ref) and np.array_equal(to_host(vpool), vp_ref)
    out = ops.paged_decode(to_dev(q), kpool, vpool, to_dev(bt), to_dev(np.asarray(lens, np.int32)),
                           k_scales=ks, v_scales=vs)
    torch.cuda.synchronize()
    got = as_f32(to_host(out), oracle.BF16)
    # against the fp32 oracle on the unquantised inputs (the bar)
    kp_src = np.zeros((nb, Hkv, BS, D), np.float32)
    vp_src = np.zeros_like(kp_src)
    oracle.append_slots(kp_src, vp_src, oracle.F32, as_f32(k, src), as_f32(v, src), oracle.F32,
                        slots, Hkv, D, BS, nb)
    if min(lens) >= 1024:
        ref = _oracle(q, kp_src, vp_src, bt, lens, oracle.F32, oracle.BF16, "grouped")
        assert max_abs_err(got, ref) <= 5e-2
    # and tightly against the oracle on the dequantised fp8 pages
    ref8 = oracle.paged_decode(as_f32(q, oracle.BF16), kp_ref, vp_ref, oracle.FP8, bt, lens, Hkv, D,
                               BS, np.float32(1 / math.sqrt(D)), oracle.GROUPED, ks_ref, vs_ref, threads=8)
    assert max_abs_err(got, ref8) <= 2e-2


def test_c2_full_size_sampled_against_oracle():
    """C2 at full size (256 seqs, ctx U[512, 8192], bf16) on the GPU; 8 sampled
    sequences are checked against the oracle on their own pages, and all 256
    against a plain PyTorch fp32 decode on the GPU, itself checked against
    the oracle on the sampled ones."""
    from zealot_amd import ops
    from tests.gpu_util import paged_tables, torch_decode_ref
    rng = np.random.default_rng(27)
    N, H, Hkv, D, BS = 256, 32, 8, 128, 16
    lens = rng.integers(512, 8193, N)
    bt, nb = paged_tables(rng, lens, BS)
    announce(f"decode C2 full size N={N} sum_ctx={int(lens.sum())} blocks={nb}")
    g = torch.Generator(device="cuda").manual_seed(27)
    kpool = torch.randn((nb, Hkv, BS, D), generator=g, device="cuda").to(torch.bfloat16)
    vpool = torch.randn((nb, Hkv, BS, D), generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn((N, H, D), generator=g, device="cuda").to(torch.bfloat16)
    btd = to_dev(bt)
    out = ops.paged_decode(q, kpool, vpool, btd, to_dev(lens.astype(np.int32)))
    torch.cuda.synchronize()
    got = as_f32(to_host(out), oracle.BF16)
    assert np.all(np.isfinite(got))
    tref = torch_decode_ref(q, kpool, vpool, bt, lens, BS).cpu().numpy()
    assert max_abs_err(got, tref) <= 2e-2  # every sequence
    pick = rng.choice(N, 8, replace=False)
    for n in pick:
        L = int(lens[n])
        pages = bt[n, : (L + BS - 1) // BS]
        idx = torch.from_numpy(pages.astype(np.int64)).cuda()
        kp = to_host(kpool.index_select(0, idx))
        vp = to_host(vpool.index_select(0, idx))
        bt1 = np.arange(len(pages), dtype=np.int32)[None, :]
        ref = _oracle(to_host(q[n:n + 1]), kp, vp, bt1, [L], oracle.BF16, oracle.BF16, "grouped")
        assert max_abs_err(got[n:n + 1], ref) <= 2e-2, int(n)
        assert max_abs_err(tref[n:n + 1], ref) <= 1e-4, int(n)  # the torch decode is the oracle's


@pytest.mark.parametrize("H,Hkv,D,dt", [(4, 4, 32, oracle.F32), (32, 8, 128, oracle.BF16)])
def test_hip_attention_paged_forward(H, Hkv, D, dt):
    """HipAttention.paged_forward, the mirror of CudaAttention::paged_forward
    (attention/cuda.rs:126-209): raw device addresses, scale 1/sqrt(D), grouped
    mapping; equal to ops.paged_decode and within tolerance of the oracle."""
    from zealot_amd import _lib
    from zealot_amd.attention import HipAttention
    lens = [1, 40, 300, 2049]
    q, kp, vp, bt, nb = decode_case(60 + D, H, Hkv, D, lens, dt)
    qd, kd, vd, btd = to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt)
    ld = to_dev(np.asarray(lens, np.int32))
    o = torch.empty_like(qd)
    zdt = _lib.F32 if dt == oracle.F32 else _lib.BF16
    att = HipAttention()
    for _ in range(2):  # the second call reuses the object's workspace
        att.paged_forward(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), btd.data_ptr(), ld.data_ptr(), o.data_ptr(),
                          len(lens), H, Hkv, D, 16, bt.shape[1], nb, q_dtype=zdt, kv_dtype=zdt)
    torch.cuda.synchronize()
    got = as_f32(to_host(o), dt)
    assert np.array_equal(got, _run(q, kp, vp, bt, lens, dt))
    assert max_abs_err(got, _oracle(q, kp, vp, bt, lens, dt, dt, "grouped")) <= TOL[dt]
    with pytest.raises(RuntimeError, match="multiple of num_kv_heads"):
        att.paged_forward(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), btd.data_ptr(), ld.data_ptr(),
                          o.data_ptr(), len(lens), H + 1, Hkv, D, 16, bt.shape[1], nb, q_dtype=zdt, kv_dtype=zdt)


def test_fp8_decode_dequantises_every_e4m3_code_exactly():
    """All 256 e4m3 codes through the fp8 decode's in-register dequantisation:
    a one-token context with zero K (every score 0, weight 1) and unit scales
    returns the V row itself, so each output element is the code's exact value
    in bf16 (every e4m3 value is a bf16 value; the two NaN codes give NaN).  The decoded values are pinned by the OCP e4m3 definition
    through oracle.f32_from_e4m3_bits (tests/test_oracle.py)."""
    from zealot_amd import ops
    H, Hkv, D, BS = 1, 1, 128, 16
    codes = np.arange(256, dtype=np.uint8)
    n = 256 // D
    kp = torch.zeros((n, Hkv, BS, D), dtype=torch.uint8, device="cuda")
    vp = torch.zeros_like(kp)
    vp[:, 0, 0, :] = torch.from_numpy(codes.reshape(n, D)).cuda()
    bt = np.arange(n, dtype=np.int32).reshape(n, 1)
    ones = torch.ones((n, Hkv), dtype=torch.float32, device="cuda")
    q = torch.zeros((n, H, D), dtype=torch.bfloat16, device="cuda")
    announce("fp8 decode: every e4m3 code")
    out = ops.paged_decode(q, kp, vp, to_dev(bt), to_dev(np.ones(n, np.int32)), k_scales=ones, v_scales=ones)
    torch.cuda.synchronize()
    got = as_f32(to_host(out), oracle.BF16).reshape(-1)
    want = oracle.f32_from_e4m3_bits(codes).reshape(-1)
    nan = np.isnan(want)
    assert nan.sum() == 2 and np.all(np.isnan(got[nan]))
    assert np.array_equal(got[~nan], want[~nan])  # exact values (-0 comes back as +0 from the accumulators)


@pytest.mark.parametrize("H,Hkv,D,dt", [(32, 8, 128, torch.bfloat16), (16, 16, 64, torch.bfloat16),
                                        (4, 4, 32, torch.float32)])
def test_decode_closed_forms(H, Hkv, D, dt):
    """Properties the softmax fixes, checked on the kernel itself rather than
    through the oracle (attention/mod.rs:64-98): a one-token context returns
    that token's V row exactly; keys all equal give the mean of V; one key far
    above the others gives its V row; adding the same vector to every key
    (exact in bf16) leaves the output unchanged.  Lengths cross several
    split-K partitions on the MFMA path (bf16) and run the generic path (f32)."""
    from zealot_amd import ops
    g = torch.Generator(device="cuda").manual_seed(H * 1000 + D)
    BS, N = 16, 6
    lens = [1, 1, 300, 2000, 4096 + 7, 700]
    pages = [(L + BS - 1) // BS for L in lens]
    NB = sum(pages) + 8
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(5)).to(torch.int32)
    bt = torch.full((N, max(pages)), -1, dtype=torch.int32)
    o = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[o:o + p]
        o += p
    btd = bt.cuda()
    ld = torch.tensor(lens, dtype=torch.int32, device="cuda")

    def quant(x):  # multiples of 1/16 in [-4, 4]: exact in bf16, and so is x + 8
        return (torch.round(x * 16).clamp(-64, 64) / 16).to(dt)

    q = quant(torch.randn((N, H, D), generator=g, device="cuda") * 0.5)
    vp = quant(torch.randn((NB, Hkv, BS, D), generator=g, device="cuda"))
    kp = quant(torch.randn((NB, Hkv, BS, D), generator=g, device="cuda") * 0.5)
    G = H // Hkv
    announce(f"decode closed forms H{H}/Hkv{Hkv}/D{D} {dt}")

    def ctx_rows(pool, i):  # sequence i's rows [len, Hkv, D] in token order
        blocks = bt[i, :pages[i]].long().cuda()
        return pool[blocks].permute(0, 2, 1, 3).reshape(-1, Hkv, D)[:lens[i]].float()

    out = ops.paged_decode(q, kp, vp, btd, ld)
    torch.cuda.synchronize()
    # one-token contexts: exactly that token's V row
    for i in (0, 1):
        v0 = ctx_rows(vp, i)[0]
        for h in range(H):
            assert torch.equal(out[i, h].float(), v0[h // G]), (i, h)
    # keys all equal (every row of every page the same vector): the mean of V
    kc = kp.clone()
    kc[:] = kp[0, 0, 0]
    outc = ops.paged_decode(q, kc, vp, btd, ld)
    torch.cuda.synchronize()
    tol = 2e-2 if dt == torch.bfloat16 else 1e-5
    for i in range(N):
        mean = ctx_rows(vp, i).mean(0)
        for h in range(H):
            assert (outc[i, h].float() - mean[h // G]).abs().max() <= tol * max(1.0, mean.abs().max()), (i, h)
    # one dominant key per (sequence, kv-head): 2^6 x q's direction at one position
    kd = kp.clone()
    pos = [0, 0, 123, 1999, 4100, 350]
    for i in range(N):
        blk, t = int(bt[i, pos[i] // BS]), pos[i] % BS
        for kvh in range(Hkv):
            qs = q[i, kvh * G:(kvh + 1) * G].float().sum(0)  # grouped heads of this kv-head
            kd[blk, kvh, t] = (torch.sign(qs) * 4).to(dt)
    sc = 64.0 / math.sqrt(D)
    outd = ops.paged_decode(q, kd, vp, btd, ld, scale=sc)
    torch.cuda.synchronize()
    checked = 0
    for i in range(2, N):
        vrow, krows = ctx_rows(vp, i)[pos[i]], ctx_rows(kd, i)
        for h in range(H):
            s_ = krows[:, h // G] @ q[i, h].float() * sc
            others = torch.cat([s_[:pos[i]], s_[pos[i] + 1:]])
            if s_[pos[i]] - others.max() >= 40.0:  # every other weight below e^-40
                checked += 1
                assert (outd[i, h].float() - vrow[h // G]).abs().max() <= 2 * tol * max(1.0, vrow.abs().max()), (i, h)
    assert checked >= H  # the construction makes most heads dominant
    # the same vector added to every key: scores shift by q.u per head, softmax unchanged
    outs = ops.paged_decode(q, (kp.float() + 8.0).to(dt), vp, btd, ld)
    torch.cuda.synchronize()
    assert (outs.float() - out.float()).abs().max() <= 2 * tol * max(1.0, out.float().abs().max())
