"""Pins the CPU oracle (oracle/zk_oracle.c) before it is trusted as the checker.

Every check here is independent of the oracle's own arithmetic: the
reference's known answers (tests/golden), torch's float8_e4m3fn and
scaled_dot_product_attention (library routines), numpy's C-order indexing
of a [blocks, Hkv, bs, D] array (the layout of src/kv_cache.rs:41-50),
closed forms, and round trips.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _arr(spec):
    if isinstance(spec, str):
        kind, n = spec.split(":")
        n = int(n)
        return np.ones(n, np.float32) if kind == "ones" else np.arange(n, dtype=np.float32)
    return np.asarray(spec, dtype=np.float32)


# ---------------------------------------------------------------- known answers

@pytest.mark.parametrize("case", GOLD["matmul"], ids=lambda c: c["source"])
def test_matmul_known_answer(case):
    c = oracle.matmul(_arr(case["a"]), _arr(case["b"]), case["m"], case["k"], case["n"])
    assert c.tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLD["cpu_attention"], ids=lambda c: c["name"])
def test_cpu_attention_known_answers(case):
    args = (case["num_seqs"], case["num_heads"], case["head_dim"], case["max_seq_len"])
    q, k, v = _arr(case["q"]), _arr(case["k"]), _arr(case["v"])
    if "expected_error" in case:
        with pytest.raises(RuntimeError, match=case["expected_error"]):
            oracle.cpu_attention(q, k, v, *args)
        return
    out = oracle.cpu_attention(q, k, v, *args)
    if "expected_len" in case:
        assert out.size == case["expected_len"]
        # all-ones V: every softmax-weighted average is exactly 1
        assert np.all(out == 1.0)
    if "expected_outputs_differ" in case:
        (a0, a1), (b0, b1) = case["expected_outputs_differ"]
        assert not np.array_equal(out[a0:a1], out[b0:b1])


@pytest.mark.parametrize("case", GOLD["repeat_interleave_kv"], ids=lambda c: c["source"])
def test_repeat_interleave_known_answer(case):
    out = oracle.repeat_interleave_kv(_arr(case["src"]), case["kv_heads"], case["num_heads"],
                                      case["seq_len"], case["head_dim"])
    assert out.tolist() == case["expected"]


# ---------------------------------------------------------------- numerics

def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 100000).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.4e38, 1e-40, np.inf, -np.inf], np.float32)])
    ours = oracle.bf16_bits_from_f32(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    # scalar C path agrees with the vectorised numpy path
    L = oracle.lib()
    for v in x[:2000]:
        assert L.or_bf16_from_f32(float(v)) == oracle.bf16_bits_from_f32(np.array([v]))[0]


def test_e4m3_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.f32_from_e4m3_bits(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.array_equal(np.signbit(ours[~nan]), np.signbit(ref[~nan]))
    assert nan.sum() == 2  # S.1111.111 only


def test_e4m3_encode_matches_torch_in_range_and_saturates():
    # every bf16 value (a superset of what the bf16 KV path feeds the quantiser)
    x = oracle.f32_from_bf16_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    L = oracle.lib()
    ours = np.array([L.or_e4m3_from_f32(float(v)) for v in x], dtype=np.uint8)
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    finite = np.isfinite(x)
    in_range = finite & (np.abs(x) <= 464.0)  # torch rounds these to <= 448
    assert np.array_equal(ours[in_range], ref[in_range])
    big = finite & (np.abs(x) > 464.0)  # torch overflows to NaN; the oracle saturates
    assert np.all((ours[big] & 0x7F) == 0x7E)
    assert np.all((ours[np.isinf(x)] & 0x7F) == 0x7E)
    nan = np.isnan(x)
    assert np.array_equal(ours[nan], ref[nan])
    # random f32 sweep near the e4m3 range
    rng = np.random.default_rng(2)
    y = (rng.standard_normal(20000) * 2.0 ** rng.integers(-12, 9, 20000)).astype(np.float32)
    y = y[np.abs(y) <= 464]
    o2 = np.array([L.or_e4m3_from_f32(float(v)) for v in y], dtype=np.uint8)
    r2 = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(o2, r2)


# ---------------------------------------------------------------- layout ops

def _tagged(T, H, D, salt=0):
    t, h, d = np.meshgrid(np.arange(T), np.arange(H), np.arange(D), indexing="ij")
    return (salt * 1e6 + t * 1000 + h * 100 + d).astype(np.float32)


@pytest.mark.parametrize("dtype", [oracle.F32, oracle.BF16])
def test_store_kv_layout_matches_c_order_indexing(dtype):
    NB, H, BS, D, T, start = 12, 3, 16, 8, 37, 5
    rng = np.random.default_rng(3)
    block_ids = rng.permutation(NB)[: (start + T + BS - 1) // BS]
    k, v = _tagged(T, H, D, 1), _tagged(T, H, D, 2)
    if dtype == oracle.BF16:
        k, v = oracle.bf16_bits_from_f32(k).reshape(T, H, D), oracle.bf16_bits_from_f32(v).reshape(T, H, D)
    kp = np.zeros((NB, H, BS, D), k.dtype)
    vp = np.zeros((NB, H, BS, D), k.dtype)
    assert oracle.store_kv(kp, vp, dtype, k, v, block_ids, start, T, H, D, BS) == 0
    for t in range(T):
        g = start + t
        blk, tib = block_ids[g // BS], g % BS
        assert np.array_equal(kp[blk, :, tib, :], k[t])
        assert np.array_equal(vp[blk, :, tib, :], v[t])
    # nothing else was written
    written = np.zeros((NB, BS), bool)
    for t in range(T):
        written[block_ids[(start + t) // BS], (start + t) % BS] = True
    assert np.all(kp.transpose(0, 2, 1, 3)[~written] == 0)


def test_store_kv_oob_is_an_error():
    kp = np.zeros((4, 1, 16, 4), np.float32)
    k = np.ones((20, 1, 4), np.float32)
    # two tokens past the single block: kv_cache.rs:234-239
    assert oracle.store_kv(kp, kp.copy(), oracle.F32, k, k, [2], 0, 20, 1, 4, 16) == -1


@pytest.mark.parametrize("threads", [1, 4])
def test_store_kv_batch_is_store_kv_per_sequence(threads):
    """The CPU baseline's append leg: the batched driver equals one
    store_kv per sequence (index-tagged payloads, disjoint random blocks), on
    one thread and on OpenMP threads; a sequence short of blocks fails."""
    NB, H, BS, D = 64, 3, 16, 8
    rng = np.random.default_rng(7)
    starts, ns = [3, 17, 0, 40], [20, 33, 16, 9]
    perm = rng.permutation(NB)
    lists, o = [], 0
    for s, n in zip(starts, ns):
        nblk = (s + n + BS - 1) // BS
        lists.append(perm[o:o + nblk])
        o += nblk
    k = oracle.bf16_bits_from_f32(_tagged(sum(ns), H, D, 5)).reshape(sum(ns), H, D)
    v = oracle.bf16_bits_from_f32(_tagged(sum(ns), H, D, 6)).reshape(sum(ns), H, D)
    kp1, vp1 = np.zeros((NB, H, BS, D), np.uint16), np.zeros((NB, H, BS, D), np.uint16)
    row = 0
    for b, s, n in zip(lists, starts, ns):
        assert oracle.store_kv(kp1, vp1, oracle.BF16, k[row:row + n], v[row:row + n], b, s, n, H, D, BS) == 0
        row += n
    kp2, vp2 = np.zeros_like(kp1), np.zeros_like(vp1)
    assert oracle.store_kv_batch(kp2, vp2, oracle.BF16, k, v, lists, starts, ns, H, D, BS, threads) == 0
    assert np.array_equal(kp1, kp2) and np.array_equal(vp1, vp2)
    assert np.count_nonzero(kp2) == np.count_nonzero(k)
    short = [lists[0], lists[1][:1], lists[2], lists[3]]
    assert oracle.store_kv_batch(kp2, vp2, oracle.BF16, k, v, short, starts, ns, H, D, BS, threads) == -1


def test_append_slots_equals_store_kv_and_skips_negative():
    NB, H, BS, D, T, start = 10, 2, 16, 16, 40, 3
    ids = np.array([7, 2, 5, 9])
    k, v = _tagged(T, H, D, 3), _tagged(T, H, D, 4)
    kp1, vp1 = np.zeros((NB, H, BS, D), np.float32), np.zeros((NB, H, BS, D), np.float32)
    oracle.store_kv(kp1, vp1, oracle.F32, k, v, ids, start, T, H, D, BS)
    g = start + np.arange(T)
    slots = ids[g // BS] * BS + g % BS
    kp2, vp2 = np.zeros_like(kp1), np.zeros_like(vp1)
    oracle.append_slots(kp2, vp2, oracle.F32, k, v, oracle.F32, slots, H, D, BS, NB)
    assert np.array_equal(kp1, kp2) and np.array_equal(vp1, vp2)
    slots2 = slots.copy()
    slots2[::2] = -1
    kp3 = np.zeros_like(kp1)
    oracle.append_slots(kp3, kp3.copy(), oracle.F32, k, v, oracle.F32, slots2, H, D, BS, NB)
    assert np.count_nonzero(kp3) == np.count_nonzero(k[1::2])


def test_gather_roundtrip_and_sentinel():
    NB, H, BS, D, T = 16, 4, 16, 8, 70
    rng = np.random.default_rng(4)
    table = rng.permutation(NB)[:5].astype(np.int32)
    k = _tagged(T, H, D, 5)
    kp = np.zeros((NB, H, BS, D), np.float32)
    oracle.store_kv(kp, kp.copy(), oracle.F32, k, k, table.astype(np.int64), 0, T, H, D, BS)
    back = oracle.gather(kp, oracle.F32, table, T, H, D, BS, np.float32)
    assert np.array_equal(back, k)
    t2 = table.copy()
    t2[2] = -1  # walk stops at the sentinel (paged_attention.cu:66-67)
    part = oracle.gather(kp, oracle.F32, t2, T, H, D, BS, np.float32)
    assert part.shape[0] == 2 * BS and np.array_equal(part, k[: 2 * BS])


def test_copy_blocks_bytes_and_canary():
    rng = np.random.default_rng(5)
    pools = [rng.integers(0, 255, size=(8, 2, 16, 4), dtype=np.uint8) for _ in range(4)]
    before = [p.copy() for p in pools]
    oracle.copy_blocks(pools, 2 * 16 * 4, [1, 6], [3, 0])
    for p, b in zip(pools, before):
        assert np.array_equal(p[3], b[1]) and np.array_equal(p[0], b[6])
        for blk in (1, 2, 4, 5, 6, 7):
            assert np.array_equal(p[blk], b[blk])


# ---------------------------------------------------------------- decode

def _paged_case(rng, N, H, Hkv, D, BS, lens, NB=None, dtype=oracle.F32):
    pages = [(L + BS - 1) // BS for L in lens]
    NB = NB or sum(pages) + 3
    perm = rng.permutation(NB)
    mb = max(max(pages), 1)
    bt = -np.ones((N, mb), np.int32)
    o = 0
    for n, p in enumerate(pages):
        bt[n, :p] = perm[o:o + p]
        o += p
    kp = rng.standard_normal((NB, Hkv, BS, D)).astype(np.float32)
    vp = rng.standard_normal((NB, Hkv, BS, D)).astype(np.float32)
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    return q, kp, vp, bt


def _dense(kp, bt_row, L, BS):
    """[L, Hkv, D] context of one sequence, with numpy indexing."""
    return np.concatenate([kp[b] for b in bt_row[: (L + BS - 1) // BS]], axis=1).transpose(1, 0, 2)[:L]


def _sdpa_ref(q, kp, vp, bt, lens, BS, scale, mapping):
    N, H, D = q.shape
    Hkv = kp.shape[1]
    out = np.zeros((N, H, D))
    for n in range(N):
        L = lens[n]
        if L == 0:
            continue
        K = torch.from_numpy(_dense(kp, bt[n], L, BS)).double()  # [L, Hkv, D]
        V = torch.from_numpy(_dense(vp, bt[n], L, BS)).double()
        heads = np.arange(H)
        kvh = heads // (H // Hkv) if mapping == oracle.GROUPED else heads % Hkv
        Kh = K[:, kvh, :].permute(1, 0, 2)  # [H, L, D]
        Vh = V[:, kvh, :].permute(1, 0, 2)
        Q = torch.from_numpy(q[n]).double()[:, None, :]
        o = torch.nn.functional.scaled_dot_product_attention(Q, Kh, Vh, scale=scale)
        out[n] = o[:, 0, :].numpy()
    return out


@pytest.mark.parametrize("mapping", [oracle.GROUPED, oracle.MODULO])
@pytest.mark.parametrize("H,Hkv,D", [(4, 4, 32), (8, 2, 16), (32, 8, 128)])
def test_decode_matches_torch_sdpa_float64(mapping, H, Hkv, D):
    rng = np.random.default_rng(6 + H + D)
    lens = [1, 15, 16, 17, 40, 0, 77]
    BS = 16
    q, kp, vp, bt = _paged_case(rng, len(lens), H, Hkv, D, BS, lens)
    scale = np.float32(1.0 / math.sqrt(D))
    out = oracle.paged_decode(q, kp, vp, oracle.F32, bt, lens, Hkv, D, BS, scale, mapping)
    ref = _sdpa_ref(q, kp, vp, bt, lens, BS, float(scale), mapping)
    assert np.max(np.abs(out - ref)) < 2e-6
    assert np.all(out[5] == 0)  # empty context -> zero row


def test_decode_gqa_modulo_equals_reference_cpu_path():
    """MODULO mapping == repeat_interleave_kv + CpuAttention last row (model_runner_cpu.rs:230-250)."""
    rng = np.random.default_rng(7)
    H, Hkv, D, BS, L = 4, 2, 8, 16, 21
    q, kp, vp, bt = _paged_case(rng, 1, H, Hkv, D, BS, [L])
    K = _dense(kp, bt[0], L, BS).reshape(L, Hkv * D)
    V = _dense(vp, bt[0], L, BS).reshape(L, Hkv * D)
    Kx = oracle.repeat_interleave_kv(K, Hkv, H, L, D).reshape(H, L, D)
    Vx = oracle.repeat_interleave_kv(V, Hkv, H, L, D).reshape(H, L, D)
    Q = np.zeros((H, L, D), np.float32)
    Q[:, L - 1, :] = q[0]  # non-causal rows are independent; only the last row is read
    dense = oracle.cpu_attention(Q, Kx, Vx, 1, H, D, L).reshape(H, L, D)[:, L - 1, :]
    out = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [L], Hkv, D, BS,
                              np.float32(1 / math.sqrt(D)), oracle.MODULO)
    assert np.max(np.abs(out[0] - dense)) < 1e-6


def test_decode_closed_forms():
    rng = np.random.default_rng(8)
    H, Hkv, D, BS = 4, 2, 16, 16
    scale = np.float32(0.25)
    # ctx = 1: O = v0 exactly
    q, kp, vp, bt = _paged_case(rng, 1, H, Hkv, D, BS, [1])
    out = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [1], Hkv, D, BS, scale)
    for h in range(H):
        assert np.array_equal(out[0, h], vp[bt[0, 0], h // 2, 0])
    # constant K: uniform weights, O = mean(V)
    L = 37
    q, kp, vp, bt = _paged_case(rng, 1, H, Hkv, D, BS, [L])
    kp[:] = 0.5
    out = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [L], Hkv, D, BS, scale)
    Vd = _dense(vp, bt[0], L, BS)
    for h in range(H):
        assert np.max(np.abs(out[0, h] - Vd[:, h // 2].mean(0))) < 1e-6
    # one dominant score: O ~= v_argmax
    q, kp, vp, bt = _paged_case(rng, 1, H, Hkv, D, BS, [L])
    Kd = _dense(kp, bt[0], L, BS)
    j = 23
    blk, t = bt[0, j // BS], j % BS
    kp[blk, :, t, :] = 40.0 * np.sign(q[0, ::2]) if H // Hkv == 2 else kp[blk, :, t, :]
    out = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [L], Hkv, D, BS, np.float32(1.0))
    for h in range(0, H, 2):
        assert np.max(np.abs(out[0, h] - vp[blk, h // 2, t])) < 1e-4
    # shift invariance: adding u with q.u = c to every key leaves O unchanged
    q, kp, vp, bt = _paged_case(rng, 1, 1, 1, D, BS, [L])
    u = rng.standard_normal(D).astype(np.float32)
    u -= (u @ q[0, 0]) / (q[0, 0] @ q[0, 0]) * q[0, 0]  # q.u = 0 -> scores unchanged up to rounding
    base = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [L], 1, D, BS, scale)
    kp2 = kp + u
    shifted = oracle.paged_decode(q, kp2, vp, oracle.F32, bt, [L], 1, D, BS, scale)
    assert np.max(np.abs(base - shifted)) < 1e-5


def test_decode_sentinel_truncates_context():
    rng = np.random.default_rng(9)
    H, Hkv, D, BS = 2, 1, 8, 16
    q, kp, vp, bt = _paged_case(rng, 1, H, Hkv, D, BS, [50])
    full = oracle.paged_decode(q, kp, vp, oracle.F32, bt, [32], Hkv, D, BS, np.float32(0.3))
    bt2 = bt.copy()
    bt2[0, 2] = -1
    cut = oracle.paged_decode(q, kp, vp, oracle.F32, bt2, [50], Hkv, D, BS, np.float32(0.3))
    assert np.array_equal(full, cut)


def test_fp8_scales_and_quantised_append():
    rng = np.random.default_rng(10)
    H, D, BS, NB = 2, 16, 16, 6
    x = (rng.standard_normal((30, H, D)) * 3).astype(np.float32)
    cu = np.array([0, 12, 30])
    sc = oracle.fp8_scales(x, oracle.F32, cu, H, D)
    for n in range(2):
        for h in range(H):
            amax = np.abs(x[cu[n]:cu[n + 1], h]).max()
            assert sc[n, h] == np.float32(amax) / np.float32(448.0)
    slots = np.arange(30) + 16
    row = np.repeat([0, 1], [12, 18]).astype(np.int32)
    kp = np.zeros((NB, H, BS, D), np.uint8)
    vp = np.zeros_like(kp)
    oracle.append_slots(kp, vp, oracle.FP8, x, x, oracle.F32, slots, H, D, BS, NB, sc, sc, row)
    deq = oracle.f32_from_e4m3_bits(kp)
    for t in range(30):
        s = slots[t]
        blk, tib = s // BS, s % BS
        got = deq[blk, :, tib, :] * sc[row[t]][:, None]
        # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 of the value (plus subnormal floor)
        err = np.abs(got - x[t])
        assert np.all(err <= np.abs(x[t]) * 2 ** -4 + sc[row[t]][:, None] * 2 ** -10 + 1e-12)
        # the amax element maps to exactly +-448
    assert np.any(np.abs(deq) == 448.0)


# ------------------------------------------------------------ chunked prefill

def _prefill_case(rng, H, Hkv, D, BS, starts, chunks):
    """Pages holding each sequence's start + chunk tokens; q for the chunk rows."""
    lens = [s + c for s, c in zip(starts, chunks)]
    _, kp, vp, bt = _paged_case(rng, len(lens), H, Hkv, D, BS, lens)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int64)
    q = rng.standard_normal((int(cu[-1]), H, D)).astype(np.float32)
    return q, kp, vp, bt, cu, lens


@pytest.mark.parametrize("mapping", [oracle.GROUPED, oracle.MODULO])
@pytest.mark.parametrize("H,Hkv,D", [(4, 4, 32), (8, 2, 16), (32, 8, 64)])
def test_prefill_causal_matches_torch_sdpa_float64(mapping, H, Hkv, D):
    """Row t of a chunk after `start` cached tokens sees positions [0, start + t]:
    torch SDPA in float64 with that explicit mask (an independent routine)."""
    rng = np.random.default_rng(60 + H + D)
    BS = 16
    starts, chunks = [0, 5, 16, 33, 100], [7, 1, 16, 40, 19]
    q, kp, vp, bt, cu, lens = _prefill_case(rng, H, Hkv, D, BS, starts, chunks)
    scale = np.float32(1.0 / math.sqrt(D))
    out = oracle.paged_prefill(q, kp, vp, oracle.F32, bt, cu, starts, Hkv, D, BS, scale, True, mapping)
    heads = np.arange(H)
    kvh = heads // (H // Hkv) if mapping == oracle.GROUPED else heads % Hkv
    for n, (s, c) in enumerate(zip(starts, chunks)):
        L = s + c
        K = torch.from_numpy(_dense(kp, bt[n], L, BS)).double()[:, kvh, :].permute(1, 0, 2)  # [H, L, D]
        V = torch.from_numpy(_dense(vp, bt[n], L, BS)).double()[:, kvh, :].permute(1, 0, 2)
        Q = torch.from_numpy(q[cu[n]:cu[n + 1]]).double().permute(1, 0, 2)  # [H, c, D]
        mask = torch.arange(L)[None, :] <= (s + torch.arange(c))[:, None]  # [c, L]
        o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=float(scale))
        assert np.max(np.abs(out[cu[n]:cu[n + 1]] - o.permute(1, 0, 2).numpy())) < 2e-6, n


def test_prefill_rows_are_decodes():
    """A one-row chunk at position p is the decode of p + 1 tokens; a causal
    chunk's row t equals the decode of start + t + 1 tokens."""
    rng = np.random.default_rng(61)
    H, Hkv, D, BS = 8, 2, 32, 16
    starts, chunks = [0, 9, 31, 64], [1, 12, 1, 20]
    q, kp, vp, bt, cu, lens = _prefill_case(rng, H, Hkv, D, BS, starts, chunks)
    scale = np.float32(0.125)
    out = oracle.paged_prefill(q, kp, vp, oracle.F32, bt, cu, starts, Hkv, D, BS, scale, True)
    for n, (s, c) in enumerate(zip(starts, chunks)):
        for t in range(c):
            dec = oracle.paged_decode(q[cu[n] + t][None], kp, vp, oracle.F32, bt[n:n + 1], [s + t + 1],
                                      Hkv, D, BS, scale)
            assert np.array_equal(out[cu[n] + t], dec[0]), (n, t)


def test_prefill_noncausal_first_chunk_is_reference_cpu_attention():
    """Not causal, start 0: every row sees the whole chunk -- CpuAttention::forward
    (attention/mod.rs:64-98) on the gathered K/V, MHA."""
    rng = np.random.default_rng(62)
    H, D, BS, L = 4, 16, 16, 37
    q, kp, vp, bt, cu, lens = _prefill_case(rng, H, H, D, BS, [0], [L])
    out = oracle.paged_prefill(q, kp, vp, oracle.F32, bt, cu, [0], H, D, BS, np.float32(1 / math.sqrt(D)), False)
    K = np.ascontiguousarray(_dense(kp, bt[0], L, BS).transpose(1, 0, 2))  # [H, L, D]
    V = np.ascontiguousarray(_dense(vp, bt[0], L, BS).transpose(1, 0, 2))
    Q = np.ascontiguousarray(q.transpose(1, 0, 2))
    dense = oracle.cpu_attention(Q, K, V, 1, H, D, L).reshape(H, L, D).transpose(1, 0, 2)
    assert np.max(np.abs(out - dense)) < 1e-6


def test_prefill_closed_forms():
    """Causal row 0 of a first chunk is v_0; a chunk row after cached tokens with
    constant K is the mean of V over its visible positions."""
    rng = np.random.default_rng(63)
    H, Hkv, D, BS = 2, 1, 8, 16
    q, kp, vp, bt, cu, lens = _prefill_case(rng, H, Hkv, D, BS, [0, 10], [5, 6])
    kp[:] = 0.5  # constant K: uniform weights
    out = oracle.paged_prefill(q, kp, vp, oracle.F32, bt, cu, [0, 10], Hkv, D, BS, np.float32(0.3), True)
    V0 = _dense(vp, bt[0], 5, BS)
    V1 = _dense(vp, bt[1], 16, BS)
    for h in range(H):
        assert np.allclose(out[0, h], V0[0, 0], atol=1e-6)
        for t in range(6):
            assert np.allclose(out[5 + t, h], V1[: 10 + t + 1, 0].mean(axis=0), atol=1e-5)
