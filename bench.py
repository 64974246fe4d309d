"""Benchmark of the paged-KV hot path on one MI355X.

Headline (value): paged decode attention GB/s at the Llama-3-8B decode shape
(C2: 256 sequences, context U[512, 8192], 32 q-heads / 8 kv-heads, D=128,
bf16 KV, block_size 16).  A step is one batched decode pass over all 256
sequences; inputs are resident in HBM before the timed region.  The same run
also measures the chunked-prefill KV append (C3: 64 x 512 tokens at
non-aligned offsets, bf16), the fp8-KV decode (C5: 512 sequences, context
U[1024, 16384]) and prefix sharing with copy-on-write through the stateful
KVCache (C4: 16 prefixes x 2048+r tokens x 32 layers, 128 forks, 64 decode
steps), the causal chunked-prefill attention of C3's chunks, one layer of
a mixed runner step (252 decodes + 4 chunks through the KVCache) and a full
32-layer decode step of a Llama-3-8B-shaped model with the dense ops, and
reports them as extra fields.

Algorithmic bytes (unique bytes that must cross HBM):
  decode  sum(ctx) * 2 * Hkv * D * elt  + Q + O + block-table entries + seq_lens
  append  2 * T * Hkv * D * elt (read)  + the same (write) + T * 8 (int64 slots)
The roofline object is for the dominant kernel (decode_partials): its bytes
are the KV bytes + Q + table entries + seq_lens, divided by its mean launch
duration from the hipEvents the library records around each launch (on the
launch stream) during a second timed region of the same steps; `value` comes
from the first timed region, which has no per-kernel events.

cpu_baseline: the CPU oracle's faithful restatement of the reference CPU path
(oracle/zk_oracle.c) timed on this host, single-threaded and with OpenMP over
the CPUs this process may use: the scalar decode (src/attention/mod.rs:64-98
over the pages) on a bounded sample of C2 (the first 128 sequences' context
lengths; the top-level value) and the per-(token, head) memcpy append
(src/kv_cache.rs:229-274) over C3's whole workload (legs.append).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
SEED = 20261201
METRIC = "paged decode attn GB/s (% of HBM peak) + KV append GB/s, Llama-3-8B shape"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def paged_tables(rng, lens, bs, slack=0.10):
    pages = [(int(L) + bs - 1) // bs for L in lens]
    nb = int(math.ceil(sum(pages) * (1 + slack))) + 1
    perm = rng.permutation(nb).astype(np.int32)
    bt = -np.ones((len(lens), max(pages)), np.int32)
    o = 0
    for n, p in enumerate(pages):
        bt[n, :p] = perm[o:o + p]
        o += p
    return bt, nb, sum(pages)


def timed(fn, steps, warmup, torch):
    """Runs fn warmup times, then times exactly `steps` calls with events on the
    current stream, bracketed by synchronize() on both sides. Returns ms/step."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(steps):
        fn(i)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def median_step_ms(fn, n, torch):
    """Median (and spread) of n individually event-timed steps on the current
    stream: the per-iteration protocol (>= 50 iterations, median) beside the
    contract's mean over the K bracketed steps."""
    s = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(ev):
        a.record(s)
        fn(i)
        b.record(s)
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) for a, b in ev])
    return {"median_ms": float(np.median(t)), "p10_ms": float(np.percentile(t, 10)),
            "p90_ms": float(np.percentile(t, 90)), "iterations": n}


def measured_traffic(key):
    """HBM bytes per launch of the workload's dominant kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/hbm_traffic.json, scaled
    by the stream-copy calibration recorded there); None if absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(key, {}).get("bytes")
    except (OSError, ValueError):
        return None


def kernel_ms(lib, name):
    import ctypes
    n = ctypes.c_int64()
    ms = ctypes.c_double()
    rc = lib.zk_timing_query(name.encode(), ctypes.byref(n), ctypes.byref(ms))
    assert rc == 0
    return (ms.value / n.value if n.value else float("nan")), n.value


# ---------------------------------------------------------------- C2 decode

def bench_decode(args, torch, ops, lib, kv="bf16"):
    if kv == "bf16":
        N, lo, hi = 256, 512, 8192
    else:
        N, lo, hi = 512, 1024, 16384
    H, Hkv, D, BS = 32, 8, 128, 16
    rng = np.random.default_rng(SEED + (0 if kv == "bf16" else 5))
    lens = rng.integers(lo, hi + 1, N)
    bt, nb, npages = paged_tables(rng, lens, BS)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(SEED)
    log(f"decode {kv}: N={N} sum_ctx={int(lens.sum())} blocks={nb}")
    q = torch.randn((N, H, D), generator=g, device=dev).to(torch.bfloat16)
    btd = torch.from_numpy(bt).to(dev)
    lensd = torch.from_numpy(lens.astype(np.int32)).to(dev)
    elt = 2 if kv == "bf16" else 1
    ks = vs = None
    if kv == "bf16":
        kp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
        vp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
    else:
        # quantise on append: bf16 N(0,1) K/V, per-(seq, head) amax scales
        kp = torch.zeros((nb, Hkv, BS, D), dtype=torch.uint8, device=dev)
        vp = torch.zeros_like(kp)
        ks = torch.empty((N, Hkv), dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        for n0 in range(0, N, 32):
            n1 = min(N, n0 + 32)
            L = lens[n0:n1]
            T = int(L.sum())
            kx = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
            vx = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
            cu = torch.from_numpy(np.concatenate([[0], np.cumsum(L)]).astype(np.int64)).to(dev)
            ks[n0:n1] = ops.fp8_scales(kx, cu)
            vs[n0:n1] = ops.fp8_scales(vx, cu)
            slots = np.concatenate([bt[n, np.arange(l) // BS].astype(np.int64) * BS + np.arange(l) % BS
                                    for n, l in zip(range(n0, n1), L)])
            rows = np.repeat(np.arange(n0, n1), L).astype(np.int32)
            ops.append(kp, vp, kx, vx, torch.from_numpy(slots).to(dev), k_scales=ks, v_scales=vs,
                       token_row=torch.from_numpy(rows).to(dev))
            del kx, vx
        torch.cuda.synchronize()
    out = torch.empty_like(q)
    ws = torch.empty(ops.decode_workspace_bytes(N, H, D, bt.shape[1], BS), dtype=torch.uint8, device=dev)

    def step(_):
        ops.paged_decode(q, kp, vp, btd, lensd, k_scales=ks, v_scales=vs, out=out, workspace=ws)

    ms = timed(step, args.steps, args.warmup, torch)
    per_iter = median_step_ms(step, max(50, args.steps), torch)
    # second timed region with the library's per-kernel hipEvents on the same stream
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    ms_ev = timed(step, args.steps, 0, torch)
    # read yardstick over the same pools: the practical ceiling of this read-bound kernel
    import ctypes
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    pool_bytes = kp.numel() * kp.element_size()

    def read_pools(_):
        for t in (kp, vp):
            lib.zk_stream_read(ctypes.c_void_p(t.data_ptr()), pool_bytes, ctypes.c_void_p(sink.data_ptr()), None)

    timed(read_pools, args.steps, 2, torch)
    rd_ms, rd_n = kernel_ms(lib, "stream_read")
    read_gbps = pool_bytes / (rd_ms * 1e-3) / 1e9
    lib.zk_timing_enable(0)
    k_ms, k_n = kernel_ms(lib, "decode_partials")
    p_ms, _ = kernel_ms(lib, "decode_plan")
    r_ms, _ = kernel_ms(lib, "decode_reduce")
    i_ms, _ = kernel_ms(lib, "decode_seq_info")
    lib.zk_timing_reset()
    sum_ctx = int(lens.sum())
    kv_bytes = sum_ctx * 2 * Hkv * D * elt
    q_bytes = N * H * D * 2
    small = npages * 4 + N * 4 + (2 * N * Hkv * 4 if kv != "bf16" else 0)
    alg = kv_bytes + 2 * q_bytes + small
    alg_kernel = kv_bytes + q_bytes + small
    gbps = alg / (ms * 1e-3) / 1e9
    kgbps = alg_kernel / (k_ms * 1e-3) / 1e9
    torch.cuda.synchronize()
    res = {
        "ms_per_step": ms, "gbps": gbps, "frac_of_peak": gbps / PEAK_HBM_GBPS,
        "new_tokens_per_s": N / (ms * 1e-3), "context_tokens_per_s": sum_ctx / (ms * 1e-3),
        "algorithmic_bytes": alg, "sum_ctx": sum_ctx, "num_seqs": N,
        "kernel_ms": {"decode_partials": k_ms, "decode_reduce": r_ms, "decode_seq_info": i_ms,
                      "decode_plan": p_ms},
        "ms_per_step_with_kernel_events": ms_ev,
        "per_iteration": per_iter, "gbps_at_median": alg / (per_iter["median_ms"] * 1e-3) / 1e9,
        "read_ceiling_gbps": read_gbps,
        "kernel_frac_of_read_ceiling": (alg_kernel / (k_ms * 1e-3) / 1e9) / read_gbps,
        "roofline": {"bound": "hbm", "achieved": kgbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": kgbps / PEAK_HBM_GBPS, "traffic": measured_traffic(f"decode_{kv}"),
                     "kernel": "decode_partials", "kernel_bytes_per_launch": alg_kernel,
                     "launches": k_n, "traffic_source": "profiles/hbm_traffic.json"},
    }
    del kp, vp, q, out, ws
    torch.cuda.empty_cache()
    return res, lens


# ---------------------------------------------------------------- C3 append

def bench_gather(args, torch, ops, lib):
    """Block-table gather (zk_gather) at C2's shape: every sequence's pages
    copied to contiguous [ctx, Hkv, D] K and V rows."""
    N, lo, hi = 256, 512, 8192
    H, Hkv, D, BS = 32, 8, 128, 16
    rng = np.random.default_rng(SEED)
    lens = rng.integers(lo, hi + 1, N)
    bt, nb, _ = paged_tables(rng, lens, BS)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(SEED)
    total = int(lens.sum())
    log(f"gather bf16: N={N} sum_ctx={total} blocks={nb}")
    kp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
    btd = torch.from_numpy(bt).to(dev)
    lensd = torch.from_numpy(lens.astype(np.int32)).to(dev)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    offd = torch.from_numpy(offs).to(dev)
    ko = torch.empty((total, Hkv, D), dtype=torch.bfloat16, device=dev)
    vo = torch.empty_like(ko)

    def step(_):
        ops.gather(kp, vp, btd, lensd, offd, ko, vo)

    ms = timed(step, args.steps, args.warmup, torch)
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    timed(step, args.steps, 0, torch)
    lib.zk_timing_enable(0)
    k_ms, _ = kernel_ms(lib, "gather")
    lib.zk_timing_reset()
    # spot check two sequences against torch indexing of the pools
    for n in (0, N - 1):
        L = int(lens[n])
        blocks = torch.from_numpy(bt[n, np.arange(L) // BS].astype(np.int64)).to(dev)
        tib = torch.from_numpy((np.arange(L) % BS).astype(np.int64)).to(dev)
        ref = kp[blocks, :, tib, :]
        assert torch.equal(ko[offs[n]: offs[n] + L], ref), "gather spot check"
    nbytes = 2 * 2 * total * Hkv * D * 2 + int(np.ceil(lens / BS).sum()) * 4  # K+V read and written, tables
    return {"ms_per_step": ms, "gbps": nbytes / (ms * 1e-3) / 1e9, "kernel_ms": k_ms,
            "kernel_gbps": nbytes / (k_ms * 1e-3) / 1e9, "algorithmic_bytes": nbytes, "sum_ctx": total,
            "num_seqs": N}


def bench_append(args, torch, ops, lib):
    Nseq, C, Hkv, D, BS = 64, 512, 8, 128, 16
    R = 4  # rotating buffer sets: 4 x 256 MiB moved > 256 MB Infinity Cache
    rng = np.random.default_rng(SEED + 1)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(SEED + 1)
    sets = []
    total_blocks = 0
    tables = []
    for r in range(R):
        starts = rng.integers(0, 4096, Nseq)
        starts[starts % BS == 0] += 1
        pages = [(int(s) + C + BS - 1) // BS for s in starts]
        tables.append((starts, pages, total_blocks))
        total_blocks += sum(pages)
    nb = int(total_blocks * 1.1) + 1
    perm = rng.permutation(nb)
    kp = torch.zeros((nb, Hkv, BS, D), dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    T = Nseq * C
    for starts, pages, base in tables:
        blocks = perm[base: base + sum(pages)]
        o = 0
        slots = []
        for s, p in zip(starts, pages):
            row = blocks[o:o + p]
            o += p
            gpos = int(s) + np.arange(C)
            slots.append(row[gpos // BS].astype(np.int64) * BS + gpos % BS)
        k = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
        sets.append((k, v, torch.from_numpy(np.concatenate(slots)).to(dev)))
    log(f"append bf16: T={T} rotating sets={R} pool blocks={nb}")

    def step(i):
        k, v, s = sets[i % R]
        ops.append(kp, vp, k, v, s)

    ms = timed(step, args.steps, args.warmup, torch)
    per_iter = median_step_ms(step, max(50, args.steps), torch)
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    timed(step, args.steps, 0, torch)
    lib.zk_timing_enable(0)
    k_ms, k_n = kernel_ms(lib, "append")
    lib.zk_timing_reset()
    alg = 2 * (2 * T * Hkv * D * 2) + T * 8
    gbps = alg / (ms * 1e-3) / 1e9
    # One step is exactly one append_copy_kernel launch, so the event-bracketed
    # steps of the first timed region time the kernel itself; the per-launch
    # event pairs of the second region add their own overhead to a ~50 us kernel.
    kgbps = gbps
    # in-repo streaming copy of the same byte count, as the attainable yardstick
    nbytes = 2 * T * Hkv * D * 2
    a = torch.empty(nbytes * R, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    import ctypes

    def cp(i):
        off = (i % R) * nbytes
        lib.zk_stream_copy(ctypes.c_void_p(b.data_ptr() + off), ctypes.c_void_p(a.data_ptr() + off),
                           nbytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    cms = timed(cp, args.steps, args.warmup, torch)
    copy_gbps = 2 * nbytes / (cms * 1e-3) / 1e9
    res = {"ms_per_step": ms, "gbps": gbps, "frac_of_peak": gbps / PEAK_HBM_GBPS,
           "tokens_per_s": T / (ms * 1e-3), "algorithmic_bytes": alg,
           "per_iteration": per_iter, "gbps_at_median": alg / (per_iter["median_ms"] * 1e-3) / 1e9,
           "stream_copy_gbps": copy_gbps, "frac_of_stream_copy": gbps / copy_gbps,
           "roofline": {"bound": "hbm", "achieved": kgbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                        "frac": kgbps / PEAK_HBM_GBPS, "traffic": measured_traffic("append_bf16"),
                        "kernel": "append", "launches": args.steps,
                        "traffic_source": "profiles/hbm_traffic.json",
                        "per_launch_event_ms": k_ms, "per_launch_event_launches": k_n}}
    del sets, kp, vp, a, b
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------- C4 prefix CoW

def bench_c4(args, torch, lib):
    """Prefix sharing with copy-on-write through the stateful KVCache: 16
    prefixes of 2048 + r tokens (r in [1, 15], so the tail block is partial)
    over 32 bf16 layers, 8 forks each; the forks' first append copies their
    shared tail (one batched copy over all 64 pools), then decode steps of
    (append_kv_batch + paged_decode) per layer for all 128 forks."""
    import zealot_amd as ze
    from zealot_amd.kv_cache import KVCache, SeqBatch
    P, F, L, H, Hkv, D, BS = 16, 8, 32, 32, 8, 128, 16
    STEPS, EV_STEPS, COW_REPS = 64, 8, 5
    rng = np.random.default_rng(SEED + 4)
    plen = 2048 + rng.integers(1, BS, P)
    grow = 1 + STEPS + EV_STEPS
    MB = (int(plen.max()) + grow + BS - 1) // BS + 1
    NB = sum((int(x) + BS - 1) // BS for x in plen) + P * F * ((BS - 1 + grow + BS - 1) // BS + 1) + 64
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(SEED + 4)
    bm = ze.BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=P * (F + 1), max_blocks_per_seq=MB)
    log(f"c4: prefixes={P} x {int(plen.min())}..{int(plen.max())} tokens, layers={L}, forks={P * F}, pool blocks={NB}")
    for p in range(P):
        pid = f"p{p}"
        cache.register_seq(pid, MB)
        for _ in range((int(plen[p]) + BS - 1) // BS):
            cache.alloc_block(pid, bm)
        for layer in range(L):
            k = torch.randn((int(plen[p]), Hkv, D), generator=g, device=dev).to(torch.bfloat16)
            v = torch.randn((int(plen[p]), Hkv, D), generator=g, device=dev).to(torch.bfloat16)
            cache.store_kv(layer, pid, k, v, 0, int(plen[p]))
    torch.cuda.synchronize()
    children = [f"p{p}.f{j}" for p in range(P) for j in range(F)]
    parent = [p for p in range(P) for _ in range(F)]
    batch = SeqBatch(children)
    n = len(children)
    R = 4
    kin = [torch.randn((n, Hkv, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(R)]
    vin = [torch.randn((n, Hkv, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(R)]
    qin = [torch.randn((n, H, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(R)]
    out = torch.empty((n, H, D), dtype=torch.bfloat16, device=dev)
    # copy-on-write: fork every prefix, then the first append copies each tail
    cow_kernel_ms, cow_call_ms = [], []
    for rep in range(COW_REPS):
        for cid, p in zip(children, parent):
            cache.fork_seq(f"p{p}", cid)
        torch.cuda.synchronize()
        lib.zk_timing_reset()
        lib.zk_timing_enable(1)
        t0 = time.perf_counter()
        cache.append_kv_batch(0, batch, kin[0], vin[0])
        torch.cuda.synchronize()
        cow_call_ms.append((time.perf_counter() - t0) * 1e3)
        lib.zk_timing_enable(0)
        c_ms, c_n = kernel_ms(lib, "copy_blocks")
        assert c_n == 1, c_n
        cow_kernel_ms.append(c_ms)
        if rep + 1 < COW_REPS:
            for cid in children:
                cache.release_seq(cid)
    lib.zk_timing_reset()
    # logical bytes: every fork's tail read and written in every pool; HBM
    # bytes: each prefix's shared tail read once (its 8 forks copy the same
    # block) and every copy written
    block_bytes = BS * Hkv * D * 2
    cow_logical = 2 * n * 2 * L * block_bytes
    cow_hbm = (P + n) * 2 * L * block_bytes
    cow_ms = float(np.median(cow_kernel_ms))
    pos = [int(plen[p]) for p in parent]  # next token position of each fork
    nblk = [(x + BS - 1) // BS for x in pos]

    def step(_):
        for i, cid in enumerate(children):
            if pos[i] == nblk[i] * BS:
                cache.alloc_block(cid, bm)
                nblk[i] += 1
        for layer in range(L):  # append + decode of the layer, one launch (zk_cache_decode_append)
            cache.decode_append(layer, batch, kin[layer % R], vin[layer % R], qin[layer % R], out=out)
        for i in range(n):
            pos[i] += 1

    step(0)  # warm-up step (its layer-0 append rewrites the CoW step's token)
    torch.cuda.synchronize()
    ctx0 = np.array(pos, np.int64)
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    for i in range(STEPS):
        step(i)
    e1.record(s)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / STEPS
    share_sg, share_pages = cache.decode_sharing()
    ms = e0.elapsed_time(e1) / STEPS
    # decode lengths of the timed steps: ctx0 + s + 1 at every layer of step s
    tok_per_layer = 2 * Hkv * D * 2
    logical_ctx = sum(int((ctx0 + i + 1).sum()) for i in range(STEPS)) / STEPS
    shared = P * (2048 // BS) * BS  # full prefix blocks, shared by 8 forks each
    unique_ctx = shared + sum(int((ctx0 + i + 1).sum()) - P * F * 2048 for i in range(STEPS)) / STEPS
    logical_bytes = logical_ctx * tok_per_layer * L
    unique_bytes = unique_ctx * tok_per_layer * L
    append_bytes = 2 * n * tok_per_layer * L + n * 8 * L
    # per-kernel times from a few more steps with the library's hipEvents
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    for i in range(EV_STEPS):
        step(i)
    torch.cuda.synchronize()
    lib.zk_timing_enable(0)
    kt = {k: kernel_ms(lib, k) for k in ("decode_partials", "decode_reduce", "decode_seq_info",
                                         "decode_plan", "append")}
    lib.zk_timing_reset()
    dec_kernel_ms = sum(kt[k][0] * kt[k][1] for k in ("decode_partials", "decode_reduce", "decode_seq_info",
                                                      "decode_plan") if kt[k][1]) / EV_STEPS
    # released handles are stale: a freed block's old handle is rejected
    h = bm.allocate()
    bm.free(h)
    try:
        bm.reference(h)
        stale_rejected = False
    except RuntimeError as e:
        stale_rejected = "Stale handle" in str(e)
    for cid in children:
        cache.release_seq(cid)
    for p in range(P):
        cache.release_seq(f"p{p}")
    assert bm.free_blocks == NB
    res = {
        "cow": {"forks": n, "pools": 2 * L, "hbm_bytes": cow_hbm, "kernel_ms": cow_ms,
                "gbps": cow_hbm / (cow_ms * 1e-3) / 1e9, "frac_of_peak": cow_hbm / (cow_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                "logical_bytes": cow_logical, "logical_gbps": cow_logical / (cow_ms * 1e-3) / 1e9,
                "traffic": measured_traffic("cow_c4"),
                "first_append_call_ms": float(np.median(cow_call_ms)), "reps": COW_REPS},
        "decode_step": {"steps": STEPS, "ms_per_step": ms, "wall_ms_per_step": wall_ms,
                        "layers": L, "seqs": n,
                        "logical_ctx_per_layer": logical_ctx, "unique_ctx_per_layer": unique_ctx,
                        "logical_bytes_per_step": logical_bytes, "unique_bytes_per_step": unique_bytes,
                        "append_bytes_per_step": append_bytes,
                        "logical_gbps": logical_bytes / (ms * 1e-3) / 1e9,
                        "unique_gbps": (unique_bytes + append_bytes) / (ms * 1e-3) / 1e9,
                        "tokens_per_s": n / (ms * 1e-3),
                        "decode_kernels_ms_per_step": dec_kernel_ms,
                        "decode_kernel_logical_gbps": logical_bytes / (dec_kernel_ms * 1e-3) / 1e9,
                        "decode_kernel_unique_gbps": unique_bytes / (dec_kernel_ms * 1e-3) / 1e9,
                        "kernel_ms": {k: v[0] for k, v in kt.items() if v[1]},
                        "prefix_subgroups": share_sg, "shared_pages_per_layer_kv_head": share_pages},
        "stale_handle_rejected": stale_rejected,
    }
    del cache, kin, vin, qin, out
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------- prefill attention

PEAK_BF16_TFLOPS = 2500.0


def bench_prefill(args, torch, ops, lib):
    """Causal chunked-prefill attention of C3's chunks: 64 sequences x 512 new
    tokens at unaligned offsets < 4096 (their K/V already in the pages), 32/8
    heads, D = 128, bf16.  Compute-bound: 4 * D flops per (query row, head,
    visible key)."""
    N, C, H, Hkv, D, BS = 64, 512, 32, 8, 128, 16
    rng = np.random.default_rng(SEED + 1)
    starts = rng.integers(0, 4096, N)
    starts[starts % BS == 0] += 1
    lens = starts + C
    bt, nb, _ = paged_tables(rng, lens, BS)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(SEED + 6)
    kp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn((nb, Hkv, BS, D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((N * C, H, D), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    btd = torch.from_numpy(bt).to(dev)
    cu = torch.arange(0, N * C + 1, C, dtype=torch.int64, device=dev)
    st = torch.from_numpy(starts.astype(np.int32)).to(dev)
    ws = torch.empty(ops.prefill_workspace_bytes(N, N * C, H, Hkv), dtype=torch.uint8, device=dev)
    log(f"prefill: N={N} chunk={C} context {int(lens.min())}..{int(lens.max())} blocks={nb}")

    def step(_):
        ops.paged_prefill(q, kp, vp, btd, cu, st, causal=True, out=out, workspace=ws)

    ms = timed(step, args.steps, args.warmup, torch)
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    timed(step, args.steps, 0, torch)
    lib.zk_timing_enable(0)
    k_ms, k_n = kernel_ms(lib, "prefill_attention")
    p_ms, _ = kernel_ms(lib, "prefill_plan")
    lib.zk_timing_reset()
    keys = int(sum(int(s) * C + C * (C + 1) // 2 for s in starts))  # visible keys over all rows
    flops = 4 * D * H * keys
    tflops = flops / (ms * 1e-3) / 1e12
    k_tflops = flops / (k_ms * 1e-3) / 1e12
    # K/V bytes the kernel streams into LDS: every item (128 query rows, the
    # two waves of a workgroup sharing each page) reads its pages once
    tq = 128 // (H // Hkv)
    kv_bytes = sum(((int(s) + min(C, (t + 1) * tq) + BS - 1) // BS) * BS * 2 * D * 2 * Hkv
                   for s in starts for t in range((C + tq - 1) // tq))
    res = {"ms_per_step": ms, "tflops": tflops, "frac_of_peak": tflops / PEAK_BF16_TFLOPS,
           "tokens_per_s": N * C / (ms * 1e-3), "flops": flops, "visible_keys": keys,
           "kernel_ms": {"prefill_attention": k_ms, "prefill_plan": p_ms},
           "kv_bytes_streamed": kv_bytes, "kv_gbps_streamed": kv_bytes / (k_ms * 1e-3) / 1e9,
           "roofline": {"bound": "mfma", "achieved": k_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": k_tflops / PEAK_BF16_TFLOPS, "traffic": None, "kernel": "prefill_attention",
                        "kernel_flops_per_launch": flops, "launches": k_n}}
    del kp, vp, q, out, ws
    torch.cuda.empty_cache()
    return res


def bench_mixed(args, torch, lib):
    """One layer of a runner step through the KVCache, as the scheduler hands
    it over: 252 decoding sequences (context U[512, 8192]) and 4 prompt chunks
    of 512 tokens (starts U[0, 4096)), 32/8 heads, D = 128, bf16.  Timed:
    zk_cache_write_batch + zk_cache_attention_batch for the whole batch (one
    append launch; the decode rows as one paged decode, the chunks as one
    chunked-prefill launch), beside the decode-only and chunk-only halves and
    the reference's per-sequence pattern (append_kv / store_kv + a one-sequence
    attention call each, cuda_runner.rs:274-461).  Layer 0 of a 2-layer cache is
    rewritten each step, so the work is the same every step."""
    from zealot_amd import BlockManager, KVCache
    from zealot_amd.kv_cache import SeqBatch
    ND, NC, C, H, Hkv, D, BS = 252, 4, 512, 32, 8, 128, 16
    rng = np.random.default_rng(SEED + 7)
    dec_ctx = rng.integers(512, 8193, ND)
    starts = rng.integers(0, 4096, NC)
    total = [int(x) for x in dec_ctx] + [int(s) + C for s in starts]
    pages = [(t + BS - 1) // BS for t in total]
    nb = sum(pages) + 16
    dev = torch.device("cuda", 0)
    bm = BlockManager(nb, BS)
    cache = KVCache(nb, BS, 2, Hkv, D, dtype=torch.bfloat16, max_seqs=ND + NC, max_blocks_per_seq=max(pages))
    ids = [f"d{i}" for i in range(ND)] + [f"c{i}" for i in range(NC)]
    for sid, p in zip(ids, pages):
        cache.register_seq(sid, p)
        for _ in range(p):
            cache.alloc_block(sid, bm)
    # fill both layers up to the tokens before the step (decode: ctx - 1, chunk: start)
    before = [int(x) - 1 for x in dec_ctx] + [int(s) for s in starts]
    g = torch.Generator(device=dev).manual_seed(SEED + 8)
    allb = SeqBatch(ids)
    T0 = sum(before)
    for layer in range(2):
        k = torch.randn((T0, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((T0, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
        cache.write_batch(layer, allb, before, k, v)
        del k, v
    nt = [1] * ND + [C] * NC
    T = sum(nt)
    k = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((T, Hkv, D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((T, H, D), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    decb, chb = SeqBatch(ids[:ND]), SeqBatch(ids[ND:])
    log(f"mixed: {ND} decodes + {NC} chunks of {C}; {nb} blocks")

    def mixed(_):
        cache.write_batch(0, allb, nt, k, v)
        cache.attention_batch(0, allb, nt, q, out=out)

    def dec_only(_):
        cache.write_batch(0, decb, nt[:ND], k[:ND], v[:ND])
        cache.attention_batch(0, decb, nt[:ND], q[:ND], out=out[:ND])

    def chunks_only(_):
        cache.write_batch(0, chb, nt[ND:], k[ND:], v[ND:])
        cache.attention_batch(0, chb, nt[ND:], q[ND:], out=out[ND:])

    def per_seq(_):  # the reference's loop: one sequence per call
        row = 0
        for i, sid in enumerate(ids):
            n = nt[i]
            if n == 1:
                cache.append_kv(0, sid, k[row:row + 1], v[row:row + 1])
            else:
                cache.store_kv(0, sid, k[row:row + n], v[row:row + n], before[i], n)
            cache.attention_batch(0, [sid], [n], q[row:row + n], out=out[row:row + n])
            row += n

    ms = timed(mixed, args.steps, args.warmup, torch)
    ms_dec = timed(dec_only, args.steps, args.warmup, torch)
    ms_ch = timed(chunks_only, args.steps, args.warmup, torch)
    ms_loop = timed(per_seq, max(2, args.steps // 10), 1, torch)
    kv_dec = sum(int(x) for x in dec_ctx) * 2 * Hkv * D * 2
    res = {"ms_per_step": ms, "decode_only_ms": ms_dec, "chunks_only_ms": ms_ch, "per_sequence_loop_ms": ms_loop,
           "speedup_vs_per_sequence_loop": ms_loop / ms, "tokens_per_step": T,
           "decode_kv_gbps_in_mixed_step": kv_dec / (ms * 1e-3) / 1e9,
           "shape": {"decodes": ND, "chunks": NC, "chunk": C, "num_heads": H, "num_kv_heads": Hkv, "head_dim": D}}
    del cache, k, v, q, out
    torch.cuda.empty_cache()
    return res


def bench_model(args, torch, lib):
    """One decode step of a Llama-3-8B-shaped model (32 layers, 32/8 heads,
    D = 128, hidden 4096, intermediate 14336, vocab 128256, bf16, random
    weights) for 64 sequences with contexts U[512, 8192], through
    HipModelRunner: embedding, per layer fused-add RMSNorm, the fused QKV /
    o / gate-up / down projections (hipBLASLt or the weight-streaming kernel,
    whichever the first call timed faster; gate|up, down and lm_head on tiled
    weights), SiLU*up in the gate|up epilogue, the KV write with the QKV
    split-k sums folded in and one paged decode for the batch, final norm and
    f32 lm_head logits.  Each
    step appends one token per sequence (contexts grow by the step count,
    < 1 %)."""
    import ctypes
    from zealot_amd import BlockManager, KVCache, PagedKVRunner
    from zealot_amd.kv_cache import SeqBatch
    from zealot_amd.model import HipModelRunner, LlamaConfig, LlamaWeights
    from zealot_amd.runner import StepPlan
    N, BS = 64, 16
    cfg = LlamaConfig.llama3_8b()
    rng = np.random.default_rng(SEED + 9)
    ctx = rng.integers(512, 8193, N)
    grow = args.warmup + args.steps + max(2, args.steps // 5) + 1
    pages = [(int(c) + grow + BS - 1) // BS for c in ctx]
    nb = sum(pages) + 16
    dev = torch.device("cuda", 0)
    bm = BlockManager(nb, BS)
    cache = KVCache(nb, BS, cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, dtype=torch.bfloat16, max_seqs=N,
                    max_blocks_per_seq=max(pages))
    ids = [f"s{i}" for i in range(N)]
    for sid, p in zip(ids, pages):
        cache.register_seq(sid, p)
        for _ in range(p):
            cache.alloc_block(sid, bm)
    g = torch.Generator(device=dev).manual_seed(SEED + 10)
    before = [int(c) - 1 for c in ctx]
    allb = SeqBatch(ids)
    T0 = sum(before)
    for layer in range(cfg.num_layers):  # context K/V (values do not matter for timing)
        kv = torch.randn((T0, cfg.num_kv_heads, cfg.head_dim), generator=g, device=dev).to(torch.bfloat16)
        cache.write_batch(layer, allb, before, kv, kv)
        del kv
    w = LlamaWeights.random(cfg, dtype=torch.bfloat16, seed=SEED + 11)
    model = HipModelRunner(cfg, w, PagedKVRunner(cache, bm))
    plan = StepPlan(allb, (ctypes.c_int32 * N)(*([1] * N)), before, N)
    tok = torch.randint(0, cfg.vocab_size, (N,), generator=g, device=dev)
    last = torch.arange(N, dtype=torch.int64, device=dev)
    log(f"model: Llama-3-8B shape, {N} seqs ctx {int(ctx.min())}..{int(ctx.max())}, {nb} blocks")

    def step(_):
        model.forward(plan, tok, last)

    ms = timed(step, args.steps, args.warmup, torch)
    prof_steps = max(2, args.steps // 5)
    lib.zk_timing_reset()
    lib.zk_timing_enable(1)
    timed(step, prof_steps, 0, torch)
    lib.zk_timing_enable(0)
    per = {}
    for nm in ("linear", "decode_partials", "decode_reduce", "decode_plan", "decode_seq_info", "append",
               "rms_norm", "silu_mul", "embedding"):
        k_ms, k_n = kernel_ms(lib, nm)
        if k_n:
            per[nm] = {"ms_per_step": k_ms * k_n / prof_steps, "launches_per_step": k_n / prof_steps}
    lib.zk_timing_reset()
    from zealot_amd import dense
    lw0 = w.layers[0]
    proj = {}
    for nm, t, od in (("qkv", lw0.qkv, None), ("o", lw0.o, None), ("gate_up", lw0.gate_up, None),
                      ("down", lw0.down, None), ("lm_head", w.lm_head, torch.float32)):
        tiled = isinstance(t, dense.TiledWeight)
        if nm == "gate_up" and tiled:  # no plan: always the one-launch SiLU kernel
            proj[nm] = {"tiled": True, "splits": 1, "tile_rows": 128, "silu_epilogue": True}
            continue
        try:
            proj[nm] = dict(dense.linear_choice(N, t.shape[0], t.shape[1], torch.bfloat16, od, tiled=tiled),
                            tiled=tiled)
        except Exception as e:  # no plan made for this shape
            proj[nm] = str(e)
    wbytes = sum(t.numel() * 2 for lw in w.layers for t in (lw.qkv, lw.o, lw.gate_up, lw.down)) + w.lm_head.numel() * 2
    kvbytes = int(sum(int(c) for c in ctx)) * cfg.num_layers * 2 * cfg.num_kv_heads * cfg.head_dim * 2
    res = {"ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3), "weight_bytes": wbytes, "kv_bytes": kvbytes,
           "gbps_weights_plus_kv": (wbytes + kvbytes) / (ms * 1e-3) / 1e9, "kernels": per,
           "projections": proj,
           "shape": {"model": "Llama-3-8B shape (random bf16 weights)", "layers": cfg.num_layers, "seqs": N,
                     "ctx": [int(ctx.min()), int(ctx.max())]}}
    del model, w, cache
    torch.cuda.empty_cache()
    return res


def bench_swap(args, torch, lib):
    """KV swap at C4's KV shape: 16 sequences x 2048 tokens x 32 layers (bf16,
    8 kv heads x 128) moved to pinned host slots and back (zk_cache_swap_out /
    zk_cache_swap_in: staging kernel + one DMA per run of host slots).  Bound
    by PCIe, not HBM: reported in GB/s of KV bytes moved per direction."""
    from zealot_amd import BlockManager, KVCache
    from zealot_amd.kv_cache import SeqBatch
    N, T, L, Hkv, D, BS = 16, 2048, 32, 8, 128, 16
    nblk = T // BS
    NB = N * nblk + 16
    bm = BlockManager(NB, BS)
    cache = KVCache(NB, BS, L, Hkv, D, dtype=torch.bfloat16, max_seqs=N, max_blocks_per_seq=nblk)
    cache.enable_swap(N * nblk)
    ids = [f"w{i}" for i in range(N)]
    for sid in ids:
        cache.register_seq(sid, nblk)
        for _ in range(nblk):
            cache.alloc_block(sid, bm)
    g = torch.Generator(device="cuda").manual_seed(SEED + 12)
    b = SeqBatch(ids)
    x = torch.randn((N * T, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    for layer in range(L):
        cache.write_batch(layer, b, [T] * N, x, x)
    del x
    nbytes = N * nblk * 2 * L * BS * Hkv * D * 2
    log(f"swap: {N} x {T} tokens x {L} layers = {nbytes / 1e9:.2f} GB per direction")
    outs, ins = [], []
    for it in range(args.warmup + max(3, args.steps // 10)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cache.swap_out(b)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        cache.swap_in(b, bm)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if it >= args.warmup:
            outs.append(t1 - t0)
            ins.append(t2 - t1)
    so, si = float(np.median(outs)), float(np.median(ins))
    res = {"bytes_per_direction": nbytes, "swap_out_ms": so * 1e3, "swap_in_ms": si * 1e3,
           "swap_out_gbps": nbytes / so / 1e9, "swap_in_gbps": nbytes / si / 1e9,
           "shape": {"seqs": N, "tokens": T, "layers": L, "kv_heads": Hkv, "head_dim": D, "dtype": "bf16"}}
    del cache
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------- CPU baseline

def host_cpu() -> dict:
    """Model string, family/model/stepping and the core counts of this host."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k in ("model name", "cpu family", "model", "stepping", "vendor_id") and k not in info:
                info[k] = v
            if len(info) == 5:
                break
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info["lscpu " + k.strip()] = v.strip()
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    info["os.cpu_count"] = os.cpu_count()
    info["affinity_cpus"] = len(os.sched_getaffinity(0))
    return info


def cpu_threads() -> int:
    """Threads for the OpenMP legs: the CPUs this process may run on."""
    return max(1, len(os.sched_getaffinity(0)))


def cpu_decode_leg(lens_all, sample_seqs, threads):
    """The oracle's scalar decode (attention/mod.rs:64-98 over the pages) on
    the first sample_seqs of the C2 context lengths."""
    import oracle
    H, Hkv, D, BS = 32, 8, 128, 16
    rng = np.random.default_rng(SEED + 2)
    lens = [int(x) for x in lens_all[:sample_seqs]]
    bt, nb, _ = paged_tables(rng, lens, BS)
    kp = oracle.bf16_bits_from_f32(rng.standard_normal((nb, Hkv, BS, D), dtype=np.float32)).reshape(nb, Hkv, BS, D)
    vp = oracle.bf16_bits_from_f32(rng.standard_normal((nb, Hkv, BS, D), dtype=np.float32)).reshape(nb, Hkv, BS, D)
    q = oracle.f32_from_bf16_bits(oracle.bf16_bits_from_f32(
        rng.standard_normal((len(lens), H, D), dtype=np.float32))).reshape(len(lens), H, D)
    scale = np.float32(1 / math.sqrt(D))
    alg = sum(lens) * 2 * Hkv * D * 2 + 2 * len(lens) * H * D * 2
    t0 = time.perf_counter()
    oracle.paged_decode(q, kp, vp, oracle.BF16, bt, lens, Hkv, D, BS, scale, threads=1)
    t1 = time.perf_counter() - t0
    t0 = time.perf_counter()
    oracle.paged_decode(q, kp, vp, oracle.BF16, bt, lens, Hkv, D, BS, scale, threads=threads)
    tn = time.perf_counter() - t0
    return {"value": alg / t1 / 1e9, "unit": "GB/s", "cores": 1, "seconds": t1,
            "omp_value": alg / tn / 1e9, "omp_cores": threads, "omp_seconds": tn,
            "sample": f"C2 decode, first {len(lens)} of the 256 context lengths (sum_ctx={sum(lens)}), bf16 KV, "
                      f"scalar fp32 loops of oracle/zk_oracle.c (or_paged_decode)"}


def cpu_append_leg(threads, reps):
    """The oracle's faithful store_kv (kv_cache.rs:229-274: one memcpy of D
    elements per (token, kv-head) for K and for V) over C3's whole workload:
    64 sequences x 512 tokens at unaligned starts, bf16, block tables drawn as
    in bench_append; median of `reps` passes."""
    import oracle
    Nseq, C, Hkv, D, BS = 64, 512, 8, 128, 16
    rng = np.random.default_rng(SEED + 1)
    starts = rng.integers(0, 4096, Nseq)
    starts[starts % BS == 0] += 1
    pages = [(int(st) + C + BS - 1) // BS for st in starts]
    nb = int(sum(pages) * 1.1) + 1
    perm = rng.permutation(nb)
    lists, o = [], 0
    for pg in pages:
        lists.append(perm[o:o + pg])
        o += pg
    T = Nseq * C
    k = rng.integers(0, 1 << 16, (T, Hkv, D), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, (T, Hkv, D), dtype=np.uint16)
    kp = np.zeros((nb, Hkv, BS, D), np.uint16)
    vp = np.zeros_like(kp)
    alg = 2 * (2 * T * Hkv * D * 2) + T * 8  # as the GPU leg: K+V read and written, slot per token
    res = {}
    for nthr in (1, threads):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            rc = oracle.store_kv_batch(kp, vp, oracle.BF16, k, v, lists, starts, [C] * Nseq, Hkv, D, BS, nthr)
            ts.append(time.perf_counter() - t0)
            assert rc == 0
        res[nthr] = float(np.median(ts))
    return {"value": alg / res[1] / 1e9, "unit": "GB/s", "cores": 1, "seconds_per_pass": res[1],
            "omp_value": alg / res[threads] / 1e9, "omp_cores": threads, "omp_seconds_per_pass": res[threads],
            "tokens_per_s": T / res[1],
            "sample": f"C3 append, the whole workload (64 x 512 tokens, bf16, 8 x 128), median of {reps} passes "
                      f"of oracle/zk_oracle.c or_store_kv (per-(token, head) memcpy), one call per sequence"}


def cpu_baseline(lens_all, sample_seqs, reps=20):
    threads = cpu_threads()
    dec = cpu_decode_leg(lens_all, sample_seqs, threads)
    app = cpu_append_leg(threads, reps)
    # the headline metric is the decode's GB/s, so the top-level figures are its leg
    return {"value": dec["value"], "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": dec["sample"] + f" ({dec['seconds']:.2f} s); append leg: " + app["sample"],
            "omp_value": dec["omp_value"], "omp_cores": threads,
            "legs": {"decode": dec, "append": app}, "host_cpu": host_cpu()}


# ---------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["decode", "gather", "append", "fp8", "c4", "prefill", "mixed", "model",
                                       "swap"],
                    default=None,
                    help="run one workload (for profiler passes)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-seqs", type=int, default=128)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode would shard by sequence / kv-head with no exchange)",
              file=sys.stderr)
        return 2
    import torch

    import zealot_amd
    from zealot_amd import ops
    lib = zealot_amd.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    result = {}
    dec = lens = gat = app = fp8 = c4 = pre = mix = mdl = swp = None
    if args.only in (None, "decode"):
        dec, lens = bench_decode(args, torch, ops, lib, "bf16")
        log(f"decode bf16: {dec['ms_per_step']:.4f} ms {dec['gbps']:.1f} GB/s")
    if args.only in (None, "gather"):
        gat = bench_gather(args, torch, ops, lib)
        log(f"gather bf16: {gat['ms_per_step']:.4f} ms {gat['gbps']:.1f} GB/s (kernel {gat['kernel_gbps']:.1f})")
    if args.only in (None, "append"):
        app = bench_append(args, torch, ops, lib)
        log(f"append bf16: {app['ms_per_step'] * 1e3:.2f} us {app['gbps']:.1f} GB/s")
    if args.only in (None, "fp8"):
        fp8, _ = bench_decode(args, torch, ops, lib, "fp8")
        log(f"decode fp8: {fp8['ms_per_step']:.4f} ms {fp8['gbps']:.1f} GB/s")
    if args.only in (None, "c4"):
        c4 = bench_c4(args, torch, lib)
        log(f"c4: cow {c4['cow']['gbps']:.1f} GB/s; step {c4['decode_step']['ms_per_step']:.3f} ms, "
            f"logical {c4['decode_step']['logical_gbps']:.1f} GB/s, unique {c4['decode_step']['unique_gbps']:.1f} GB/s")
    if args.only in (None, "prefill"):
        pre = bench_prefill(args, torch, ops, lib)
        log(f"prefill: {pre['ms_per_step']:.3f} ms {pre['tflops']:.1f} TFLOP/s "
            f"(kernel {pre['roofline']['achieved']:.1f} TFLOP/s)")
    if args.only in (None, "mixed"):
        mix = bench_mixed(args, torch, lib)
        log(f"mixed step: {mix['ms_per_step']:.3f} ms (decode-only {mix['decode_only_ms']:.3f}, chunks-only "
            f"{mix['chunks_only_ms']:.3f}, per-sequence loop {mix['per_sequence_loop_ms']:.2f})")
    if args.only in (None, "model"):
        mdl = bench_model(args, torch, lib)
        log(f"model decode step: {mdl['ms_per_step']:.3f} ms, {mdl['tokens_per_s']:.0f} tokens/s")
    if args.only in (None, "swap"):
        swp = bench_swap(args, torch, lib)
        log(f"swap: out {swp['swap_out_gbps']:.1f} GB/s, in {swp['swap_in_gbps']:.1f} GB/s")
    cpu = None
    if args.only is None and not args.no_cpu_baseline:
        cpu = cpu_baseline(lens, args.cpu_sample_seqs)
        a = cpu["legs"]["append"]
        log(f"cpu baseline: decode {cpu['value']:.3f} GB/s (1 core), {cpu['omp_value']:.2f} GB/s "
            f"({cpu['omp_cores']} cores); append {a['value']:.2f} GB/s (1 core), {a['omp_value']:.2f} GB/s")
    head = next((x for x in (dec, app, fp8) if x is not None), None)
    if head is None and gat is not None:  # --only gather
        head = {"gbps": gat["gbps"], "ms_per_step": gat["ms_per_step"], "roofline": None}
    if head is None and c4 is not None:  # --only c4
        head = {"gbps": c4["decode_step"]["logical_gbps"], "ms_per_step": c4["decode_step"]["ms_per_step"],
                "roofline": None}
    if head is None and pre is not None:  # --only prefill
        head = {"gbps": pre["tflops"], "ms_per_step": pre["ms_per_step"], "roofline": pre["roofline"]}
    if head is None and mix is not None:  # --only mixed
        head = {"gbps": mix["decode_kv_gbps_in_mixed_step"], "ms_per_step": mix["ms_per_step"], "roofline": None}
    if head is None and mdl is not None:  # --only model
        head = {"gbps": mdl["gbps_weights_plus_kv"], "ms_per_step": mdl["ms_per_step"], "roofline": None}
    if head is None:  # --only swap
        head = {"gbps": swp["swap_out_gbps"], "ms_per_step": swp["swap_out_ms"], "roofline": None}
    result = {
        "metric": METRIC,
        "value": round(head["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) bf16 Q/K/V (seeded torch/numpy generators), random non-contiguous block tables",
        "config": {"workload": "C2 paged decode, Llama-3-8B shape: 256 seqs, ctx U[512,8192], "
                               "32 q-heads / 8 kv-heads, head_dim 128, block_size 16, bf16 KV, one query per seq",
                   "num_seqs": 256, "num_heads": 32, "num_kv_heads": 8, "head_dim": 128,
                   "block_size": 16, "seed": SEED, "parallelism": "single GPU"},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "decode_bf16": dec,
        "gather_bf16": gat,
        "append_bf16": app,
        "decode_fp8": fp8,
        "prefix_cow_c4": c4,
        "prefill_attention": pre,
        "runner_step_mixed": mix,
        "model_decode_step": mdl,
        "kv_swap": swp,
        "gpu": torch.cuda.get_device_name(0),
    }
    if args.only is not None:
        result["config"]["workload"] = f"--only {args.only}"
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
