"""A batched Llama-shaped runner step (zealot_amd.model.HipModelRunner) on
the MI355X: scheduler -> one bind -> per layer one dense op chain, one KV
write and one attention call for the whole batch -> logits, against the
oracle's per-sequence restatement of cuda_runner.rs:271-660
(oracle/llama_ref.py) on the same weights and the same token stream.

Requests of different prompt lengths run through chunked prefill and decode
(greedy tokens from the GPU logits, fed to both).  Bars: f32 weights and
pools -- logits within 2e-4 of the largest |logit| (f32 rounding order of the
GEMMs and attention); bf16 -- within 6e-2 of the largest |logit| (bf16
activations between ops, f32 reference) and the same argmax on at least 90 %
of the rows.  A third run squeezes four requests into eight blocks so the
scheduler preempts by swap (zk_cache_swap_out / _in through the runner) and
by recompute; the logits must not notice.  At the Llama-3-8B widths, one run
also pins the PyTorch fp32 restatement of the full-size model test against
the oracle, and one takes prefill steps of more than 64 rows."""
import numpy as np
import pytest
import torch

from tests.gpu_util import announce, torch_model_decode_ref

pytestmark = pytest.mark.gpu


def _np_matmul(x, w):
    """x . w^T in float32 through numpy (BLAS): the oracle's or_matmul in
    another summation order (tests/test_oracle_dense.py pins the two)."""
    return np.ascontiguousarray(x, np.float32) @ np.asarray(w, np.float32).T


def _run(dtype, tol, argmax_frac, swap=False, cfg=None, short=False, long_prefill=False, pin_torch_ref=False):
    """long_prefill: prefill steps of more than 64 rows (chunks of 128, up
    to 256 prefill tokens a step), so the tiled weights' products run on
    their row-major copies.  pin_torch_ref: on the first all-decode step, the
    PyTorch fp32 restatement the full-size model test uses
    (tests.gpu_util.torch_model_decode_ref) is checked against the oracle on
    the oracle's own context K/V (1e-4 of the largest |logit|)."""
    import zealot_amd as ze
    from oracle.llama_ref import LlamaRef, weights_to_numpy
    from zealot_amd import KVCache, PagedKVRunner, Priority, Scheduler, SchedulerConfig
    from zealot_amd.model import HipModelRunner, LlamaConfig, LlamaWeights
    cfg = cfg or LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=8,
                             num_kv_heads=2, head_dim=64)
    # with swap: 8 blocks for four requests, so the scheduler preempts by
    # swap (and once by recompute) while the reference keeps every sequence
    NB, BS = (8, 16) if swap else (64, 16)
    max_prefill, chunk = (256, 128) if long_prefill else (64, 32)
    bm = ze.BlockManager(NB, BS)
    sched = Scheduler(SchedulerConfig(max_num_seqs=4, block_size=BS, num_gpu_blocks=NB,
                                      max_prefill_tokens=max_prefill, prefill_chunk_size=chunk,
                                      swap_blocks=64 if swap else 0), block_manager=bm)
    cache = KVCache(NB, BS, cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, dtype=dtype, max_seqs=8,
                    max_blocks_per_seq=NB)
    if swap:
        cache.enable_swap(64)
    w = LlamaWeights.random(cfg, dtype=dtype, seed=11)
    runner = HipModelRunner(cfg, w, PagedKVRunner(cache, bm))
    ref = LlamaRef(cfg, weights_to_numpy(w), matmul=_np_matmul if cfg.hidden_size > 1024 else None)
    rng = np.random.default_rng(12)
    if swap:
        prompts = {"a": 45, "b": 7, "c": 70, "d": 20}
        max_new = {"a": 20, "b": 30, "c": 12, "d": 25}
        prio = {"a": Priority.Lowest, "b": Priority.High, "c": Priority.Medium, "d": Priority.Highest}
    elif long_prefill:
        prompts = {"a": 300, "b": 7, "c": 150}
        max_new = {"a": 3, "b": 4, "c": 2}
        prio = {r: Priority.Medium for r in prompts}
    elif short:
        prompts = {"a": 45, "b": 7, "c": 40}
        max_new = {"a": 3, "b": 4, "c": 2}
        prio = {r: Priority.Medium for r in prompts}
    else:
        prompts = {"a": 45, "b": 7, "c": 70}
        max_new = {"a": 6, "b": 9, "c": 4}
        prio = {r: Priority.Medium for r in prompts}
    for rid, p in prompts.items():
        sched.add(sched.make_sequence(rid, list(rng.integers(0, cfg.vocab_size, p)), max_new[rid], prio[rid]))
    worst, agree, rows, steps, swaps, widest, pinned = 0.0, 0, 0, 0, 0, 0, False
    while not sched.is_idle():
        steps += 1
        assert steps < 100
        out = sched.schedule()
        for rid in out.preempted:
            ref.drop(rid)
        swaps += len(out.swapped_out)
        announce(f"model {dtype} step {steps}: {[(e.request_id, e.num_tokens, e.tokens_before) for e in out.batch]}")
        entries = [(e.request_id, e.step_input(), e.tokens_before) for e in out.batch]
        widest = max(widest, sum(len(x[1]) for x in entries))
        pin_now = pin_torch_ref and not pinned and all(not e.is_prefill() for e in out.batch)
        if pin_now:  # the oracle's context K/V before this step
            ctx = {rid: [[torch.from_numpy(a.copy()) for a in kv] for kv in ref.kv[rid]] for rid, _, _ in entries}
        logits = runner.step(out).cpu().numpy()
        expect = ref.step(entries)
        if pin_now:
            rids = [rid for rid, _, _ in entries]
            tok = torch.tensor([x[1][0] for x in entries], dtype=torch.int64, device="cuda")

            def ctx_kv(layer, n):
                K, V = ctx[rids[n]][layer]
                return (K.cuda().permute(1, 0, 2).contiguous(), V.cuda().permute(1, 0, 2).contiguous())

            tref = torch_model_decode_ref(cfg, w, tok, ctx_kv).cpu().numpy()
            perr = float(np.abs(tref - expect).max() / np.abs(expect).max())
            announce(f"torch model restatement vs oracle: {perr:.2e} of max |logit|")
            assert perr <= 1e-4, perr
            pinned = True
        scale = np.abs(expect).max()
        worst = max(worst, float(np.abs(logits - expect).max() / scale))
        agree += int((logits.argmax(1) == expect.argmax(1)).sum())
        rows += len(entries)
        for i, e in enumerate(out.batch):
            if not e.is_prefill() or e.is_final_chunk():
                e.push_token(int(logits[i].argmax()))
                if e.is_prefill():
                    e.mark_prefilled()
        for e in out.batch:
            if e.is_prefill():
                sched.advance_prefill(e.request_id)
        for e in out.batch:
            info = sched.seq_info(e.request_id)
            if info["state"] == 1 and info["output_len"] >= max_new[e.request_id]:
                runner.drop_state(e.request_id)
                ref.drop(e.request_id)
                sched.finish(e.request_id)
    torch.cuda.synchronize()
    assert worst <= tol, worst
    assert agree >= argmax_frac * rows, (agree, rows)
    assert bm.free_blocks == NB
    assert pinned or not pin_torch_ref
    if long_prefill:
        assert widest > 64, widest  # a step the tiled weights served from their row-major copies
    if swap:
        assert swaps >= 1 and cache.swap_space()[1] == 64


def test_model_step_f32_matches_reference():
    _run(torch.float32, 2e-4, 1.0)


def test_model_step_bf16_close_to_reference():
    _run(torch.bfloat16, 6e-2, 0.9)


def test_model_step_with_swap_preemption_matches_reference():
    """Eight blocks for four requests: sequences are swapped out and back in
    (and one is recomputed) mid-stream; the logits still follow the
    reference, which never preempts."""
    _run(torch.float32, 2e-4, 1.0, swap=True)


def test_model_step_llama3_width_bf16_close_to_reference():
    """Two layers at the Llama-3-8B widths the bench times (hidden 4096, 32
    query / 8 KV heads of 128, intermediate 14336; the vocabulary cut to 1024):
    the tiled gate|up, down and lm_head products, the fused QKV write and the
    128-dim decode and prefill at their real shapes, against the oracle."""
    from zealot_amd.model import LlamaConfig
    cfg = LlamaConfig(vocab_size=1024, hidden_size=4096, intermediate_size=14336, num_layers=2, num_heads=32,
                      num_kv_heads=8, head_dim=128)
    _run(torch.bfloat16, 6e-2, 0.9, cfg=cfg, short=True, pin_torch_ref=True)


def test_model_step_llama3_width_long_prefill_close_to_reference():
    """The same widths with prefill steps of up to 256 rows: the tiled
    gate|up, down (and lm_head) weights serve those steps from their
    row-major copies on the GEMM plan, decode steps from the tiled layout;
    both against the oracle."""
    from zealot_amd.model import LlamaConfig
    cfg = LlamaConfig(vocab_size=1024, hidden_size=4096, intermediate_size=14336, num_layers=2, num_heads=32,
                      num_kv_heads=8, head_dim=128)
    _run(torch.bfloat16, 6e-2, 0.9, cfg=cfg, long_prefill=True)


def test_model_decode_step_at_bench_shape():
    """The bench's model step at its full shape (Llama-3-8B: 32 layers, hidden
    4096, 32/8 heads of 128, intermediate 14336, vocab 128256, random bf16
    weights; 64 sequences with contexts U[512, 8192] of random K/V in the
    cache) against a plain PyTorch fp32 restatement of the same step on the
    GPU: the op order of HipModelRunner.forward, fp32 throughout (the HIP
    path rounds activations to bf16 between ops), context K/V read from the
    cache's pages and the step token's own K/V from the reference's own
    projection (tests.gpu_util.torch_model_decode_ref, pinned against the
    oracle by the two-layer Llama-width test).  Bars: logits within 5e-2 of the largest |logit| (2.6e-2
    measured) and the same argmax on at least 75 % of the sequences (92 %
    measured)."""
    import ctypes
    import math
    import zealot_amd as ze
    from zealot_amd import KVCache, PagedKVRunner, dense
    from zealot_amd.kv_cache import SeqBatch
    from zealot_amd.model import HipModelRunner, LlamaConfig, LlamaWeights
    from zealot_amd.runner import StepPlan
    N, BS = 64, 16
    cfg = LlamaConfig.llama3_8b()
    H, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    G = H // Hkv
    rng = np.random.default_rng(91)
    ctx = rng.integers(512, 8193, N)
    pages = [(int(c) + BS - 1) // BS for c in ctx]
    nb = sum(pages) + 16
    announce(f"model step at bench shape: {N} seqs ctx {int(ctx.min())}..{int(ctx.max())}, {nb} blocks")
    bm = ze.BlockManager(nb, BS)
    cache = KVCache(nb, BS, cfg.num_layers, Hkv, D, dtype=torch.bfloat16, max_seqs=N, max_blocks_per_seq=max(pages))
    ids = [f"s{i}" for i in range(N)]
    for sid, p in zip(ids, pages):
        cache.register_seq(sid, p)
        for _ in range(p):
            cache.alloc_block(sid, bm)
    g = torch.Generator(device="cuda").manual_seed(91)
    before = [int(c) - 1 for c in ctx]
    allb = SeqBatch(ids)
    T0 = sum(before)
    for layer in range(cfg.num_layers):
        k = torch.randn((T0, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((T0, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        cache.write_batch(layer, allb, before, k, v)
        del k, v
    w = LlamaWeights.random(cfg, dtype=torch.bfloat16, seed=92)
    model = HipModelRunner(cfg, w, PagedKVRunner(cache, bm))
    plan = StepPlan(allb, (ctypes.c_int32 * N)(*([1] * N)), before, N)
    tok = torch.randint(0, cfg.vocab_size, (N,), generator=g, device="cuda")
    last = torch.arange(N, dtype=torch.int64, device="cuda")
    logits = model.forward(plan, tok, last)
    torch.cuda.synchronize()

    blocks = [cache.seq_state(s).block_ids for s in ids]

    def ctx_kv(layer, n):  # the context K/V the HIP step read: the cache's pages
        b = before[n]
        npg = (b + BS - 1) // BS
        idx = torch.tensor(blocks[n][:npg], dtype=torch.int64, device="cuda")
        kp, vp = cache.k_pool(layer), cache.v_pool(layer)
        K = kp.index_select(0, idx).float().permute(1, 0, 2, 3).reshape(Hkv, npg * BS, D)[:, :b]
        V = vp.index_select(0, idx).float().permute(1, 0, 2, 3).reshape(Hkv, npg * BS, D)[:, :b]
        return K, V

    ref = torch_model_decode_ref(cfg, w, tok, ctx_kv)
    got, want = logits.float(), ref
    err = float((got - want).abs().max() / want.abs().max())
    agree = float((got.argmax(1) == want.argmax(1)).float().mean())
    announce(f"model step at bench shape: max |logit err| / max |logit| = {err:.3e}, argmax agreement {agree:.2f}")
    assert err <= 5e-2, err
    assert agree >= 0.75, agree
