"""Helpers shared by the GPU parity tests: seeded inputs, host<->device copies.

Inputs are generated on the host with numpy (PCG64, seeded) and fed identically
to the HIP path and to the oracle.  bf16 data is carried as uint16 bit patterns
on the host and as torch.bfloat16 on the device; fp8 pools as uint8.
"""
from __future__ import annotations

import math

import numpy as np
import torch

import oracle

DEV = "cuda"


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a).to(DEV)


def to_host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    if t.dtype == getattr(torch, "float8_e4m3fn", None):
        return t.view(torch.uint8).cpu().numpy()
    return t.cpu().numpy()


def as_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    """Values of a host array of the given oracle dtype, as float32."""
    if dtype == oracle.BF16:
        return oracle.f32_from_bf16_bits(a).reshape(a.shape)
    if dtype == oracle.FP8:
        return oracle.f32_from_e4m3_bits(a).reshape(a.shape)
    return a.astype(np.float32)


def normal(rng, shape, dtype: int) -> np.ndarray:
    """N(0,1) values (fp64 -> fp32 -> dtype with round-to-nearest-even)."""
    x = rng.standard_normal(shape).astype(np.float32)
    if dtype == oracle.BF16:
        return oracle.bf16_bits_from_f32(x).reshape(shape)
    return x


def paged_tables(rng, lens, block_size, slack=0.1, min_free=3):
    """Random non-contiguous block tables for the given context lengths.

    Returns (block_tables [N, max_blocks] int32 with -1 padding, num_blocks)."""
    pages = [(int(L) + block_size - 1) // block_size for L in lens]
    total = sum(pages)
    nb = int(math.ceil(total * (1 + slack))) + min_free
    perm = rng.permutation(nb).astype(np.int32)
    mb = max(max(pages), 1)
    bt = -np.ones((len(lens), mb), np.int32)
    o = 0
    for n, p in enumerate(pages):
        bt[n, :p] = perm[o:o + p]
        o += p
    return bt, nb


def decode_case(seed, H, Hkv, D, lens, kv_dtype, q_dtype=None, block_size=16):
    rng = np.random.default_rng(seed)
    q_dtype = kv_dtype if q_dtype is None else q_dtype
    bt, nb = paged_tables(rng, lens, block_size)
    kp = normal(rng, (nb, Hkv, block_size, D), kv_dtype)
    vp = normal(rng, (nb, Hkv, block_size, D), kv_dtype)
    q = normal(rng, (len(lens), H, D), q_dtype)
    return q, kp, vp, bt, nb


def max_abs_err(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def torch_decode_ref(q, kpool, vpool, bt, lens, block_size, k_scales=None, v_scales=None, fp8=False):
    """Plain PyTorch fp32 paged decode on the GPU, every sequence: out[n, h] =
    softmax(q[n, h] . K^T / sqrt(D)) V over the sequence's first lens[n]
    tokens of its pages, kv-head h // (H / Hkv) (grouped).  fp8 pools are
    uint8 e4m3 codes dequantised with the per-(sequence, kv-head) scales.
    For whole-batch checks of full-size runs; tests pin it against the oracle
    on the sequences they sample."""
    N, H, D = q.shape
    Hkv = kpool.shape[1]
    G = H // Hkv
    out = torch.empty((N, H, D), dtype=torch.float32, device=q.device)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        for n in range(N):
            L = int(lens[n])
            npg = (L + block_size - 1) // block_size
            idx = torch.from_numpy(np.ascontiguousarray(bt[n, :npg]).astype(np.int64)).to(q.device)

            def pages(pool, scales):
                p = pool.index_select(0, idx)  # [npg, Hkv, BS, D]
                p = p.view(torch.float8_e4m3fn).float() if fp8 else p.float()
                p = p.permute(1, 0, 2, 3).reshape(Hkv, npg * block_size, D)[:, :L]
                if scales is not None:
                    p = p * scales[n].view(Hkv, 1, 1)
                return p

            K, V = pages(kpool, k_scales), pages(vpool, v_scales)
            qn = q[n].float().view(Hkv, G, D)
            s = torch.matmul(qn, K.transpose(1, 2).contiguous()) / math.sqrt(D)  # [Hkv, G, L]
            out[n] = torch.matmul(torch.softmax(s, dim=-1), V).reshape(H, D)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    return out


def torch_prefill_ref(q, kpool, vpool, block_ids, start, block_size):
    """Plain PyTorch fp32 causal chunked prefill of one chunk on the GPU:
    q [C, H, D] are the chunk's rows at positions start .. start + C - 1 of a
    sequence whose pages are block_ids; row t attends keys 0 .. start + t
    (grouped kv-heads).  Returns [C, H, D] float32."""
    C, H, D = q.shape
    Hkv = kpool.shape[1]
    G = H // Hkv
    ctx = start + C
    npg = (ctx + block_size - 1) // block_size
    idx = torch.as_tensor(np.asarray(block_ids[:npg], np.int64), device=q.device)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        def pages(pool):
            p = pool.index_select(0, idx).float()
            return p.permute(1, 0, 2, 3).reshape(Hkv, npg * block_size, D)[:, :ctx]

        K, V = pages(kpool), pages(vpool)
        qn = q.float().view(C, Hkv, G, D).permute(1, 2, 0, 3).reshape(Hkv, G * C, D)
        s = torch.matmul(qn, K.transpose(1, 2).contiguous()) / math.sqrt(D)  # [Hkv, G * C, ctx]
        s = s.view(Hkv, G, C, ctx)
        rows = torch.arange(C, device=q.device).view(C, 1)
        keys = torch.arange(ctx, device=q.device).view(1, ctx)
        s = s.masked_fill((keys > start + rows).view(1, 1, C, ctx), float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1).view(Hkv, G * C, ctx), V)  # [Hkv, G * C, D]
        return o.view(Hkv, G, C, D).permute(2, 0, 1, 3).reshape(C, H, D)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev


def torch_model_decode_ref(cfg, w, tok, ctx_kv):
    """Plain PyTorch fp32 restatement of one decode step of
    zealot_amd.model.HipModelRunner.forward (src/cuda_runner.rs:271-660 op
    order) on the GPU: one step token per sequence (tok [N] int64), each
    attending its context K/V from ctx_kv(layer, n) -> (K, V), float32
    [Hkv, tokens, D] on the device, then its own K/V from the step's
    projection.  Weights are the model's (TiledWeight read back row-major),
    every activation stays fp32.  Returns the fp32 logits [N, vocab].
    Whole-batch check of full-size model steps; tests pin it against
    oracle/llama_ref.py on a small model."""
    from zealot_amd import dense
    H, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    G = H // Hkv
    N = tok.numel()

    def f32(t):
        return (t.rowmajor() if isinstance(t, dense.TiledWeight) else t).float()

    def rms(x, wt):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.rms_eps) * wt.float()

    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        resid = w.embedding.float()[tok]
        for layer, lw in enumerate(w.layers):
            qkv = rms(resid, lw.attn_norm) @ f32(lw.qkv).T
            q, kn, vn = qkv[:, :H * D], qkv[:, H * D:(H + Hkv) * D], qkv[:, (H + Hkv) * D:]
            attn = torch.empty((N, H * D), dtype=torch.float32, device=tok.device)
            for n in range(N):
                K, V = ctx_kv(layer, n)
                K = torch.cat([K, kn[n].view(Hkv, 1, D)], 1)
                V = torch.cat([V, vn[n].view(Hkv, 1, D)], 1)
                s = torch.matmul(q[n].view(Hkv, G, D), K.transpose(1, 2).contiguous()) / math.sqrt(D)
                attn[n] = torch.matmul(torch.softmax(s, -1), V).reshape(H * D)
            resid = resid + attn @ f32(lw.o).T
            normed = rms(resid, lw.ffn_norm)
            gate, up = dense.split_gate_up(f32(lw.gate_up))
            act = torch.nn.functional.silu(normed @ gate.T) * (normed @ up.T)
            resid = resid + act @ f32(lw.down).T
        return rms(resid, w.final_norm) @ f32(w.lm_head).T
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
