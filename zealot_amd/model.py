"""A batched Llama-shaped ModelRunner step on the gfx950 path: the dense ops
(zealot_amd.dense) around one KV write and one attention call per layer for
the whole schedule() batch.

Same math as the reference runner's step (src/cuda_runner.rs:271-660):
embedding -> per layer [RMSNorm -> q/k/v projections -> KV store -> paged
attention -> o_proj -> residual add -> RMSNorm -> gate/up projections ->
SiLU(gate) * up -> down projection -> residual add] -> final RMSNorm of each
sequence's last token -> lm_head logits (no rotary embedding, as in the
reference).  What differs is the shape of the work:
  - one launch per op for all sequences of the batch (the reference loops
    over sequences, cuda_runner.rs:274);
  - q/k/v come from ONE projection against a fused [(H + 2 Hkv) D, hidden]
    weight (its split-k sums, when it has them, added by the kernel that
    writes K and V to the pages: zk_cache_write_batch_qkv), gate/up from one
    against [2 I, hidden] whose gate and up rows
    alternate in blocks of 16, so the projection's waves hold the gate and
    up outputs of the same columns and write SiLU(gate) * up themselves
    (dense.linear_silu_mul); K and V are appended and
    q attended straight out of the fused output through row strides (no
    transpose kernels, no copies; cf. cuda_runner.rs:373-392);
  - each residual add is fused into the RMSNorm that follows it, and so,
    for the o and down projections, is the projection's split-k sum when it
    runs on the weight-streaming kernel (dense.linear_rms_norm); the final
    norm runs only over the last row of each sequence;
  - the large decode-time weights (gate|up, down, lm_head) are kept tiled
    (dense.TiledWeight): the weight-streaming kernel reads them with
    contiguous 1 KiB loads; their row-major copies serve steps of more than
    64 rows (prefill, mixed) on the GEMM plan, since the weight-streaming
    kernel reads a weight once per 64 rows;
  - weights are random-initialised here (there is no checkpoint loader in
    this build; the reference loads HF weights, model_loader.rs:241).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import dense
from .runner import PagedKVRunner, StepPlan


@dataclass
class LlamaConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_eps: float = 1e-6

    @staticmethod
    def llama3_8b(num_layers: int = 32) -> "LlamaConfig":
        return LlamaConfig(128256, 4096, 14336, num_layers, 32, 8, 128)


@dataclass
class LayerWeights:
    attn_norm: torch.Tensor  # [hidden]
    qkv: torch.Tensor        # [(H + 2 Hkv) D, hidden]: q rows, then k, then v
    o: torch.Tensor          # [hidden, H D]
    ffn_norm: torch.Tensor   # [hidden]
    gate_up: object          # [2 I, hidden]: gate and up rows interleaved in blocks of 16 (dense.interleave_gate_up);
                             # a dense.TiledWeight of it for bf16 models
    down: object             # [hidden, I] (a dense.TiledWeight for bf16 models)


@dataclass
class LlamaWeights:
    embedding: torch.Tensor  # [vocab, hidden]
    layers: list
    final_norm: torch.Tensor  # [hidden]
    lm_head: object           # [vocab, hidden] (a dense.TiledWeight for bf16 models)

    @staticmethod
    def random(cfg: LlamaConfig, dtype=torch.bfloat16, device="cuda", seed: int = 0,
               tiled: bool = True, keep_full: bool = True) -> "LlamaWeights":
        """N(0, 1/fan_in) projections and N(1, 0.1) norm weights (seeded);
        with tiled (bf16 only) gate|up, down and lm_head as dense.TiledWeight,
        keeping their row-major copies for steps of more than 64 rows unless
        keep_full is off (decode-only callers: half the memory of those
        weights)."""
        g = torch.Generator(device=device).manual_seed(seed)
        tile = ((lambda t: dense.tile_weight(t, keep_full=keep_full)) if tiled and dtype == torch.bfloat16
                else (lambda t: t))

        def lin(n, k):
            return (torch.randn((n, k), generator=g, device=device) / math.sqrt(k)).to(dtype)

        def norm(n):
            return (1 + 0.1 * torch.randn((n,), generator=g, device=device)).to(dtype)

        H, Hkv, D, hid, I = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size, cfg.intermediate_size
        layers = [LayerWeights(norm(hid), lin((H + 2 * Hkv) * D, hid), lin(hid, H * D), norm(hid),
                               tile(dense.interleave_gate_up(lin(I, hid), lin(I, hid))), tile(lin(hid, I)))
                  for _ in range(cfg.num_layers)]
        emb = torch.randn((cfg.vocab_size, hid), generator=g, device=device).to(dtype)
        return LlamaWeights(emb, layers, norm(hid), tile(lin(cfg.vocab_size, hid)))


class HipModelRunner:
    """ModelRunner::step (engine.rs:15-37) for a schedule() batch: returns the
    f32 logits [len(batch), vocab] of each sequence's last step token."""

    def __init__(self, cfg: LlamaConfig, weights: LlamaWeights, kv: PagedKVRunner):
        c = kv.cache
        if (c.num_layers, c.num_kv_heads, c.head_dim) != (cfg.num_layers, cfg.num_kv_heads, cfg.head_dim):
            raise ValueError("KV cache shape does not match the model")
        self.cfg, self.w, self.kv = cfg, weights, kv

    def drop_state(self, request_id: str) -> None:
        self.kv.drop_state(request_id)

    def step(self, out) -> torch.Tensor:
        """One step over ScheduleOutput `out` (zealot_amd.scheduler)."""
        plan = self.kv.begin_step(out)
        if not out.batch:
            return torch.empty((0, self.cfg.vocab_size), dtype=torch.float32, device=self.w.embedding.device)
        ids = [t for e in out.batch for t in e.step_input()]
        dev = self.w.embedding.device
        ids_dev = torch.tensor(ids, dtype=torch.int64, device=dev)
        last = torch.tensor(plan_last_rows(plan), dtype=torch.int64, device=dev)
        return self.forward(plan, ids_dev, last)

    def forward(self, plan: StepPlan, ids: torch.Tensor, last_rows: torch.Tensor) -> torch.Tensor:
        cfg, w = self.cfg, self.w
        H, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        T = plan.total_tokens
        if ids.numel() != T:
            raise ValueError("one token id per step row")
        qd, kd = H * D, Hkv * D
        resid = dense.embedding(ids, w.embedding)  # the residual stream [T, hidden]
        normed = torch.empty_like(resid)
        dense.rms_norm(resid, w.layers[0].attn_norm, cfg.rms_eps, out=normed)
        last = len(w.layers) - 1
        for layer, lw in enumerate(w.layers):
            if normed.dtype == torch.bfloat16:  # projection and KV write in one call
                qkv = self.kv.write_qkv(layer, plan, normed, lw.qkv, H)
            else:
                qkv = dense.linear(normed, lw.qkv)
                self.kv.write(layer, plan, qkv[:, qd:qd + kd].view(T, Hkv, D), qkv[:, qd + kd:].view(T, Hkv, D))
            q = qkv[:, :qd].view(T, H, D)
            attn = self.kv.attention(layer, plan, q)
            # resid += o_proj(attn); normed = norm(resid)
            dense.linear_rms_norm(attn.view(T, qd), lw.o, lw.ffn_norm, cfg.rms_eps, residual=resid, out=normed,
                                  residual_out=resid)
            act = dense.linear_silu_mul(normed, lw.gate_up)
            if layer < last:  # resid += down_proj(act); normed = the next layer's attention norm of resid
                dense.linear_rms_norm(act, lw.down, w.layers[layer + 1].attn_norm, cfg.rms_eps, residual=resid,
                                      out=normed, residual_out=resid)
        delta = dense.linear(act, w.layers[last].down)
        final, _ = dense.rms_norm(delta, w.final_norm, cfg.rms_eps, residual=resid, rows=last_rows)
        return dense.linear(final, w.lm_head, out_dtype=torch.float32)


def plan_last_rows(plan: StepPlan) -> list:
    """Row of each entry's last step token in the packed batch."""
    rows, o = [], 0
    for n in plan.num_tokens[:len(plan.ids)]:
        o += int(n)
        rows.append(o - 1)
    return rows
