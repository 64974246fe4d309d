"""CPU restatement of the reference runner's step math -- TEST INFRASTRUCTURE.

src/cuda_runner.rs:271-660 per sequence: embedding (embedding.cu) -> per
layer: rms_norm (rms_norm.cu) -> q/k/v = normed . W^T (cublasSgemm_v2) ->
KV store -> paged attention over everything cached, causal within the chunk
(attention.cu:117-121 / paged_attention.cu) -> o_proj -> add -> rms_norm ->
gate/up -> silu_gate_mul (activation.cu) -> down -> add; final rms_norm of
the last token -> lm_head.  All in float32 with the oracle's C kernels
(or_rms_norm, or_silu_gate_mul, or_add, or_embedding, or_matmul,
or_paged_prefill over a private contiguous page table).  The fused q|k|v and
gate|up weights are split back into the reference's separate projections.

Pinned through its parts (tests/test_oracle_dense.py, tests/test_oracle.py);
the composition itself is the reference's op order.
"""
from __future__ import annotations

import numpy as np

from . import BF16, F32, GROUPED, add, embedding, f32_from_bf16_bits, linear, paged_prefill, rms_norm, silu_gate_mul


class LlamaRef:
    """weights: dict of float32 numpy arrays with the fused layouts of
    zealot_amd.model.LlamaWeights (qkv [(H+2Hkv)D, hid], gate_up [2I, hid] with
    gate and up rows interleaved in blocks of 16)."""

    def __init__(self, cfg, weights, matmul=None):
        """matmul(x, w) = x . w^T: the oracle's or_matmul by default; a wide
        model's test may pass numpy's float32 product (the same sums in another
        order, pinned against or_matmul in tests/test_oracle_dense.py)."""
        self.cfg = cfg
        self.w = weights
        self.mm = matmul or linear
        self.kv = {}  # request id -> per layer [K (tokens, Hkv, D), V]
        # gate_up rows: gate and up interleaved in blocks of 16 -> the two projections
        I = cfg.intermediate_size
        self.gate_up = []
        for lw in weights["layers"]:
            gu = lw["gate_up"].reshape(I // 16, 2, 16, -1)
            self.gate_up.append((np.ascontiguousarray(gu[:, 0].reshape(I, -1)),
                                 np.ascontiguousarray(gu[:, 1].reshape(I, -1))))

    def drop(self, rid):
        self.kv.pop(rid, None)

    def _attend(self, rid, layer, q, start):
        """Chunk rows q [n, H, D] at positions start.. over the sequence's cache."""
        cfg = self.cfg
        K, V = self.kv[rid][layer]
        T, Hkv, D = K.shape
        pages = max(1, (T + 15) // 16)
        kp = np.zeros((pages * 16, Hkv, D), np.float32)
        vp = np.zeros_like(kp)
        kp[:T], vp[:T] = K, V
        kp = np.ascontiguousarray(kp.reshape(pages, 16, Hkv, D).transpose(0, 2, 1, 3))
        vp = np.ascontiguousarray(vp.reshape(pages, 16, Hkv, D).transpose(0, 2, 1, 3))
        bt = np.arange(pages, dtype=np.int32)[None, :]
        cu = np.array([0, q.shape[0]], np.int64)
        return paged_prefill(q, kp, vp, F32, bt, cu, [start], Hkv, D, 16,
                             np.float32(1 / np.sqrt(cfg.head_dim)), True, GROUPED)

    def step(self, entries):
        """entries: list of (request id, token ids of this step, tokens_before).
        Returns logits [len(entries), vocab] (float32)."""
        cfg, w, mm = self.cfg, self.w, self.mm
        H, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        qd, kd = H * D, Hkv * D
        logits = []
        for rid, ids, before in entries:
            n = len(ids)
            if before == 0:
                self.kv[rid] = [[np.zeros((0, Hkv, D), np.float32)] * 2 for _ in range(cfg.num_layers)]
            assert self.kv[rid][0][0].shape[0] == before
            h = embedding(np.asarray(ids, np.int64), w["embedding"])
            for layer in range(cfg.num_layers):
                lw = w["layers"][layer]
                normed = rms_norm(h, lw["attn_norm"], cfg.rms_eps)
                q = mm(normed, lw["qkv"][:qd])
                k = mm(normed, lw["qkv"][qd:qd + kd])
                v = mm(normed, lw["qkv"][qd + kd:])
                K, V = self.kv[rid][layer]
                self.kv[rid][layer] = [np.concatenate([K, k.reshape(n, Hkv, D)]),
                                       np.concatenate([V, v.reshape(n, Hkv, D)])]
                attn = self._attend(rid, layer, q.reshape(n, H, D), before).reshape(n, qd)
                h = add(mm(attn, lw["o"]), h)
                normed = rms_norm(h, lw["ffn_norm"], cfg.rms_eps)
                gate_w, up_w = self.gate_up[layer]
                gate = mm(normed, gate_w)
                up = mm(normed, up_w)
                h = add(mm(silu_gate_mul(gate, up), lw["down"]), h)
            final = rms_norm(h[-1:], w["final_norm"], cfg.rms_eps)
            logits.append(mm(final, w["lm_head"])[0])
        return np.stack(logits)


def weights_to_numpy(weights):
    """zealot_amd.model.LlamaWeights (f32 or bf16 torch tensors) -> float32
    numpy dict (bf16 values exactly)."""
    def f(t):
        if hasattr(t, "rowmajor"):  # a weight kept in the kernel's tiled layout
            t = t.rowmajor()
        t = t.detach().cpu()
        if str(t.dtype) == "torch.bfloat16":
            import torch
            return f32_from_bf16_bits(t.view(torch.int16).numpy().view(np.uint16)).reshape(tuple(t.shape))
        return t.float().numpy()
    return {"embedding": f(weights.embedding), "final_norm": f(weights.final_norm), "lm_head": f(weights.lm_head),
            "layers": [{"attn_norm": f(l.attn_norm), "qkv": f(l.qkv), "o": f(l.o), "ffn_norm": f(l.ffn_norm),
                        "gate_up": f(l.gate_up), "down": f(l.down)} for l in weights.layers]}


__all__ = ["LlamaRef", "weights_to_numpy", "BF16"]
