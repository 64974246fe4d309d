"""The fused gate|up weight layout of the model's projections (CPU):
interleave_gate_up puts gate and up rows in alternating blocks of 16 and
split_gate_up undoes it."""
import pytest
import torch


def test_interleave_then_split_is_identity_and_blocks_alternate():
    from zealot_amd import dense
    g = torch.arange(64 * 3, dtype=torch.float32).reshape(64, 3)
    u = -g - 1
    w = dense.interleave_gate_up(g, u)
    assert w.shape == (128, 3)
    for b in range(4):
        assert torch.equal(w[32 * b:32 * b + 16], g[16 * b:16 * b + 16])
        assert torch.equal(w[32 * b + 16:32 * b + 32], u[16 * b:16 * b + 16])
    g2, u2 = dense.split_gate_up(w)
    assert torch.equal(g2, g) and torch.equal(u2, u)


def test_interleave_rejects_ragged_blocks():
    from zealot_amd import dense
    with pytest.raises(ValueError):
        dense.interleave_gate_up(torch.zeros(24, 4), torch.zeros(24, 4))
