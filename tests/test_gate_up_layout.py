"""The fused gate|up weight layout of the model's projections (CPU):
interleave_gate_up puts gate and up rows in alternating blocks of 16 and
split_gate_up undoes it; the tiled weight layout and its inverse."""
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


def test_tiled_weight_rowmajor_inverts_the_layout_definition():
    """TiledWeight.rowmajor (torch ops, here on the CPU) against the tiled
    layout restated unit by unit: unit (j, b, r, u) holds columns
    128 j + 8 (u ^ r) .. + 7 of row 16 b + r."""
    import numpy as np
    from zealot_amd import dense
    n, k = 48, 384
    w = np.random.default_rng(3).integers(0, 1 << 16, size=(n, k), dtype=np.uint16)
    t = np.empty(n * k, np.uint16)
    for j in range(k // 128):
        for b in range(n // 16):
            for r in range(16):
                for u in range(16):
                    o = ((j * (n // 16) + b) * 16 + r) * 128 + 8 * u
                    t[o:o + 8] = w[16 * b + r, 128 * j + 8 * (u ^ r):128 * j + 8 * (u ^ r) + 8]
    tw = dense.TiledWeight(torch.from_numpy(t.view(np.int16)).view(torch.bfloat16), n, k)
    assert tw.shape == (n, k) and tw.numel() == n * k
    back = tw.rowmajor().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(back, w)


def test_tiled_weight_rejects_wrong_buffers():
    from zealot_amd import dense
    with pytest.raises(ValueError):
        dense.TiledWeight(torch.zeros(48 * 128, dtype=torch.float32), 48, 128)
    with pytest.raises(ValueError):
        dense.TiledWeight(torch.zeros(47 * 128, dtype=torch.bfloat16), 48, 128)


def test_dense_wrappers_check_operand_sizes_before_any_launch():
    """The dense wrappers hand plain pointers to kernels that trust the sizes:
    a caller's out / residual / weight of the wrong size or dtype is rejected
    on the host (CPU tensors here: the check comes before any device work)."""
    import pytest
    import torch
    from zealot_amd import dense
    x = torch.zeros((4, 64), dtype=torch.bfloat16)
    w = torch.zeros(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        dense.rms_norm(x, w, out=torch.zeros((4, 32), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        dense.rms_norm(x, torch.zeros(32, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        dense.rms_norm(x, w, out=torch.zeros((4, 64), dtype=torch.float32))
    with pytest.raises(ValueError):
        dense.rms_norm(x, w, residual=torch.zeros((3, 64), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        dense.add(x, torch.zeros((4, 63), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        dense.linear(x, torch.zeros((16, 64), dtype=torch.bfloat16), out=torch.zeros((4, 8), dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        dense.linear_rms_norm(x, torch.zeros((16, 64), dtype=torch.bfloat16), torch.zeros(8, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        dense.linear_silu_mul(x, torch.zeros((32, 64), dtype=torch.bfloat16), out=torch.zeros((4, 8), dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        dense.silu_mul(x, torch.zeros((4, 64), dtype=torch.float32))
