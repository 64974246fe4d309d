"""Pins of the oracle's dense ops (rms_norm.cu, activation.cu, embedding.cu and
the projection y = x . W^T) against independent float64 restatements of the
textbook formulas and closed forms (CPU only)."""
import numpy as np
import pytest

import oracle


@pytest.mark.parametrize("rows,dim", [(1, 1), (3, 7), (5, 256), (2, 4096)])
def test_rms_norm_matches_float64_formula(rows, dim):
    rng = np.random.default_rng(rows * 100 + dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32) * 3
    w = rng.standard_normal(dim).astype(np.float32)
    got = oracle.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.allclose(got, ref, rtol=2e-6, atol=2e-6)


def test_rms_norm_closed_forms():
    # a constant row c normalises to sign(c) * w (up to eps); zero row -> 0
    w = np.linspace(-2, 2, 64).astype(np.float32)
    for c in (5.0, -0.25):
        got = oracle.rms_norm(np.full((1, 64), c, np.float32), w, 0.0)
        assert np.allclose(got[0], np.sign(c) * w, rtol=1e-6)
    assert np.all(oracle.rms_norm(np.zeros((1, 64), np.float32), w, 1e-6) == 0)
    # scale invariance: rms_norm(a x) == rms_norm(x) for a > 0 (eps = 0)
    x = np.random.default_rng(1).standard_normal((2, 33)).astype(np.float32)
    assert np.allclose(oracle.rms_norm(8 * x, w[:33], 0.0), oracle.rms_norm(x, w[:33], 0.0), rtol=1e-5)


def test_silu_gate_mul():
    rng = np.random.default_rng(2)
    g = rng.standard_normal(1000).astype(np.float32) * 6
    u = rng.standard_normal(1000).astype(np.float32)
    got = oracle.silu_gate_mul(g, u)
    g64 = g.astype(np.float64)
    assert np.allclose(got, g64 / (1 + np.exp(-g64)) * u, rtol=1e-6, atol=1e-7)
    # silu(0) = 0; silu(g) -> g for large g, -> 0 for very negative g
    assert oracle.silu_gate_mul(np.array([0.0, 40.0, -40.0], np.float32), np.ones(3, np.float32)).tolist()[:2] \
        == [0.0, 40.0]
    assert abs(oracle.silu_gate_mul(np.array([-40.0], np.float32), np.ones(1, np.float32))[0]) < 1e-15


def test_add_and_embedding():
    a = np.arange(10, dtype=np.float32)
    assert oracle.add(a, a).tolist() == (2 * a).tolist()
    table = (np.arange(6)[:, None] * 1000 + np.arange(5)[None, :]).astype(np.float32)  # row id tagged
    ids = np.array([3, 0, 5, 3], np.int64)
    got = oracle.embedding(ids, table)
    assert np.array_equal(got, table[ids])


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (16, 64, 48)])
def test_linear_is_x_times_w_transposed(m, k, n):
    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    got = oracle.linear(x, w)
    assert got.shape == (m, n)
    assert np.allclose(got, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-5, atol=1e-5)
    # numpy's float32 product (the wide model test's matmul for LlamaRef): the
    # same sums in another order
    assert np.allclose(x @ w.T, got, rtol=1e-5, atol=1e-5)
    # a one-hot row picks a column of W^T
    e = np.zeros((1, k), np.float32)
    e[0, k - 1] = 1
    assert np.array_equal(oracle.linear(e, w)[0], w[:, k - 1])
