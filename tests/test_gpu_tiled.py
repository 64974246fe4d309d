"""Tiled weights (zk_weight_tile, zk_linear_tiled, zk_linear_rms_norm_tiled,
zk_linear_silu_mul_tiled) on the MI355X.

The tiled layout is pinned by its definition restated in numpy: unit
(j, b, r, u) of the tiled buffer holds columns 128 j + 8 (u ^ r) .. + 7 of row
16 b + r.  The products over tiled weights must equal the weight-streaming
kernel over the row-major weights in the same configuration (tile rows,
split of k) bit for bit: the same bytes reach LDS in the same places, only
the loads' addresses differ.  With more than 64 rows of x the tiled kernel
covers them in blocks of 64, which must equal one row-major call per block.
Sanity bar against the float64 product as for the row-major kernel (1e-2 of
the largest |y| for bf16 outputs)."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, normal, to_dev, to_host

pytestmark = pytest.mark.gpu


def _tile_np(w16: np.ndarray) -> np.ndarray:
    """The tiled layout of a row-major [n, k] array of 16-bit words, by the
    definition (one 8-element unit at a time)."""
    n, k = w16.shape
    out = np.empty(n * k, dtype=w16.dtype)
    nb, kj = n // 16, k // 128
    for j in range(kj):
        for b in range(nb):
            for r in range(16):
                for u in range(16):
                    o = ((j * nb + b) * 16 + r) * 128 + 8 * u
                    c = 128 * j + 8 * (u ^ r)
                    out[o:o + 8] = w16[16 * b + r, c:c + 8]
    return out


def _weight(rng, n, k):
    return oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)


@pytest.mark.parametrize("n,k", [(16, 128), (48, 256), (160, 384), (1024, 512)])
def test_weight_tile_matches_the_layout_definition(n, k):
    from zealot_amd import dense
    rng = np.random.default_rng(n * 7 + k)
    w = rng.integers(0, 1 << 16, size=(n, k), dtype=np.uint16)
    announce(f"weight_tile {n}x{k}")
    wd = to_dev(w).view(torch.bfloat16)
    t = dense.tile_weight(wd)
    torch.cuda.synchronize()
    got = t.data.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, _tile_np(w))
    assert torch.equal(t.rowmajor().view(torch.int16), wd.view(torch.int16))


def test_weight_tile_rejects_bad_shapes_and_overlap():
    from zealot_amd import _lib, dense
    from zealot_amd._lib import ZealotError
    w = torch.zeros((32, 256), dtype=torch.bfloat16, device="cuda")
    for n, k in ((24, 256), (32, 200)):
        with pytest.raises(ZealotError):
            _lib.check(_lib.lib().zk_weight_tile(w.data_ptr(), torch.empty_like(w).data_ptr(), n, k, None))
    with pytest.raises(ZealotError):  # in place
        _lib.check(_lib.lib().zk_weight_tile(w.data_ptr(), w.data_ptr(), 32, 256, None))
    with pytest.raises(ValueError):
        dense.tile_weight(w.float())


def _rowmajor_blocks(x, w, splits, rows, out_dtype):
    """The row-major weight-streaming kernel, one call per 64 rows of x."""
    from zealot_amd import dense
    return torch.cat([dense.linear_skinny(x[i:i + 64], w, splits, rows, out_dtype=out_dtype)
                      for i in range(0, x.shape[0], 64)])


@pytest.mark.parametrize("m,n,k,od", [(64, 4096, 1024, "bf16"), (1, 256, 512, "bf16"), (17, 640, 256, "bf16"),
                                      (64, 28672, 4096, "bf16"), (64, 4096, 14336, "bf16"), (50, 1024, 512, "f32"),
                                      (150, 512, 1024, "bf16"), (130, 1280, 256, "f32")])
def test_linear_tiled_is_the_rowmajor_kernel_bit_for_bit(m, n, k, od):
    from zealot_amd import dense
    rng = np.random.default_rng(m + n + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    w16 = _weight(rng, n, k)
    w = to_dev(w16)
    odt = torch.float32 if od == "f32" else torch.bfloat16
    announce(f"linear_tiled {m}x{n}x{k} {od}")
    wt = dense.tile_weight(w)
    got = dense.linear(x, wt, out_dtype=odt)
    ch = dense.linear_choice(m, n, k, torch.bfloat16, odt, tiled=True)
    assert ch["splits"] >= 1 and ch["tile_rows"] in (64, 128), ch
    ref = _rowmajor_blocks(x, w, ch["splits"], ch["tile_rows"], odt)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16 if od == "bf16" else torch.int32),
                       ref.view(torch.int16 if od == "bf16" else torch.int32)), ch
    xs = as_f32(to_host(x), oracle.BF16).astype(np.float64)
    want = xs @ as_f32(w16, oracle.BF16).astype(np.float64).T
    gotf = got.float().cpu().numpy()
    assert np.abs(gotf - want).max() <= 1e-2 * np.abs(want).max()


@pytest.mark.parametrize("m,n,k,with_res", [(64, 4096, 4096, True), (64, 4096, 14336, True), (9, 1024, 512, False),
                                            (100, 512, 1024, True)])
def test_linear_rms_norm_tiled_is_the_unfused_sequence_bit_for_bit(m, n, k, with_res):
    """Through the configuration the tiled plan ran: split sums added by the
    norm kernel (fused_splits > 1) or the tiled projection, then zk_rms_norm."""
    from zealot_amd import dense
    rng = np.random.default_rng(m * 3 + n + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    w = to_dev(_weight(rng, n, k))
    g = to_dev(normal(rng, (n,), oracle.BF16))
    r0 = to_dev(normal(rng, (m, n), oracle.BF16)) if with_res else None
    announce(f"linear_rms_norm_tiled {m}x{n}x{k} residual={with_res}")
    wt = dense.tile_weight(w)
    res = r0.clone() if with_res else None
    got = dense.linear_rms_norm(x, wt, g, 1e-5, residual=res, residual_out=res)
    out = got[0] if with_res else got
    ch = dense.linear_choice(m, n, k, tiled=True)
    if ch["fused_splits"] > 1:
        y = _rowmajor_blocks(x, w, ch["fused_splits"], ch["fused_rows"], torch.bfloat16)
    else:
        y = dense.linear(x, wt)
    ref = dense.rms_norm(y, g, 1e-5, residual=r0.clone() if with_res else None)
    ref_out = ref[0] if with_res else ref
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), ch
    if with_res:
        assert torch.equal(res.view(torch.int16), ref[1].view(torch.int16))


@pytest.mark.parametrize("m,n,k,splits,rows", [(64, 4096, 14336, 7, 128), (100, 512, 1024, 4, 64)])
def test_linear_rms_norm_tiled_pinned_split_is_the_unfused_sequence_bit_for_bit(m, n, k, splits, rows):
    """The tiled plan pinned to a split of k (zk_linear_pin_split): the norm
    kernel adds the split sums of the tiled projection, bit for bit the
    row-major kernel with that split, then zk_rms_norm."""
    from zealot_amd import dense
    rng = np.random.default_rng(m * 5 + n + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    w = to_dev(_weight(rng, n, k))
    g = to_dev(normal(rng, (n,), oracle.BF16))
    r0 = to_dev(normal(rng, (m, n), oracle.BF16))
    announce(f"linear_rms_norm_tiled pinned split {m}x{n}x{k} splits={splits} rows={rows}")
    wt = dense.tile_weight(w)
    dense.linear_rms_norm(x, wt, g, 1e-5, residual=r0.clone())  # makes the plan
    before = dense.linear_choice(m, n, k, tiled=True)
    dense.pin_split(m, n, k, splits, rows, tiled=True)
    try:
        assert dense.linear_choice(m, n, k, tiled=True)["fused_splits"] == splits
        res = r0.clone()
        out, _ = dense.linear_rms_norm(x, wt, g, 1e-5, residual=res, residual_out=res)
        y = _rowmajor_blocks(x, w, splits, rows, torch.bfloat16)
        ref_out, ref_res = dense.rms_norm(y, g, 1e-5, residual=r0.clone())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(res.view(torch.int16), ref_res.view(torch.int16))
    finally:
        dense.pin_split(m, n, k, before["fused_splits"], before["fused_rows"], tiled=True)


@pytest.mark.parametrize("m,inter,k", [(64, 14336, 4096), (7, 1024, 512), (200, 512, 1024)])
def test_linear_silu_mul_tiled_is_the_unfused_sequence_bit_for_bit(m, inter, k):
    """One launch over the tiled interleaved gate|up weight against the
    row-major kernel (128-row tiles, no split) and SiLU * up of its rounded
    gate / up columns; close to the float64 product."""
    from zealot_amd import dense
    rng = np.random.default_rng(m + inter * 5 + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    gate, up = _weight(rng, inter, k), _weight(rng, inter, k)
    w = dense.interleave_gate_up(to_dev(gate), to_dev(up))
    announce(f"linear_silu_mul_tiled {m}x{inter}x{k}")
    act = dense.linear_silu_mul(x, dense.tile_weight(w))
    y = _rowmajor_blocks(x, w, 1, 128, torch.bfloat16).view(m, inter // 16, 2, 16)
    ref = dense.silu_mul(y[:, :, 0].reshape(m, inter), y[:, :, 1].reshape(m, inter))
    torch.cuda.synchronize()
    assert torch.equal(act.view(torch.int16), ref.view(torch.int16))
    xs = as_f32(to_host(x), oracle.BF16).astype(np.float64)
    g64 = xs @ as_f32(gate, oracle.BF16).astype(np.float64).T
    u64 = xs @ as_f32(up, oracle.BF16).astype(np.float64).T
    want = g64 / (1 + np.exp(-g64)) * u64
    got = as_f32(to_host(act), oracle.BF16)
    assert np.abs(got - want).max() <= 3e-2 * np.abs(want).max()
