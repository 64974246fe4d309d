"""Dense ops around the path (zk_rms_norm, zk_silu_mul, zk_add, zk_embedding,
zk_linear) on the MI355X against the oracle's restatements of rms_norm.cu,
activation.cu, embedding.cu and the cublasSgemm_v2 product.

Bars: add and embedding bit-exact (f32 sum / bf16 round of the f32 sum; rows
copied); f32 rms_norm / silu_mul within 2e-6 relative (f32 rounding order);
bf16 outputs within one bf16 rounding (2^-8 relative) of the f32 value of the
same bf16 inputs; f32 linear within 1e-5 relative of the float64 product,
bf16 linear within 1e-2 of the largest |y| (f32 accumulation, bf16 output);
zk_linear_rms_norm bit-exact against the unfused sequence through the same
projection configuration."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import announce, as_f32, normal, to_dev, to_host

pytestmark = pytest.mark.gpu


def _vals(a, dt):
    return a if dt == "f32" else as_f32(a, oracle.BF16)


def _rand(rng, shape, dt, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return x if dt == "f32" else oracle.bf16_bits_from_f32(x).reshape(shape)


def _close(got, ref, dt, rtol_f32=2e-6):
    if dt == "f32":
        return np.allclose(got, ref, rtol=rtol_f32, atol=rtol_f32 * max(1.0, np.abs(ref).max()))
    return np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("rows,dim", [(1, 4096), (7, 4096), (5, 1000), (3, 8192), (2, 24), (4, 7)])
def test_rms_norm(dt, rows, dim):
    from zealot_amd import dense
    rng = np.random.default_rng(rows * 7 + dim)
    x, w = _rand(rng, (rows, dim), dt, 3.0), _rand(rng, (dim,), dt)
    announce(f"rms_norm {dt} {rows}x{dim}")
    got = _vals(to_host(dense.rms_norm(to_dev(x), to_dev(w), 1e-6)), dt)
    ref = oracle.rms_norm(_vals(x, dt), _vals(w, dt), 1e-6)
    assert _close(got, ref, dt)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_add_rms_norm_fused_in_place_and_selected_rows(dt):
    from zealot_amd import dense
    rng = np.random.default_rng(3)
    rows, dim = 9, 4096
    x, r, w = _rand(rng, (rows, dim), dt), _rand(rng, (rows, dim), dt), _rand(rng, (dim,), dt)
    announce(f"add+rms_norm {dt}")
    rd = to_dev(r)
    out, res = dense.rms_norm(to_dev(x), to_dev(w), 1e-6, residual=rd, residual_out=rd)
    s = oracle.add(_vals(x, dt), _vals(r, dt))
    s_stored = s if dt == "f32" else as_f32(oracle.bf16_bits_from_f32(s).reshape(s.shape), oracle.BF16)
    assert np.array_equal(_vals(to_host(res), dt), s_stored)  # the new residual, rounded as stored
    assert _close(_vals(to_host(out), dt), oracle.rms_norm(s_stored, _vals(w, dt), 1e-6), dt)
    # selected rows: the final norm of the last token of each sequence
    sel = torch.tensor([8, 0, 3], dtype=torch.int64, device="cuda")
    out2, res2 = dense.rms_norm(to_dev(x), to_dev(w), 1e-6, residual=to_dev(r), rows=sel)
    assert np.array_equal(_vals(to_host(res2), dt), s_stored[[8, 0, 3]])
    assert _close(_vals(to_host(out2), dt), oracle.rms_norm(s_stored[[8, 0, 3]], _vals(w, dt), 1e-6), dt)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols", [(5, 14336), (3, 100), (1, 8)])
def test_silu_mul_on_fused_gate_up(dt, rows, cols):
    from zealot_amd import dense
    rng = np.random.default_rng(rows + cols)
    gu = _rand(rng, (rows, 2 * cols), dt, 4.0)
    announce(f"silu_mul {dt} {rows}x{cols}")
    g = to_dev(gu)
    got = _vals(to_host(dense.silu_mul(g[:, :cols], g[:, cols:])), dt)
    v = _vals(gu, dt)
    ref = oracle.silu_gate_mul(np.ascontiguousarray(v[:, :cols]), np.ascontiguousarray(v[:, cols:]))
    assert _close(got, ref, dt, rtol_f32=4e-6)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n", [1, 13, 4096 * 33])
def test_add_bit_exact(dt, n):
    from zealot_amd import dense
    rng = np.random.default_rng(n)
    a, b = _rand(rng, (n,), dt), _rand(rng, (n,), dt)
    announce(f"add {dt} {n}")
    got = to_host(dense.add(to_dev(a), to_dev(b)))
    s = oracle.add(_vals(a, dt), _vals(b, dt))
    assert np.array_equal(got, s if dt == "f32" else oracle.bf16_bits_from_f32(s).reshape(s.shape))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_embedding_rows_and_out_of_range(dt):
    from zealot_amd import dense
    rng = np.random.default_rng(5)
    vocab, dim = 1000, 4096
    table = _rand(rng, (vocab, dim), dt)
    ids = np.array([5, 999, 0, 5, 1000, -1, 123], np.int64)
    announce(f"embedding {dt}")
    got = to_host(dense.embedding(to_dev(ids), to_dev(table)))
    ok = (ids >= 0) & (ids < vocab)
    ref = oracle.embedding(ids[ok], _vals(table, dt))
    assert np.array_equal(_vals(got[ok], dt), ref)
    assert np.all(got[~ok] == 0)  # the reference reads out of bounds here


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (37, 6144, 4096), (256, 512, 1024), (5, 7, 3)])
def test_linear_f32(m, n, k):
    from zealot_amd import dense
    rng = np.random.default_rng(m + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    announce(f"linear f32 {m}x{n}x{k}")
    got = to_host(dense.linear(to_dev(x), to_dev(w)))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max()) * 4
    if m * n * k <= 10 ** 6:  # the oracle's scalar product on small shapes
        assert np.allclose(got, oracle.linear(x, w), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("m,n,k,out_f32", [(1, 4096, 4096, False), (300, 28672, 4096, False),
                                           (7, 128256, 4096, True), (64, 4096, 14336, False),
                                           (16, 6144, 4096, False), (33, 1000, 512, False), (64, 28672, 4096, True),
                                           (48, 37, 768, True)])
def test_linear_bf16(m, n, k, out_f32):
    from zealot_amd import dense
    rng = np.random.default_rng(m + n)
    x = normal(rng, (m, k), oracle.BF16)
    w = oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)
    announce(f"linear bf16 {m}x{n}x{k}")
    y = dense.linear(to_dev(x), to_dev(w), out_dtype=torch.float32 if out_f32 else None)
    got = to_host(y) if out_f32 else as_f32(to_host(y), oracle.BF16)
    xs, ws = as_f32(x, oracle.BF16), as_f32(w, oracle.BF16)
    cols = rng.choice(n, size=min(n, 512), replace=False)  # a sample of outputs against float64
    ref = xs.astype(np.float64) @ ws[cols].astype(np.float64).T
    assert np.abs(got[:, cols] - ref).max() <= 1e-2 * np.abs(ref).max()



@pytest.mark.parametrize("m,n,k,rows,splits,out_f32", [(1, 64, 1024, 64, 1, False), (16, 4096, 4096, 128, 1, False),
                                                       (37, 6144, 4096, 64, 2, False), (64, 4096, 14336, 128, 7, False),
                                                       (64, 4096, 4096, 64, 4, True), (50, 1024, 2048, 128, 2, True),
                                                       (17, 192, 4096, 64, 8, False), (33, 256, 512, 128, 1, True)])
def test_linear_skinny_kernel(m, n, k, rows, splits, out_f32):
    """The weight-streaming kernel at each m-tile count and split of k, against
    the float64 product of the same bf16 operands; splits > 1 add the ranges
    in a fixed order, so two calls agree bit for bit."""
    from zealot_amd import dense
    rng = np.random.default_rng(m * 7 + splits + rows)
    x = normal(rng, (m, k), oracle.BF16)
    w = oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)
    announce(f"linear_skinny {m}x{n}x{k} rows={rows} splits={splits}")
    xd, wd = to_dev(x), to_dev(w)
    y1 = dense.linear_skinny(xd, wd, splits, rows, out_dtype=torch.float32 if out_f32 else None)
    y2 = dense.linear_skinny(xd, wd, splits, rows, out_dtype=torch.float32 if out_f32 else None)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16) if not out_f32 else y1, y2.view(torch.int16) if not out_f32 else y2)
    got = to_host(y1) if out_f32 else as_f32(to_host(y1), oracle.BF16)
    ref = as_f32(x, oracle.BF16).astype(np.float64) @ as_f32(w, oracle.BF16).astype(np.float64).T
    tol = (1e-5 if out_f32 else 1e-2) * np.abs(ref).max()
    assert np.abs(got - ref).max() <= tol
    if m * n * k <= 4 * 10 ** 6:  # the oracle's scalar product on small shapes
        ref32 = oracle.linear(as_f32(x, oracle.BF16), as_f32(w, oracle.BF16))
        assert np.abs(got - ref32).max() <= tol


def test_linear_skinny_rejects_unsupported_shapes():
    from zealot_amd import dense
    from zealot_amd._lib import ZealotError
    x = torch.zeros((65, 1024), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 1024), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ZealotError):
        dense.linear_skinny(x, w)  # m > 64
    with pytest.raises(ZealotError):
        dense.linear_skinny(x[:8], w, splits=16, tile_rows=64)  # k % (128 * splits) != 0
    with pytest.raises(ZealotError):
        dense.linear_skinny(x[:8], w[:48], tile_rows=64)  # n % tile_rows != 0
    with pytest.raises(ZealotError):
        dense.linear_skinny(x[:8], w, tile_rows=128)  # n % tile_rows != 0


def test_linear_misaligned_operands_after_tuning():
    """A shape whose cached choice may be the skinny kernel (16-byte aligned
    operands only) still runs for operands 2 bytes off alignment: zk_linear
    falls back to the hipBLASLt algorithm kept beside it."""
    from zealot_amd import dense
    rng = np.random.default_rng(77)
    m, n, k = 64, 4096, 4096
    x = normal(rng, (m, k), oracle.BF16)
    w = oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)
    announce("linear bf16 aligned, then misaligned x / y")
    xd, wd = to_dev(x), to_dev(w)
    y_al = dense.linear(xd, wd)  # tunes the shape
    xbuf = torch.empty(m * k + 8, dtype=torch.bfloat16, device="cuda")
    x_mis = xbuf[1:1 + m * k].view(m, k)
    x_mis.copy_(xd)
    ybuf = torch.empty(m * n + 8, dtype=torch.bfloat16, device="cuda")
    y_mis = ybuf[1:1 + m * n].view(m, n)
    dense.linear(x_mis, wd, out=y_mis)
    torch.cuda.synchronize()
    ref = as_f32(x, oracle.BF16).astype(np.float64) @ as_f32(w, oracle.BF16).astype(np.float64).T
    for y in (y_al, y_mis):
        got = as_f32(to_host(y.contiguous()), oracle.BF16)
        assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()


def test_linear_on_two_streams_at_once():
    """Each stream has its own workspaces: split-k products (whose sums pass
    through a workspace) on two streams in flight together both come out
    right."""
    from zealot_amd import dense
    rng = np.random.default_rng(91)
    m, n, k = 64, 4096, 4096
    ws = [oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)
          for _ in range(2)]
    xs = [normal(rng, (m, k), oracle.BF16) for _ in range(2)]
    wd, xd = [to_dev(w) for w in ws], [to_dev(x) for x in xs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    torch.cuda.synchronize()  # the operands were written on the default stream
    announce("linear + linear_skinny(splits=4) on two streams")
    outs = []
    for rep in range(3):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
                dense.linear_skinny(xd[i], wd[i], 4, 64, out=y, stream=st)
                z = dense.linear(xd[i], wd[i], stream=st)
                outs.append((i, y, z))
    torch.cuda.synchronize()
    for i, y, z in outs:
        ref = as_f32(xs[i], oracle.BF16).astype(np.float64) @ as_f32(ws[i], oracle.BF16).astype(np.float64).T
        for t in (y, z):
            got = as_f32(to_host(t), oracle.BF16)
            assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()


def test_linear_on_more_streams_than_kept_workspaces():
    """Ten streams in turn: the ninth and tenth take the workspaces of the
    least recently used streams (after the device drains), and every product
    is still right, including on a stream whose workspace was replaced."""
    from zealot_amd import dense
    rng = np.random.default_rng(93)
    m, n, k = 64, 4096, 4096
    w = oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k)
    x = normal(rng, (m, k), oracle.BF16)
    wd, xd = to_dev(w), to_dev(x)
    ref = as_f32(x, oracle.BF16).astype(np.float64) @ as_f32(w, oracle.BF16).astype(np.float64).T
    streams = [torch.cuda.Stream() for _ in range(10)]  # default priority
    torch.cuda.synchronize()
    announce("linear_skinny(splits=4) on 10 streams, then the first again")
    outs = []
    for st in streams + streams[:1]:
        with torch.cuda.stream(st):
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            dense.linear_skinny(xd, wd, 4, 64, out=y, stream=st)
            outs.append(y)
        st.synchronize()
    for y in outs:
        got = as_f32(to_host(y), oracle.BF16)
        assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize("m,n,k,with_res", [(64, 4096, 14336, True), (64, 4096, 4096, True), (7, 4096, 4096, False),
                                            (33, 1024, 2048, True), (200, 512, 1024, True)])
def test_linear_rms_norm_is_the_unfused_sequence_bit_for_bit(m, n, k, with_res):
    """zk_linear_rms_norm against the unfused sequence through the projection
    configuration it ran (zk_linear_choice): the weight-streaming kernel with
    split k whose sums the norm kernel adds, or zk_linear's own choice, then
    zk_rms_norm; new residual and normed rows agree bit for bit."""
    from zealot_amd import dense
    rng = np.random.default_rng(m + n + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    w = to_dev(oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k))
    g = to_dev(normal(rng, (n,), oracle.BF16))
    r0 = to_dev(normal(rng, (m, n), oracle.BF16)) if with_res else None
    announce(f"linear_rms_norm {m}x{n}x{k} residual={with_res}")
    res = r0.clone() if with_res else None
    got = dense.linear_rms_norm(x, w, g, 1e-5, residual=res, residual_out=res)
    out = got[0] if with_res else got
    ch = dense.linear_choice(m, n, k)
    if ch["fused_splits"] > 1:
        y = dense.linear_skinny(x, w, ch["fused_splits"], ch["fused_rows"])
    else:
        y = dense.linear(x, w)
    ref = dense.rms_norm(y, g, 1e-5, residual=r0.clone() if with_res else None)
    ref_out = ref[0] if with_res else ref
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    if with_res:
        assert torch.equal(res.view(torch.int16), ref[1].view(torch.int16))
    # and the float64 product of the same operands, through the oracle's norm
    xs, ws = as_f32(to_host(x), oracle.BF16), as_f32(to_host(w), oracle.BF16)
    yy = xs.astype(np.float64) @ ws.astype(np.float64).T
    if with_res:
        yy = yy + as_f32(to_host(r0), oracle.BF16)
    want = oracle.rms_norm(yy.astype(np.float32), as_f32(to_host(g), oracle.BF16), 1e-5)
    gotf = as_f32(to_host(out), oracle.BF16)
    assert np.abs(gotf - want).max() <= 3e-2 * np.abs(want).max()


@pytest.mark.parametrize("m,n,k,splits,rows", [(64, 4096, 4096, 4, 64), (33, 1024, 2048, 8, 128), (7, 4096, 14336, 7, 64)])
def test_linear_rms_norm_pinned_split_is_the_unfused_sequence_bit_for_bit(m, n, k, splits, rows):
    """The plan pinned to a split of k (zk_linear_pin_split), so the norm
    kernel that adds the split sums (rms_norm_partials) runs whatever the
    tuning chose: bit for bit the weight-streaming kernel with that split,
    then zk_rms_norm, new residual included."""
    from zealot_amd import dense
    rng = np.random.default_rng(m * 7 + n + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    w = to_dev(oracle.bf16_bits_from_f32((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).reshape(n, k))
    g = to_dev(normal(rng, (n,), oracle.BF16))
    r0 = to_dev(normal(rng, (m, n), oracle.BF16))
    announce(f"linear_rms_norm pinned split {m}x{n}x{k} splits={splits} rows={rows}")
    dense.linear_rms_norm(x, w, g, 1e-5, residual=r0.clone())  # makes the plan
    before = dense.linear_choice(m, n, k)
    dense.pin_split(m, n, k, splits, rows)
    try:
        assert dense.linear_choice(m, n, k)["fused_splits"] == splits
        res = r0.clone()
        out, _ = dense.linear_rms_norm(x, w, g, 1e-5, residual=res, residual_out=res)
        y = dense.linear_skinny(x, w, splits, rows)
        ref_out, ref_res = dense.rms_norm(y, g, 1e-5, residual=r0.clone())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
        assert torch.equal(res.view(torch.int16), ref_res.view(torch.int16))
    finally:
        dense.pin_split(m, n, k, before["fused_splits"], before["fused_rows"])


def test_pin_split_rejects_what_does_not_fit():
    from zealot_amd import dense
    from zealot_amd._lib import ZealotError
    x = torch.zeros((8, 1024), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((512, 1024), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ZealotError, match="no plan"):
        dense.pin_split(8, 512, 3072, 2, 64)
    dense.linear(x, w)
    with pytest.raises(ZealotError, match="does not fit"):
        dense.pin_split(8, 512, 1024, 16, 64)  # k % (128 * 16) != 0
    with pytest.raises(ZealotError, match="does not fit"):
        dense.pin_split(8, 512, 1024, 1, 64)   # no split


@pytest.mark.parametrize("m,inter,k", [(64, 14336, 4096), (7, 1024, 512), (33, 512, 256), (200, 512, 1024)])
def test_linear_silu_mul_is_the_unfused_sequence_bit_for_bit(m, inter, k):
    """zk_linear_silu_mul (gate and up rows interleaved in blocks of 16)
    against zk_linear on the same weight followed by SiLU * up of the rounded
    gate / up columns: bit for bit whether the projection's own waves formed
    the product (weight-streaming kernel, 128-row tiles, no split) or a second
    kernel did; and close to the float64 product."""
    from zealot_amd import dense
    rng = np.random.default_rng(m + inter + k)
    x = to_dev(normal(rng, (m, k), oracle.BF16))
    gate = oracle.bf16_bits_from_f32((rng.standard_normal((inter, k)) / np.sqrt(k)).astype(np.float32)).reshape(inter, k)
    up = oracle.bf16_bits_from_f32((rng.standard_normal((inter, k)) / np.sqrt(k)).astype(np.float32)).reshape(inter, k)
    w = dense.interleave_gate_up(to_dev(gate), to_dev(up))
    announce(f"linear_silu_mul {m}x{inter}x{k}")
    act = dense.linear_silu_mul(x, w)
    y = dense.linear(x, w).view(m, inter // 16, 2, 16)
    ref = dense.silu_mul(y[:, :, 0].reshape(m, inter), y[:, :, 1].reshape(m, inter))
    torch.cuda.synchronize()
    assert torch.equal(act.view(torch.int16), ref.view(torch.int16)), dense.linear_choice(m, 2 * inter, k)
    xs = as_f32(to_host(x), oracle.BF16).astype(np.float64)
    g64 = xs @ as_f32(gate, oracle.BF16).astype(np.float64).T
    u64 = xs @ as_f32(up, oracle.BF16).astype(np.float64).T
    want = g64 / (1 + np.exp(-g64)) * u64
    got = as_f32(to_host(act), oracle.BF16)
    assert np.abs(got - want).max() <= 3e-2 * np.abs(want).max()
