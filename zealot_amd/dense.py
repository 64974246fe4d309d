"""Dense ops around the paged-KV path over the C ABI (include/zealot_dense.h):
rms_norm (optionally fused with the residual add), silu_mul, add, embedding
and linear (hipBLASLt or the weight-streaming kernel; TiledWeight for weights
kept in that kernel's tiled layout).  Torch device tensors in, launches on
torch's current stream; the kernels are in zealot_amd/csrc/dense_ops.hip,
gemm.cpp and skinny_gemm.hip."""
from __future__ import annotations

import torch

from . import _lib
from .ops import _dev, _stream, zk_dtype


def _dt(t: torch.Tensor) -> int:
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"dense ops take float32 or bfloat16 tensors, got {t.dtype}")
    return zk_dtype(t)


def _sized(t, name: str, numel: int, dtype) -> None:
    """The kernels take plain pointers and trust the sizes: every operand is
    checked against the elements and dtype the launch will touch."""
    if t is None:
        return
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} elements, the op needs {numel}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def rms_norm(x, weight, eps: float = 1e-6, residual=None, out=None, residual_out=None, rows=None, stream=None):
    """out = rms_norm(s) * weight, s = x (+ residual, written to residual_out,
    which may be `residual`), over x's rows or over the rows listed in `rows`
    (device int64); rms_norm.cu:4-55."""
    dim = x.shape[-1]
    n = rows.numel() if rows is not None else x.numel() // dim
    if rows is None and x.numel() != n * dim:
        raise ValueError("x must hold whole rows of dim elements")
    if out is None:
        out = torch.empty((n, dim), dtype=x.dtype, device=x.device)
    if residual is not None and residual_out is None:
        residual_out = torch.empty((n, dim), dtype=x.dtype, device=x.device)
    _sized(weight, "weight", dim, x.dtype)
    _sized(out, "out", n * dim, x.dtype)
    if rows is None:
        _sized(residual, "residual", n * dim, x.dtype)
    elif residual is not None and (residual.numel() != x.numel() or residual.dtype != x.dtype):
        raise ValueError("residual must match x (its rows are selected by `rows` too)")
    _sized(residual_out, "residual_out", n * dim, x.dtype)
    _lib.check(_lib.lib().zk_rms_norm(
        _dev(x, "x"), None if residual is None else _dev(residual, "residual"), _dev(weight, "weight"),
        _dev(out, "out"), None if residual_out is None else _dev(residual_out, "residual_out"),
        None if rows is None else _dev(rows, "rows", torch.int64), n, dim, float(eps), _dt(x), _stream(stream)))
    return out if residual is None else (out, residual_out)


def silu_mul(gate, up, out=None, stream=None):
    """silu(gate) * up (activation.cu:4-12); gate / up may be column slices
    of one [rows, 2 * cols] tensor (a fused gate|up projection)."""
    rows, cols = gate.shape
    if up.dtype != gate.dtype:
        raise TypeError("gate and up must share a dtype")
    for name, t in (("gate", gate), ("up", up)):
        _dev(t, name, contiguous=False)
        if t.shape != (rows, cols) or t.stride(1) != 1:
            raise ValueError(f"{name} must be [rows, cols] with contiguous rows")
    if out is None:
        out = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
    _sized(out, "out", rows * cols, gate.dtype)
    _lib.check(_lib.lib().zk_silu_mul(gate.data_ptr(), up.data_ptr(), _dev(out, "out"), rows, cols, gate.stride(0),
                                      up.stride(0), _dt(gate), _stream(stream)))
    return out


def add(a, b, out=None, stream=None):
    _sized(b, "b", a.numel(), a.dtype)
    if out is None:
        out = torch.empty_like(a)
    _sized(out, "out", a.numel(), a.dtype)
    _lib.check(_lib.lib().zk_add(_dev(a, "a"), _dev(b, "b"), _dev(out, "out"), a.numel(), _dt(a), _stream(stream)))
    return out


def embedding(ids, table, out=None, stream=None):
    """table[ids] (embedding.cu:4-22); out-of-range ids give zero rows."""
    n = ids.numel()
    if out is None:
        out = torch.empty((n, table.shape[1]), dtype=table.dtype, device=table.device)
    _sized(out, "out", n * table.shape[1], table.dtype)
    _lib.check(_lib.lib().zk_embedding(_dev(ids, "ids", torch.int64), _dev(table, "table"), _dev(out, "out"), n,
                                       table.shape[0], table.shape[1], _dt(table), _stream(stream)))
    return out


class TiledWeight:
    """A bf16 weight [n, k] in the weight-streaming kernel's tiled layout
    (zk_weight_tile): [k / 128][n / 16][16 rows][16 units of 8], unit u of row
    r holding columns 8 (u ^ r) .. of its 128-column chunk.  linear,
    linear_rms_norm and linear_silu_mul take it in place of the row-major
    tensor; the products read it with contiguous 1 KiB loads (17-19 % faster
    on the large decode projections).  `data` is the flat device buffer.

    The weight-streaming kernel reads the whole weight once per 64 rows of
    x, so it suits decode-sized products only.  `full`, when kept (the
    row-major [n, k] weight), serves products of more than TILED_MAX_ROWS
    rows (prefill and mixed steps) on zk_linear's GEMM plan instead."""

    __slots__ = ("data", "n", "k", "full")

    def __init__(self, data: torch.Tensor, n: int, k: int, full: torch.Tensor | None = None):
        if data.dtype != torch.bfloat16 or data.numel() != n * k or not data.is_contiguous():
            raise ValueError("a tiled weight is a contiguous bf16 buffer of n * k elements")
        if full is not None and (full.dtype != torch.bfloat16 or tuple(full.shape) != (n, k)
                                 or not full.is_contiguous()):
            raise ValueError("the row-major copy is a contiguous bf16 [n, k] tensor")
        self.data, self.n, self.k, self.full = data, n, k, full

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def device(self):
        return self.data.device

    def numel(self) -> int:
        return self.n * self.k

    def rowmajor(self) -> torch.Tensor:
        """The row-major [n, k] weight (the inverse permutation, on the device)."""
        n, k = self.n, self.k
        # moved as int16 words, so every bit pattern (NaN payloads too) survives
        t = self.data.view(torch.int16).view(k // 128, n // 16, 16, 16, 8).permute(1, 2, 0, 3, 4)  # [b r j u e]
        r = torch.arange(16, device=t.device).view(16, 1)
        idx = (torch.arange(16, device=t.device).view(1, 16) ^ r).view(1, 16, 1, 16, 1).expand(t.shape)
        return torch.gather(t, 3, idx).reshape(n, k).view(torch.bfloat16)  # [b r j c e] = t[b r j (c ^ r) e]


def tile_weight(weight: torch.Tensor, stream=None, keep_full: bool = False) -> TiledWeight:
    """The tiled form of a row-major bf16 weight [n, k] (n % 16 == 0,
    k % 128 == 0), in a new buffer; keep_full keeps `weight` beside it for
    products of more than TILED_MAX_ROWS rows."""
    n, k = weight.shape
    if weight.dtype != torch.bfloat16:
        raise ValueError("tiled weights are bf16")
    out = torch.empty(n * k, dtype=torch.bfloat16, device=weight.device)
    _lib.check(_lib.lib().zk_weight_tile(_dev(weight, "weight"), _dev(out, "out"), n, k, _stream(stream)))
    return TiledWeight(out, n, k, weight.contiguous() if keep_full else None)


# Rows of x up to which a TiledWeight's product runs on the weight-streaming
# kernel even when its row-major copy is kept: that kernel reads the weight
# once per 64 rows, a GEMM once.
TILED_MAX_ROWS = 64


def _route(x, weight):
    """The weight a product of x runs on: a TiledWeight's row-major copy for
    more than TILED_MAX_ROWS rows, when it keeps one."""
    if isinstance(weight, TiledWeight) and weight.full is not None and x.shape[0] > TILED_MAX_ROWS:
        return weight.full
    return weight


def _tiled_x(x, weight):
    if x.dtype != torch.bfloat16 or x.shape[1] != weight.k:
        raise ValueError("tiled weights take bf16 x [m, k]")


def linear(x, weight, out=None, out_dtype=None, stream=None):
    """x [m, k] . weight[n, k]^T on hipBLASLt (the cublasSgemm_v2 sites) or the
    weight-streaming kernel, whichever the first call of the shape timed
    faster; a TiledWeight runs on the weight-streaming kernel (on its
    row-major copy, if kept, for more than TILED_MAX_ROWS rows)."""
    m, k = x.shape
    n = weight.shape[0]
    weight = _route(x, weight)
    if isinstance(weight, TiledWeight):
        _tiled_x(x, weight)
        if out is None:
            out = torch.empty((m, n), dtype=out_dtype or x.dtype, device=x.device)
        _sized(out, "out", m * n, out.dtype)  # the C ABI checks the dtype pair
        _lib.check(_lib.lib().zk_linear_tiled(_dev(x, "x"), _dev(weight.data, "weight"), _dev(out, "out"), m, n, k,
                                              zk_dtype(out), _stream(stream)))
        return out
    if weight.shape[1] != k or weight.dtype != x.dtype:
        raise ValueError("weight must be [n, k] of x's dtype")
    od = out_dtype or x.dtype
    if out is None:
        out = torch.empty((m, n), dtype=od, device=x.device)
    _sized(out, "out", m * n, out.dtype)  # the C ABI checks the dtype pair
    _lib.check(_lib.lib().zk_linear(_dev(x, "x"), _dev(weight, "weight"), _dev(out, "out"), m, n, k, _dt(x),
                                    zk_dtype(out), _stream(stream)))
    return out


def linear_rms_norm(x, weight, norm_weight, eps: float = 1e-6, residual=None, out=None, residual_out=None,
                    stream=None):
    """rms_norm(linear(x, weight), norm_weight, eps, residual, ...) bit for
    bit, for bf16 in two launches instead of three when the projection runs on
    the weight-streaming kernel with split k (its sums feed the norm
    directly); f32 runs the two calls.  Returns out, or (out, residual_out)
    with a residual."""
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k or weight.dtype != x.dtype:
        raise ValueError("weight must be [n, k] of x's dtype")
    weight = _route(x, weight)
    tiled = isinstance(weight, TiledWeight)
    if tiled:
        _tiled_x(x, weight)
    elif x.dtype != torch.bfloat16:
        return rms_norm(linear(x, weight), norm_weight, eps, residual=residual, out=out, residual_out=residual_out,
                        stream=stream)
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    if residual is not None and residual_out is None:
        residual_out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    _sized(norm_weight, "norm_weight", n, x.dtype)
    for name, t in (("out", out), ("residual", residual), ("residual_out", residual_out)):
        _sized(t, name, m * n, x.dtype)
    fn = _lib.lib().zk_linear_rms_norm_tiled if tiled else _lib.lib().zk_linear_rms_norm
    _lib.check(fn(
        _dev(x, "x"), _dev(weight.data if tiled else weight, "weight"), m, n, k,
        None if residual is None else _dev(residual, "residual"),
        _dev(norm_weight, "norm_weight"), float(eps), _dev(out, "out"),
        None if residual_out is None else _dev(residual_out, "residual_out"), _stream(stream)))
    return out if residual is None else (out, residual_out)


GATE_UP_BLOCK = 16  # rows of gate (then of up) per block of a fused gate|up weight


def interleave_gate_up(gate, up):
    """The fused [2 I, hidden] gate|up weight for linear_silu_mul: gate and up
    rows interleaved in blocks of GATE_UP_BLOCK."""
    i, hid = gate.shape
    if up.shape != gate.shape or i % GATE_UP_BLOCK:
        raise ValueError("gate and up must be [I, hidden] with I a multiple of 16")
    b = GATE_UP_BLOCK
    return torch.stack([gate.reshape(i // b, b, hid), up.reshape(i // b, b, hid)], 1).reshape(2 * i, hid).contiguous()


def split_gate_up(gate_up):
    """(gate, up) of a weight from interleave_gate_up."""
    n, hid = gate_up.shape
    b = GATE_UP_BLOCK
    v = gate_up.reshape(n // (2 * b), 2, b, hid)
    return v[:, 0].reshape(n // 2, hid), v[:, 1].reshape(n // 2, hid)


def linear_silu_mul(x, gate_up, out=None, gu=None, stream=None):
    """silu(x . gate^T) * (x . up^T) for a gate|up weight from
    interleave_gate_up, bit for bit linear() followed by SiLU * up of its
    rounded outputs; for bf16 one launch when the projection runs on the
    weight-streaming kernel without split."""
    m, k = x.shape
    n = gate_up.shape[0]
    if gate_up.shape[1] != k or gate_up.dtype != x.dtype or n % (2 * GATE_UP_BLOCK):
        raise ValueError("gate_up must be [2 I, k] of x's dtype, I a multiple of 16")
    gate_up = _route(x, gate_up)
    if isinstance(gate_up, TiledWeight):  # one launch, no projection buffer
        _tiled_x(x, gate_up)
        if out is None:
            out = torch.empty((m, n // 2), dtype=x.dtype, device=x.device)
        _sized(out, "out", m * (n // 2), x.dtype)
        _lib.check(_lib.lib().zk_linear_silu_mul_tiled(_dev(x, "x"), _dev(gate_up.data, "gate_up"), _dev(out, "out"),
                                                       m, n // 2, k, _stream(stream)))
        return out
    if x.dtype != torch.bfloat16:  # f32: the projection, then SiLU * up of its column blocks
        y = linear(x, gate_up).view(m, n // (2 * GATE_UP_BLOCK), 2, GATE_UP_BLOCK)
        return silu_mul(y[:, :, 0].reshape(m, n // 2), y[:, :, 1].reshape(m, n // 2), out=out, stream=stream)
    if out is None:
        out = torch.empty((m, n // 2), dtype=x.dtype, device=x.device)
    if gu is None:
        gu = torch.empty((m, n), dtype=x.dtype, device=x.device)
    _sized(out, "out", m * (n // 2), x.dtype)
    _sized(gu, "gu", m * n, x.dtype)
    _lib.check(_lib.lib().zk_linear_silu_mul(_dev(x, "x"), _dev(gate_up, "gate_up"), _dev(out, "out"), m, n // 2, k,
                                             _dev(gu, "gu"), _stream(stream)))
    return out


def linear_choice(m, n, k, in_dtype=torch.bfloat16, out_dtype=None, tiled=False) -> dict:
    """What the projection plan for this shape runs (after a first call made
    it): splits 0 = hipBLASLt, else the weight-streaming kernel with that split
    of k and tile_rows; fused_* is what linear_rms_norm runs.  tiled: the plan
    for a TiledWeight of that shape."""
    import ctypes
    code = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
    c = (ctypes.c_int * 4)()
    if tiled:
        _lib.check(_lib.lib().zk_linear_tiled_choice(m, n, k, code[out_dtype or in_dtype], c))
    else:
        _lib.check(_lib.lib().zk_linear_choice(m, n, k, code[in_dtype], code[out_dtype or in_dtype], c))
    return {"splits": c[0], "tile_rows": c[1], "fused_splits": c[2], "fused_rows": c[3]}


def pin_split(m, n, k, fused_splits, fused_rows, in_dtype=torch.bfloat16, out_dtype=None, tiled=False) -> None:
    """Pin the split-k configuration linear_rms_norm / write_batch_qkv fold
    for the plan an earlier call made for this shape (fused_splits 0: none)."""
    code = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
    _lib.check(_lib.lib().zk_linear_pin_split(m, n, k, code[in_dtype], code[out_dtype or in_dtype], int(tiled),
                                              fused_splits, fused_rows))


def linear_skinny(x, weight, splits=1, tile_rows=128, out=None, out_dtype=None, stream=None):
    """The weight-streaming kernel zk_linear may choose for bf16 and m <= 64,
    called directly: tiles of tile_rows weight rows, k split in `splits`."""
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k or weight.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise ValueError("x and weight must be bf16, weight [n, k]")
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype or x.dtype, device=x.device)
    _lib.check(_lib.lib().zk_linear_skinny(_dev(x, "x"), _dev(weight, "weight"), _dev(out, "out"), m, n, k,
                                           zk_dtype(out), tile_rows, splits, _stream(stream)))
    return out
