"""Launches past 512 MB read a small share of their rows with the default
cache policy instead of the non-temporal one (LN + modulate and the fused
join + LN: each row's first 1 KB piece; the gated residual: each tile's
first residual row). The policy changes only how the bytes travel, so a
large launch must give, bit for bit, what smaller launches (every load
non-temporal) give on the same rows: checked here for f16 and f32 on
launches above the threshold against the same rows in pieces below it,
with batch offsets (a gathered modulate / gate) and a ragged tail."""
import pytest
import torch

from t2h import ops

pytestmark = pytest.mark.gpu

C = 1536
LIMIT = 512 << 20   # the library's threshold, in bytes moved per launch


def _rows_over(nbytes_per_row):
    return LIMIT // nbytes_per_row + 1237   # a ragged tail past the threshold


def _pieces(rows, n):
    step = (rows + n - 1) // n
    return [(s, min(s + step, rows)) for s in range(0, rows, step)]


def _offsets(rows, dev):
    # three batches; the pieces below cut across batch boundaries
    return torch.tensor([0, rows // 3, (2 * rows) // 3 + 5, rows], dtype=torch.int64, device=dev)


def _local_offsets(offsets, lo, hi):
    o = offsets.clamp(lo, hi) - lo
    return o


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_ln_modulate_large_equals_pieces(dev, dt):
    e = torch.finfo(dt).bits // 8
    rows = _rows_over(2 * C * e)
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn((rows, C), generator=g, device=dev).to(dt)
    shift = torch.randn((3, C), generator=g, device=dev) * 0.1
    scale = torch.randn((3, C), generator=g, device=dev) * 0.1
    off = _offsets(rows, dev)
    big = ops.ln_modulate(x, 1e-6, shift=shift, scale=scale, offsets=off)
    for lo, hi in _pieces(rows, 4):
        # the batches this piece touches, with offsets relative to the piece
        part = ops.ln_modulate(x[lo:hi], 1e-6, shift=shift, scale=scale, offsets=_local_offsets(off, lo, hi))
        assert torch.equal(part.view(torch.int16 if e == 2 else torch.int32),
                           big[lo:hi].view(torch.int16 if e == 2 else torch.int32)), (dt, lo, hi)


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_gate_residual_large_equals_pieces(dev, dt):
    e = torch.finfo(dt).bits // 8
    rows = _rows_over(3 * C * e)
    g = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn((rows, C), generator=g, device=dev).to(dt)
    h = torch.randn((rows, C), generator=g, device=dev).to(dt)
    gate = torch.randn((3, C), generator=g, device=dev) * 0.1
    bias = torch.randn((C,), generator=g, device=dev) * 0.02
    off = _offsets(rows, dev)
    big = ops.gate_residual(x, h, gate=gate, bias=bias, offsets=off)
    for lo, hi in _pieces(rows, 4):
        part = ops.gate_residual(x[lo:hi], h[lo:hi], gate=gate, bias=bias, offsets=_local_offsets(off, lo, hi))
        assert torch.equal(part.view(torch.int16 if e == 2 else torch.int32),
                           big[lo:hi].view(torch.int16 if e == 2 else torch.int32)), (dt, lo, hi)


def test_join_ln_large_equals_pieces(dev):
    dt = torch.float16
    rows = _rows_over(4 * C * 2)
    g = torch.Generator(device=dev).manual_seed(13)
    x = torch.randn((rows, C), generator=g, device=dev).to(dt)
    h = torch.randn((rows, C), generator=g, device=dev).to(dt)
    gate = torch.randn((3, C), generator=g, device=dev) * 0.1
    bias = torch.randn((C,), generator=g, device=dev) * 0.02
    shift = torch.randn((3, C), generator=g, device=dev) * 0.1
    scale = torch.randn((3, C), generator=g, device=dev) * 0.1
    off = _offsets(rows, dev)
    xb, yb = torch.empty_like(x), torch.empty_like(x)
    ops.gate_residual_ln_modulate(x, h, gate=gate, bias=bias, shift=shift, scale=scale, offsets=off,
                                  x_out=xb, y_out=yb)
    for lo, hi in _pieces(rows, 4):
        xp, yp = torch.empty_like(x[lo:hi]), torch.empty_like(x[lo:hi])
        ops.gate_residual_ln_modulate(x[lo:hi], h[lo:hi], gate=gate, bias=bias, shift=shift, scale=scale,
                                      offsets=_local_offsets(off, lo, hi), x_out=xp, y_out=yp)
        assert torch.equal(xp.view(torch.int16), xb[lo:hi].view(torch.int16)), (lo, hi)
        assert torch.equal(yp.view(torch.int16), yb[lo:hi].view(torch.int16)), (lo, hi)
