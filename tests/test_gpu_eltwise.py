"""GPU parity: activation(+bias) incl. GELU-tanh, gated residual (+ bias
fold, gathered gate), timestep embedding, through the C ABI, against the C
oracle (modules/nn.mojo:588-647; modules/transformer/modulated.mojo:22-33;
gpu/block.mojo:86-110; gpu/linear.mojo:662-684;
models/sparse_structure_flow.mojo:60-76). Metric/tolerances: tests/_parity.py."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, bits_equal, host, max_err, storage_round, to_dev
from t2h import nn, ops, sparse, workloads

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def test_config3_gelu_f16_full_size(dev):
    """BASELINE config 3a: h[32768,6144] f16 ~ N(0,1), bias[6144] ~ N(0,0.02),
    GELU-tanh(h + b). Full tensor on the GPU; 512 seeded rows against the oracle."""
    rows, f = 32768, 6144
    g = torch.Generator(device=dev).manual_seed(3)
    h = torch.randn((rows, f), generator=g, device=dev, dtype=torch.float32).half()
    bias = orc.randn(301, (f,), std=0.02)
    out = ops.activation(h, ops.ACT_GELU_TANH, bias=to_dev(bias, dev))
    idx = np.sort(np.random.default_rng(3).choice(rows, 512, replace=False))
    hs = host(h[idx])
    want = orc.gelu_tanh_bias(hs, bias)
    assert_close(out[idx], want, torch.float16, "config3 GELU f16")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2048, 6144), (100, 8192), (33, 1536), (7, 1000), (5, 3)])
def test_gelu_tanh_bias(dev, dtype, shape):
    x = storage_round(orc.randn(310, shape, std=3.0), dtype)
    bias = orc.randn(311, (shape[1],), std=0.02)
    got = ops.activation(to_dev(x, dev, dtype), ops.ACT_GELU_TANH, bias=to_dev(bias, dev))
    assert_close(got, orc.gelu_tanh_bias(x, bias), dtype, f"GELU {dtype} {shape}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(9, 520), (3, 4104), (6, 512), (13, 264)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_activation_slab_edges(dev, dtype, shape, with_bias):
    """The one-vector-per-thread layout (1 KB column slabs of 4-row tiles) at
    its edges: a last slab with a single live lane (520 f16 / bf16, 264 and
    4104 f32), exactly one slab (512 f16), rows off the 4-row tile, and rows
    narrower than a slab (264 f16), with and without the bias staged per
    slab. The guard elements after the output stay untouched."""
    rows, cols = shape
    x = storage_round(orc.randn(330 + cols, shape, std=3.0), dtype)
    bias = orc.randn(331 + cols, (cols,), std=0.02) if with_bias else None
    buf = torch.full((rows * cols + 256,), 7.0, dtype=dtype, device=dev)
    out = buf[: rows * cols].view(rows, cols)
    ops.activation(to_dev(x, dev, dtype), ops.ACT_GELU_TANH, bias=to_dev(bias, dev) if with_bias else None,
                   out=out)
    want = orc.gelu_tanh_bias(x, bias) if with_bias else orc.activation(x, ops.ACT_GELU_TANH)
    assert_close(out, want, dtype, f"GELU {dtype} {shape} bias={with_bias}")
    assert bool((buf[rows * cols:] == 7).all())


@pytest.mark.parametrize("kind", [ops.ACT_RELU, ops.ACT_SILU, ops.ACT_GELU, ops.ACT_GELU_TANH])
def test_activation_kinds(dev, kind):
    x = orc.randn(320 + kind, (513, 1536), std=4.0)
    got = nn.activation(to_dev(x, dev), kind)
    assert_close(got, orc.activation(x, kind), torch.float32, f"activation {kind}")


def test_gelu_limits(dev):
    """gelu(0) = 0, large |x|: gelu(x) -> x (x >> 0), -> 0 (x << 0), no NaN/inf."""
    x = np.array([[0.0, -0.0, 1e-30, -1e-30, 10.0, -10.0, 80.0, -80.0, 3e4, -3e4, 1e-3, -1e-3]], np.float32)
    got = host(nn.activation(to_dev(x, dev), ops.ACT_GELU_TANH))
    assert np.all(np.isfinite(got))
    assert got[0, 0] == 0.0 and got[0, 1] == 0.0
    assert_close(got, orc.activation(x, ops.ACT_GELU_TANH), torch.float32, "gelu limits")


def test_config3_gated_residual_f16(dev):
    """BASELINE config 3b: out = x + gate*y, x,y [32768,1536] f16, gate ~ N(0,0.1).
    f32 arithmetic identical to the oracle, one f16 rounding: bit-exact."""
    rows, c = 32768, 1536
    x = orc.round_f16(orc.randn(401, (rows, c)))
    y = orc.round_f16(orc.randn(402, (rows, c)))
    gate = orc.randn(403, (c,), std=0.1)
    got = ops.gate_residual(to_dev(x, dev, torch.float16), to_dev(y, dev, torch.float16), gate=to_dev(gate, dev))
    want = orc.gate_residual(x, y, gate)
    assert bits_equal(got, want, torch.float16), "f16 gated residual must be bit-exact"
    assert_close(got, want, torch.float16, "config3b")


@pytest.mark.parametrize("dtype", DTYPES)
def test_gate_residual_variants_bit_exact(dev, dtype):
    rows, c = 999, 1536
    x = storage_round(orc.randn(411, (rows, c)), dtype)
    h = storage_round(orc.randn(412, (rows, c)), dtype)
    gate = orc.randn(413, (c,), std=0.1)
    bias = orc.randn(414, (c,), std=0.05)
    dx, dh = to_dev(x, dev, dtype), to_dev(h, dev, dtype)
    cases = {
        "gate+bias": (ops.gate_residual(dx, dh, gate=to_dev(gate, dev), bias=to_dev(bias, dev)),
                      orc.gate_residual(x, h, gate, bias=bias)),
        "ungated+bias": (ops.gate_residual(dx, dh, bias=to_dev(bias, dev)),
                         orc.binop_flat(x, orc.add_bias(h, bias), orc.OP_ADD)),
        "plain add": (ops.gate_residual(dx, dh), orc.binop_flat(x, h, orc.OP_ADD)),
        "_gate only": (ops.gate_residual(None, dh, gate=to_dev(gate, dev)),
                       orc.gate(h.reshape(1, rows, c), gate.reshape(1, c)).reshape(rows, c)),
    }
    for name, (got, want) in cases.items():
        assert bits_equal(got, want, dtype), f"{name} {dtype} not bit-exact"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(9, 520), (13, 264), (6, 4104), (11, 1536)])
def test_gate_residual_tile_edges(dev, dtype, shape):
    """The row-tiled gated residual at its edges: widths that are not a whole
    number of 16-byte-vector blocks (520, 264, 4104), rows off the 4-row
    tile, batch boundaries inside a tile (offsets 0, 3, 3, 6: an empty batch,
    and rows 3-5 whose tile starts in batch 0) and rows_per_batch 5; with and
    without bias, without x, in place over x. Bit-exact with the oracle; the
    guard elements after the output stay untouched."""
    rows, c = shape
    x = storage_round(orc.randn(440 + c, shape), dtype)
    h = storage_round(orc.randn(441 + c, shape), dtype)
    gate = orc.randn(442 + c, (4, c), std=0.1)
    bias = orc.randn(443 + c, (c,), std=0.05)
    offsets = np.array([0, 3, 3, min(6, rows), rows], np.int64)
    by5 = np.array(list(range(0, rows, 5)) + [rows], np.int64)
    dx, dh, dg, db = to_dev(x, dev, dtype), to_dev(h, dev, dtype), to_dev(gate, dev), to_dev(bias, dev)
    buf = torch.full((rows * c + 256,), 7.0, dtype=dtype, device=dev)
    out = buf[: rows * c].view(rows, c)
    cases = [
        (dict(gate=dg, bias=db, offsets=to_dev(offsets, dev)), orc.gate_residual(x, h, gate, offsets, bias)),
        (dict(gate=dg, offsets=to_dev(offsets, dev)), orc.gate_residual(x, h, gate, offsets)),
        (dict(gate=dg, bias=db, rows_per_batch=5), orc.gate_residual(x, h, gate, by5, bias)),
        (dict(bias=db), orc.gate_residual(x, h, None, None, bias)),
    ]
    for kw, want in cases:
        buf.fill_(7.0)
        ops.gate_residual(dx, dh, out=out, **kw)
        assert bits_equal(out, want, dtype), f"{dtype} {shape} {sorted(kw)}"
        assert bool((buf[rows * c:] == 7).all())
    gated = orc.binop_rows(h, gate, orc.batch_broadcast_map(offsets), orc.OP_MUL)
    assert bits_equal(ops.gate_residual(None, dh, gate=dg, offsets=to_dev(offsets, dev)), gated, dtype)
    ops.gate_residual(dx, dh, gate=dg, bias=db, offsets=to_dev(offsets, dev), out=dx)   # in place
    assert bits_equal(dx, orc.gate_residual(x, h, gate, offsets, bias), dtype)


def test_dense_gate_api(dev):
    n, l, c = 2, 300, 1536
    x = orc.randn(421, (n, l, c))
    h = orc.randn(422, (n, l, c))
    g = orc.randn(423, (n, c), std=0.1)
    assert np.array_equal(host(nn._gate(to_dev(h, dev), to_dev(g, dev))), orc.gate(h, g))
    want = orc.binop_flat(x, orc.gate(h, g), orc.OP_ADD)
    assert np.array_equal(host(nn.gate_residual(to_dev(x, dev), to_dev(h, dev), to_dev(g, dev))), want)


def test_sparse_gated_residual_config4(dev):
    coords, offsets = workloads.config4()
    t = coords.shape[0]
    x = orc.randn(431, (t, 1536))
    h = orc.randn(432, (t, 1536))
    gate = orc.randn(433, (2, 1536), std=0.1)
    dco = to_dev(coords, dev)
    sx = sparse.SparseTensor(to_dev(x, dev), dco)
    sh = sparse.SparseTensor(to_dev(h, dev), dco)
    got = sparse.gated_residual(sx, sh, to_dev(gate, dev))
    assert np.array_equal(host(got.feats), orc.gate_residual(x, h, gate, offsets=offsets))
    # the reference's two-step form: x + h.elemwise_batch(gate, MUL)
    got2 = sx + sh.elemwise_batch(to_dev(gate, dev), sparse.OP_MUL)
    assert torch.equal(got2.feats, got.feats)


@pytest.mark.parametrize("dim", [256, 255, 64, 1024])
def test_timestep_embedding(dev, dim):
    rng = orc.Rng(501)
    t = rng.uniform((64,), 0.0, 1.0)
    for tt in (t, (t * np.float32(1000.0)).astype(np.float32)):  # the pipeline passes t * 1000
        got = nn.TimestepEmbedder(dim).timestep_embedding(to_dev(tt, dev))
        assert_close(got, orc.timestep_embedding(tt, dim), torch.float32, f"timestep dim={dim}")
    z = host(ops.timestep_embedding(torch.zeros(3, device=dev), dim))
    half = dim // 2
    assert np.all(z[:, :half] == 1.0) and np.all(z[:, half:] == 0.0)


def test_activation_errors(dev):
    with pytest.raises(ValueError, match="unknown activation"):
        nn.activation(torch.zeros((2, 8), device=dev), 7)
