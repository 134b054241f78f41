"""GPU parity: LayerNorm + adaLN modulate (dense and batch-gathered) and the
fused gated-residual + LayerNorm join, through the C ABI, against the C oracle
(modules/nn.mojo:314-369, 660-689; sparse/transformer/modulated.mojo:60-65;
gpu/block.mojo:47-110). Metric and tolerances: tests/_parity.py."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import TOL, assert_close, bits_equal, host, max_err, storage_round, to_dev
from t2h import nn, ops, sparse, workloads

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def test_config1_ln_modulate_f32(dev):
    """fp32 x[4096,1536], shift/scale [1536] ~ N(0, 0.1), eps 1e-6."""
    x = orc.randn(101, (4096, 1536))
    shift = orc.randn(102, (1536,), std=0.1)
    scale = orc.randn(103, (1536,), std=0.1)
    want = orc.ln_modulate(x, shift, scale, eps=1e-6)
    got = ops.ln_modulate(to_dev(x, dev), 1e-6, shift=to_dev(shift, dev), scale=to_dev(scale, dev))
    assert_close(got, want, torch.float32, "config1 LN+modulate")
    # the Mojo-shaped API: modulate(norm1(x), shift, scale) over [N, L, C]
    norm = nn.LayerNorm32(1536, 1e-6, affine=False)
    x3 = to_dev(x.reshape(1, 4096, 1536), dev)
    got2 = nn.modulate(norm.forward(x3), to_dev(shift.reshape(1, 1536), dev), to_dev(scale.reshape(1, 1536), dev))
    assert_close(got2.reshape(4096, 1536), want, torch.float32, "LayerNorm32 + modulate")
    fused = nn.layernorm_modulate(norm, x3, to_dev(shift.reshape(1, 1536), dev), to_dev(scale.reshape(1, 1536), dev))
    assert torch.equal(fused, got2), "fused LN+modulate differs from LN then modulate"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cols", [1536, 1024, 2048, 512, 256, 3072])
def test_ln_modulate_widths(dev, dtype, cols):
    rows = 777
    x = orc.randn(200 + cols, (rows, cols), std=3.0, mean=0.5)
    xs = storage_round(x, dtype)
    shift = orc.randn(201, (cols,), std=0.1)
    scale = orc.randn(202, (cols,), std=0.1)
    got = ops.ln_modulate(to_dev(x, dev, dtype), 1e-6, shift=to_dev(shift, dev), scale=to_dev(scale, dev))
    assert got.dtype == dtype
    assert_close(got, orc.ln_modulate(xs, shift, scale, eps=1e-6), dtype, f"LN+mod {dtype} C={cols}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cols", [1, 3, 100, 1000, 1537, 4160])
def test_ln_generic_widths(dev, dtype, cols):
    """Widths that are not a multiple of one wave's 16-byte lanes use the
    block-per-row kernel."""
    rows = 97
    x = orc.randn(300 + cols, (rows, cols))
    xs = storage_round(x, dtype)
    w = orc.randn(301, (cols,), mean=1.0, std=0.2)
    b = orc.randn(302, (cols,), std=0.2)
    got = ops.ln_modulate(to_dev(x, dev, dtype), 1e-5, weight=to_dev(w, dev), bias=to_dev(b, dev))
    assert_close(got, orc.layernorm(xs, 1e-5, True, w, b), dtype, f"affine LN {dtype} C={cols}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_ln_plain_and_affine(dev, dtype):
    x = orc.randn(401, (1000, 1536), std=2.0)
    xs = storage_round(x, dtype)
    for eps in (1e-5, 1e-6):
        got = nn.LayerNorm32(1536, eps, affine=False).forward(to_dev(x, dev, dtype))
        assert_close(got, orc.layernorm(xs, eps), dtype, f"plain LN eps={eps}")
    norm = nn.LayerNorm32(1536, 1e-6, affine=True)
    norm.weight = to_dev(orc.randn(402, (1536,), mean=1.0, std=0.1), dev)
    norm.bias = to_dev(orc.randn(403, (1536,), std=0.1), dev)
    got = norm.forward(to_dev(x, dev, dtype))
    want = orc.layernorm(xs, 1e-6, True, host(norm.weight), host(norm.bias))
    assert_close(got, want, dtype, "affine LN (norm2)")


def test_ln_closed_forms(dev):
    """Constant rows normalise to exactly 0; a row with variance v maps to
    (x - mean)/sqrt(v + eps)."""
    x = np.full((8, 1536), 3.25, np.float32)
    got = host(ops.ln_modulate(to_dev(x, dev), 1e-6))
    assert np.all(got == 0.0)
    x = np.tile(np.array([1.0, -1.0], np.float32), (4, 768))
    got = host(ops.ln_modulate(to_dev(x, dev), 1e-6))
    np.testing.assert_allclose(got, x / np.sqrt(1.0 + 1e-6), rtol=1e-6)


def test_ln_dense_batch_broadcast(dev):
    """modulate over [N, L, C] with shift/scale [N, C] (rows_per_batch = L)."""
    n, l, c = 3, 50, 1536
    x = orc.randn(501, (n, l, c))
    shift = orc.randn(502, (n, c), std=0.1)
    scale = orc.randn(503, (n, c), std=0.1)
    want = orc.modulate(orc.layernorm(x.reshape(-1, c), 1e-6).reshape(n, l, c), shift, scale)
    norm = nn.LayerNorm32(c, 1e-6, affine=False)
    got = nn.layernorm_modulate(norm, to_dev(x, dev), to_dev(shift, dev), to_dev(scale, dev))
    assert_close(got, want, torch.float32, "dense batched LN+mod")
    got2 = nn.modulate(to_dev(orc.layernorm(x.reshape(-1, c), 1e-6).reshape(n, l, c), dev), to_dev(shift, dev),
                       to_dev(scale, dev))
    assert np.array_equal(host(got2), want), "modulate must be bit-exact"


def test_config4_sparse_ln_modulate(dev):
    """ragged B=2 shells on 64^3, fp32 feats [T,1536],
    LN + per-batch modulate gathered by batch id."""
    coords, offsets = workloads.config4()
    t = coords.shape[0]
    feats = orc.randn(601, (t, 1536))
    shift = orc.randn(602, (2, 1536), std=0.1)
    scale = orc.randn(603, (2, 1536), std=0.1)
    st = sparse.SparseTensor(to_dev(feats, dev), to_dev(coords, dev))
    assert np.array_equal(host(st.offsets).astype(np.int64), orc.cal_offsets(coords, 2)), "offsets must be bit-exact"
    want = orc.ln_modulate(feats, shift, scale, offsets=offsets, eps=1e-6)
    got = sparse.norm_mod_shift_scale(st, 1e-6, to_dev(shift, dev), to_dev(scale, dev))
    assert_close(got.feats, want, torch.float32, "config4 sparse LN+mod")
    # unfused: norm1 then _mod_shift_scale, bit-exact gather
    n = orc.layernorm(feats, 1e-6)
    got2 = sparse._mod_shift_scale(st.replace(to_dev(n, dev)), to_dev(shift, dev), to_dev(scale, dev))
    assert np.array_equal(host(got2.feats), orc.mod_shift_scale(n, shift, scale, offsets))


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_join_ln(dev, dtype):
    """x_out = x + (h + bias) * gate; y = LN(x_out)*(1+scale)+shift in one pass
    equals the two-kernel sequence bit for bit, and the oracle to tolerance."""
    rows, c = 1234, 1536
    x = storage_round(orc.randn(701, (rows, c)), dtype)
    h = storage_round(orc.randn(702, (rows, c)), dtype)
    bias = orc.randn(703, (c,), std=0.05)
    gate = orc.randn(704, (c,), std=0.1)
    shift = orc.randn(705, (c,), std=0.1)
    scale = orc.randn(706, (c,), std=0.1)
    dx, dh = to_dev(x, dev, dtype), to_dev(h, dev, dtype)
    db, dg, ds, dc = (to_dev(a, dev) for a in (bias, gate, shift, scale))
    xo, yo = ops.gate_residual_ln_modulate(dx, dh, gate=dg, bias=db, eps=1e-6, shift=ds, scale=dc)
    x_ref = ops.gate_residual(dx, dh, gate=dg, bias=db)
    y_ref = ops.ln_modulate(x_ref, 1e-6, shift=ds, scale=dc)
    assert torch.equal(xo, x_ref), "fused join x_out differs from gate_residual"
    assert torch.equal(yo, y_ref), "fused join y_out differs from ln_modulate(gate_residual)"
    xo_want = orc.gate_residual(x, h, gate, bias=bias)
    assert bits_equal(xo, xo_want, dtype), "joined residual must equal the oracle rounded once"
    y_want = orc.ln_modulate(storage_round(xo_want, dtype), shift, scale, eps=1e-6)
    assert_close(yo, y_want, dtype, "fused join LN+mod")


def test_fused_join_sparse_and_affine(dev):
    coords, offsets = workloads.config4()
    t = coords.shape[0]
    x = orc.randn(801, (t, 1536))
    h = orc.randn(802, (t, 1536))
    gate = orc.randn(803, (2, 1536), std=0.1)
    shift = orc.randn(804, (2, 1536), std=0.1)
    scale = orc.randn(805, (2, 1536), std=0.1)
    off = to_dev(offsets, dev)
    xo, yo = ops.gate_residual_ln_modulate(to_dev(x, dev), to_dev(h, dev), gate=to_dev(gate, dev), eps=1e-6,
                                           shift=to_dev(shift, dev), scale=to_dev(scale, dev), offsets=off)
    xw = orc.gate_residual(x, h, gate, offsets=offsets)
    assert np.array_equal(host(xo), xw)
    assert_close(yo, orc.ln_modulate(xw, shift, scale, offsets=offsets, eps=1e-6), torch.float32, "sparse join")
    # norm2 (affine) after an ungated residual: gpu/block.mojo:339-367
    w = orc.randn(806, (1536,), mean=1.0, std=0.1)
    b = orc.randn(807, (1536,), std=0.1)
    xo2, yo2 = ops.gate_residual_ln_modulate(to_dev(x, dev), to_dev(h, dev), eps=1e-6, weight=to_dev(w, dev),
                                             norm_bias=to_dev(b, dev))
    xw2 = orc.binop_flat(x, h, orc.OP_ADD)
    assert np.array_equal(host(xo2), xw2)
    assert_close(yo2, orc.layernorm(xw2, 1e-6, True, w, b), torch.float32, "ungated join + affine LN")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_fused_gated_join_affine_multibatch(dev, dtype):
    """The block's self join + norm2: per-batch gate with an affine norm over
    config-4 rows, whose batch boundary (row 19,838) falls inside an 8-row
    block, so one block mixes batches (the per-batch gate row is read per
    row; the affine weight/bias are per channel)."""
    coords, offsets = workloads.config4()
    assert offsets[1] % 8 != 0
    t = coords.shape[0]
    x = storage_round(orc.randn(811, (t, 1536)), dtype)
    h = storage_round(orc.randn(812, (t, 1536)), dtype)
    gate = orc.randn(813, (2, 1536), std=0.5)
    w = orc.randn(814, (1536,), mean=1.0, std=0.1)
    b = orc.randn(815, (1536,), std=0.1)
    xo, yo = ops.gate_residual_ln_modulate(to_dev(x, dev, dtype), to_dev(h, dev, dtype), gate=to_dev(gate, dev),
                                           eps=1e-6, weight=to_dev(w, dev), norm_bias=to_dev(b, dev),
                                           offsets=to_dev(offsets, dev))
    xw = storage_round(orc.gate_residual(x, h, gate, offsets=offsets), dtype)
    assert bits_equal(xo, xw, dtype)
    assert_close(yo, orc.layernorm(xw, 1e-6, True, w, b), dtype, f"gated join + affine LN {dtype}")


@pytest.mark.parametrize("in_place", [False, True])
@pytest.mark.parametrize("cols", [1, 100, 1000, 1280, 1536, 1537])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_fused_join_generic_widths(dev, dtype, cols, in_place):
    """The fused join + LN at widths off the one-wave-per-row fast path (all
    but 1536; f32 1280 is 5 vectors per lane, which has no fast variant),
    with x_out a separate tensor or x itself (x_out may alias x). The stored
    residual must equal the oracle's rounded once, and the LN must read it,
    not x + gate*h recomputed over an already updated x."""
    rows = 37
    x = storage_round(orc.randn(3000 + cols, (rows, cols)), dtype)
    h = storage_round(orc.randn(3001, (rows, cols)), dtype)
    bias = orc.randn(3002, (cols,), std=0.05)
    gate = orc.randn(3003, (cols,), std=0.5)
    shift = orc.randn(3004, (cols,), std=0.1)
    scale = orc.randn(3005, (cols,), std=0.1)
    dx, dh = to_dev(x, dev, dtype), to_dev(h, dev, dtype)
    db, dg, ds, dc = (to_dev(a, dev) for a in (bias, gate, shift, scale))
    xo, yo = ops.gate_residual_ln_modulate(dx, dh, gate=dg, bias=db, eps=1e-6, shift=ds, scale=dc,
                                           x_out=dx if in_place else None)
    assert (xo.data_ptr() == dx.data_ptr()) == in_place
    xw = storage_round(orc.gate_residual(x, h, gate, bias=bias), dtype)
    assert bits_equal(xo, xw, dtype), f"joined residual, cols {cols}"
    assert_close(yo, orc.ln_modulate(xw, shift, scale, eps=1e-6), dtype, f"join LN+mod cols {cols} in_place {in_place}")


@pytest.mark.parametrize("cols", [100, 1000, 1280, 1536])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_block_join_ln_generic_widths(dev, dtype, cols):
    """t2h_block_join_ln always updates x in place (gpu/block.mojo:324-349,
    356-381): gated join + modulated norm and ungated join + affine norm over
    the 12*C const buffer, at fast and generic widths."""
    from t2h import block

    rows = 29
    x = storage_round(orc.randn(3100, (rows, cols)), dtype)
    h = storage_round(orc.randn(3101, (rows, cols)), dtype)
    m = [orc.randn(3102 + i, (1, cols), std=0.1) for i in range(6)]
    w2 = orc.randn(3108, (cols,), mean=1.0, std=0.1)
    b2 = orc.randn(3109, (cols,), std=0.05)
    biases = [orc.randn(3110 + i, (cols,), std=0.02) for i in range(3)]
    bk = block.pack_block_consts([to_dev(mm, dev) for mm in m], to_dev(w2, dev), to_dev(b2, dev),
                                 *[to_dev(b, dev) for b in biases])
    v = lambda k: host(bk)[k * cols:(k + 1) * cols]
    # self join (bias 2C, gate 3C) + norm2 affine (4C, 5C)
    dx = to_dev(x, dev, dtype)
    dst = torch.empty_like(dx)
    ops.block_join_ln(dx, to_dev(h, dev, dtype), dst, bk, 2 * cols, 1, 4 * cols, 2)
    xw = storage_round(orc.gate_residual(x, h, v(3), bias=v(2)), dtype)
    assert bits_equal(dx, xw, dtype), f"gated join cols {cols}"
    assert_close(dst, orc.layernorm(xw, 1e-6, True, v(4), v(5)), dtype, f"join + affine LN cols {cols}")
    # cross join (bias 6C, ungated) + norm3 modulate (8C, 9C)
    dx = to_dev(x, dev, dtype)
    ops.block_join_ln(dx, to_dev(h, dev, dtype), dst, bk, 6 * cols, 0, 8 * cols, 1)
    xw = storage_round(orc.gate_residual(x, h, None, bias=v(6)), dtype)
    assert bits_equal(dx, xw, dtype), f"ungated join cols {cols}"
    assert_close(dst, orc.ln_modulate(xw, v(8), v(9), eps=1e-6), dtype, f"join + LN mod cols {cols}")


def test_modulation_chunk_views(dev):
    """Modulation.chunks (share_mod) -> six strided [B, C] views read in place."""
    b, c = 2, 1536
    mod = orc.randn(901, (b, 6 * c), std=0.5)
    modulation = orc.randn(902, (6 * c,), std=0.5)
    m_want = orc.modulation_add(mod, modulation)
    chunks = sparse.Modulation(to_dev(modulation, dev)).chunks(to_dev(mod, dev), c)
    assert np.array_equal(host(torch.cat(chunks, 1)), m_want)
    coords, offsets = workloads.config4()
    x = orc.randn(903, (coords.shape[0], c))
    got = ops.ln_modulate(to_dev(x, dev), 1e-6, shift=chunks[0], scale=chunks[1], offsets=to_dev(offsets, dev))
    want = orc.ln_modulate(x, m_want[:, :c], m_want[:, c:2 * c], offsets=offsets, eps=1e-6)
    assert_close(got, want, torch.float32, "LN+mod from strided chunks")


def test_modulation_linear_path(dev):
    """Modulation.chunks without share_mod: lin(SiLU(mod)) (modulated.mojo:49-50),
    the linear a stand-in the device and numpy compute identically
    (an exact power-of-two scale and a column roll)."""
    b, c = 3, 256
    mod = orc.randn(911, (b, c), std=2.0)
    lin = lambda h: torch.roll(h.repeat(1, 6), 1, dims=1) * 0.5
    chunks = sparse.Modulation(lin=lin).chunks(to_dev(mod, dev), c)
    silu = orc.activation(mod, orc.ACT_SILU)
    want = (np.roll(np.tile(silu, (1, 6)), 1, axis=1) * np.float32(0.5)).astype(np.float32)
    assert_close(torch.cat(chunks, 1), want, torch.float32, "lin(SiLU(mod)) chunks")
    with pytest.raises(ValueError, match="not both"):
        sparse.Modulation()


def test_in_place_and_empty(dev):
    x = orc.randn(1001, (64, 1536))
    d = to_dev(x, dev)
    ops.ln_modulate(d, 1e-6, out=d)
    assert_close(d, orc.layernorm(x, 1e-6), torch.float32, "in-place LN")
    e = torch.empty((0, 1536), device=dev)
    assert ops.ln_modulate(e, 1e-6).shape == (0, 1536)


def test_ln_errors(dev):
    norm = nn.LayerNorm32(1536, 1e-6, affine=False)
    with pytest.raises(ValueError, match="last dim mismatch"):
        norm.forward(torch.zeros((4, 1024), device=dev))
    with pytest.raises(ValueError, match="shift/scale shape mismatch"):
        nn.modulate(torch.zeros((1, 4, 1536), device=dev), torch.zeros(1024, device=dev),
                    torch.zeros(1536, device=dev))


def test_deterministic(dev):
    x = to_dev(orc.randn(1101, (3000, 1536)), dev)
    a = ops.ln_modulate(x, 1e-6)
    b = ops.ln_modulate(x, 1e-6)
    assert torch.equal(a, b)
