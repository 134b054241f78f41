"""GPU parity: the MFMA weight GEMM (t2h_linear) against the C oracle's
restatement of the reference's GEMM (gpu/linear.mojo:108-160, 326-388) with
the bias add and activation of gelu_tanh_bias (662-684).

Bars:
- integer-valued operands make every product and partial sum exact, so the
  GPU's different summation order must still give the oracle's bits;
- random f16/bf16 operands: both sides sum the same exact products in f32 in
  different orders, so each output is within 2 * k * 2^-24 * sum|a w| of the
  oracle (f32 output), and within the storage bar of tests/_parity.py after
  rounding to f16/bf16.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, host, storage_round, to_dev
from t2h import ops

pytestmark = pytest.mark.gpu


def _operands(seed, m, n, k, dtype, std_w=0.02):
    a = storage_round(orc.randn(seed, (m, k)), dtype)
    w = storage_round(orc.randn(seed + 1, (n, k), std=std_w), dtype)
    return a, w


def _sum_bound(a, w):
    return 2.0 * a.shape[1] * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(w).astype(np.float64).T)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_integer_operands_bit_exact(dev, dtype):
    """Small-integer operands, ragged rows (300 = 2 token tiles + 44): every
    output equals the oracle bit for bit; pins the MFMA operand and output
    lane layouts and the tile bookkeeping."""
    rng = np.random.default_rng(11)
    m, n, k = 300, 512, 256
    a = rng.integers(-6, 7, (m, k)).astype(np.float32)
    w = rng.integers(-6, 7, (n, k)).astype(np.float32)
    out = ops.linear(to_dev(a, dev, dtype), to_dev(w, dev, dtype), out_dtype=torch.float32)
    want = orc.linear(a, w)
    assert np.array_equal(host(out), want)
    # 16-bit output (the LDS-staged row store): |sums| < 256 are exact in f16
    # and bf16 needs |sums| < 256 too, so clip the operands
    a2, w2 = np.clip(a, -2, 2), np.clip(w, -2, 2)
    out16 = ops.linear(to_dev(a2, dev, dtype), to_dev(w2, dev, dtype))
    want16 = orc.linear(a2, w2)
    assert np.abs(want16).max() < 256
    assert np.array_equal(host(out16), want16)


@pytest.mark.parametrize("out_dtype,act", [(torch.float32, None), (torch.float16, ops.ACT_RELU)])
def test_more_tiles_than_cus_bit_exact(dev, out_dtype, act):
    """66 token tiles (the last one ragged: 16740 = 65 * 256 + 100) x 7
    feature tiles = 462 tiles: more than one per CU, and a count that is not
    a multiple of 8, so the XCD deal of the tile numbers has unequal ranges.
    Integer operands and bias, |sums| <= 772, so f32 and f16 outputs (ReLU
    keeps integers) equal the oracle bit for bit."""
    rng = np.random.default_rng(23)
    m, n, k = 16740, 1792, 192
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    w = rng.integers(-2, 3, (n, k)).astype(np.float32)
    b = rng.integers(-4, 5, (n,)).astype(np.float32)
    out = ops.linear(to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16), bias=to_dev(b, dev),
                     act=ops.ACT_NONE if act is None else act, out_dtype=out_dtype)
    want = orc.linear(a, w, bias=b, act=act)
    assert out.dtype == out_dtype
    assert np.array_equal(host(out), want)


def test_long_k_tile_order_bit_exact(dev):
    """K = 4096 (64 k steps; the tile order groups 2 token tiles instead of
    4) with 3 token tiles, the last ragged: a group of 2 and a remainder of
    1. Operands in {-1, 0, 1}: exact sums, |sums| < 2048, so both the f32
    and the f16 output equal the oracle bit for bit, as does the gated
    residual join on the same GEMM."""
    rng = np.random.default_rng(29)
    m, n, k = 600, 512, 4096
    a = rng.integers(-1, 2, (m, k)).astype(np.float32)
    w = rng.integers(-1, 2, (n, k)).astype(np.float32)
    want = orc.linear(a, w)
    assert np.abs(want).max() < 2048
    ad, wd = to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16)
    assert np.array_equal(host(ops.linear(ad, wd, out_dtype=torch.float32)), want)
    assert np.array_equal(host(ops.linear(ad, wd)), want)
    res = rng.integers(-8, 9, (m, n)).astype(np.float32)
    got = ops.linear_gate_residual(ad, wd, to_dev(res, dev, torch.float32))
    assert np.array_equal(host(got), orc.gate_residual(res, want, None, None, None))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 129, 1000])
def test_random_operands_within_sum_bound(dev, dtype, m):
    n, k = 768, 1536
    a, w = _operands(1200 + m, m, n, k, dtype)
    want = orc.linear(a, w)
    got = host(ops.linear(to_dev(a, dev, dtype), to_dev(w, dev, dtype), out_dtype=torch.float32))
    assert np.all(np.abs(got - want) <= _sum_bound(a, w))
    got16 = ops.linear(to_dev(a, dev, dtype), to_dev(w, dev, dtype))
    assert got16.dtype == dtype
    assert_close(got16, storage_round(want, dtype), dtype, "linear, 16-bit output")


@pytest.mark.parametrize("act", [ops.ACT_NONE, ops.ACT_GELU_TANH, ops.ACT_SILU, ops.ACT_RELU])
def test_bias_and_activation_epilogue(dev, act):
    """out = act(fl(acc + bias)): the MLP's first linear with gelu_tanh_bias
    (and the other activations) in the GEMM's store, f16 output."""
    m, n, k = 513, 1024, 512
    a, w = _operands(1300, m, n, k, torch.float16)
    b = orc.randn(1302, (n,), std=0.02)
    out = ops.linear(to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16), bias=to_dev(b, dev), act=act)
    want = orc.linear(a, w, bias=b, act=act)
    assert_close(out, want, torch.float16, f"linear act {act}")


def test_strided_rows_and_leading_dims(dev):
    """x rows ldx > k apart (a column slice of a wider buffer) and a [B, L, k]
    input: the same numbers as the contiguous call."""
    m, n, k = 200, 256, 128
    a, w = _operands(1400, m, n, k, torch.float16)
    wide = torch.zeros((m, k + 64), dtype=torch.float16, device=dev)
    wide[:, 32:32 + k] = to_dev(a, dev, torch.float16)
    wd = to_dev(w, dev, torch.float16)
    got = ops.linear(wide[:, 32:32 + k], wd, out_dtype=torch.float32)
    ref = ops.linear(to_dev(a, dev, torch.float16), wd, out_dtype=torch.float32)
    assert torch.equal(got, ref)
    got3 = ops.linear(to_dev(a, dev, torch.float16).reshape(4, 50, k), wd, out_dtype=torch.float32)
    assert got3.shape == (4, 50, n) and torch.equal(got3.reshape(m, n), ref)
    # output rows of a wider buffer (ldo > n), 16-bit staged store
    wide_out = torch.full((m, n + 128), 7.0, dtype=torch.float16, device=dev)
    ops.linear(to_dev(a, dev, torch.float16), wd, out=wide_out[:, 64:64 + n])
    assert torch.equal(wide_out[:, 64:64 + n], ops.linear(to_dev(a, dev, torch.float16), wd))
    assert bool((wide_out[:, :64] == 7).all()) and bool((wide_out[:, 64 + n:] == 7).all())


def test_zero_rows_and_shape_errors(dev):
    w = torch.zeros((256, 64), dtype=torch.float16, device=dev)
    assert ops.linear(torch.zeros((0, 64), dtype=torch.float16, device=dev), w).shape == (0, 256)
    with pytest.raises(ValueError, match="multiple of 256"):
        ops.linear(torch.zeros((4, 64), dtype=torch.float16, device=dev),
                   torch.zeros((128, 64), dtype=torch.float16, device=dev))
    with pytest.raises(ValueError, match="in_features 40 is not a multiple of"):
        ops.linear(torch.zeros((4, 40), dtype=torch.float16, device=dev),
                   torch.zeros((256, 40), dtype=torch.float16, device=dev))
    with pytest.raises(ValueError, match="f16 or bf16"):
        ops.linear(torch.zeros((4, 64), device=dev), torch.zeros((256, 64), device=dev))


# ---- linear + gated residual join (t2h_linear_gate_residual) -------------------
def _int_case(seed, m, n, k, lo=-4, hi=5):
    rng = np.random.default_rng(seed)
    a = rng.integers(lo, hi, (m, k)).astype(np.float32)
    w = rng.integers(lo, hi, (n, k)).astype(np.float32)
    return rng, a, w


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gate_residual_integer_bit_exact(dev, dtype):
    """Exact GEMM sums (small integers), per-batch power-of-two gates over two
    ragged sparse batches, integer bias and residual: every output equals the
    oracle's gate_residual on the oracle's GEMM bit for bit, written to a
    fresh tensor and in place over the residual (the block's x += ...)."""
    m, n, k = 300, 512, 128
    rng, a, w = _int_case(21, m, n, k, -2, 3)
    bias = rng.integers(-3, 4, (n,)).astype(np.float32)
    gate = (2.0 ** rng.integers(-2, 2, (2, n))).astype(np.float32)
    res = rng.integers(-8, 9, (m, n)).astype(np.float32)
    offsets = np.array([0, 137, m], np.int64)
    want = orc.gate_residual(res, orc.linear(a, w), gate, offsets, bias)
    assert np.abs(want).max() < 256
    args = dict(bias=to_dev(bias, dev), gate=to_dev(gate, dev), offsets=to_dev(offsets, dev))
    ad, wd = to_dev(a, dev, dtype), to_dev(w, dev, dtype)
    rd = to_dev(res, dev, dtype)
    got = ops.linear_gate_residual(ad, wd, rd, **args)
    assert np.array_equal(host(got), want)
    ops.linear_gate_residual(ad, wd, rd, out=rd, **args)
    assert np.array_equal(host(rd), want)
    # f32 residual stream
    r32 = to_dev(res, dev)
    assert np.array_equal(host(ops.linear_gate_residual(ad, wd, r32, **args)), want)


def test_gate_residual_f32_stream_random(dev):
    """Random f16 operands onto an f32 residual stream (the reference's f32
    residual), per-batch gates by rows_per_batch: within the GEMM's sum bound
    times |gate| of the oracle (the rest of the join is the same f32
    roundings)."""
    m, n, k = 1000, 768, 1536
    a, w = _operands(2100, m, n, k, torch.float16)
    bias = orc.randn(2102, (n,), std=0.02)
    gate = orc.randn(2103, (4, n), std=0.1)
    res = orc.randn(2104, (m, n))
    want = orc.gate_residual(res, orc.linear(a, w), gate, np.array([0, 250, 500, 750, m], np.int64), bias)
    got = host(ops.linear_gate_residual(to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16), to_dev(res, dev),
                                        bias=to_dev(bias, dev), gate=to_dev(gate, dev), rows_per_batch=250))
    g_rows = np.repeat(np.abs(gate), 250, axis=0)
    bound = _sum_bound(a, w) * g_rows + 2.0 ** -22 * np.maximum(np.abs(want), 1.0)
    assert np.all(np.abs(got - want) <= bound)


def test_gate_residual_ungated_no_bias_f16(dev):
    """The cross join x += h + bias without a gate, and without a bias: f16
    residual, the storage tolerance of tests/_parity.py."""
    m, n, k = 513, 256, 512
    a, w = _operands(2200, m, n, k, torch.float16)
    res = storage_round(orc.randn(2201, (m, n)), torch.float16)
    bias = orc.randn(2202, (n,), std=0.02)
    ad, wd, rd = to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16), to_dev(res, dev, torch.float16)
    assert_close(ops.linear_gate_residual(ad, wd, rd, bias=to_dev(bias, dev)),
                 orc.gate_residual(res, orc.linear(a, w), None, None, bias), torch.float16, "ungated")
    assert_close(ops.linear_gate_residual(ad, wd, rd), orc.gate_residual(res, orc.linear(a, w), None), torch.float16,
                 "ungated, no bias")


@pytest.mark.parametrize("k", [64, 128, 192])
def test_one_two_three_k_steps_bit_exact(dev, k):
    """1, 2 and 3 k steps of 64 (the pipelines' prologue and tails, and the
    stage buffer the last step leaves free for the residual rows, which
    alternates with the step count): integer operands, bit-exact, for the
    linear (f32 and 16-bit out) and the gated residual (f16 and f32 streams)."""
    m, n = 300, 512
    rng, a, w = _int_case(30 + k, m, n, k, -2, 3)
    bias = rng.integers(-3, 4, (n,)).astype(np.float32)
    ad, wd = to_dev(a, dev, torch.float16), to_dev(w, dev, torch.float16)
    want = orc.linear(a, w, bias=bias)
    assert np.abs(want).max() < 256
    assert np.array_equal(host(ops.linear(ad, wd, bias=to_dev(bias, dev), out_dtype=torch.float32)), want)
    assert np.array_equal(host(ops.linear(ad, wd, bias=to_dev(bias, dev))), want)
    gate = (2.0 ** rng.integers(-2, 2, (1, n))).astype(np.float32)
    res = rng.integers(-8, 9, (m, n)).astype(np.float32)
    offsets = np.array([0, m], np.int64)
    want_r = orc.gate_residual(res, orc.linear(a, w), gate, offsets, bias)
    assert np.abs(want_r).max() < 256
    args = dict(bias=to_dev(bias, dev), gate=to_dev(gate, dev), offsets=to_dev(offsets, dev))
    assert np.array_equal(host(ops.linear_gate_residual(ad, wd, to_dev(res, dev, torch.float16), **args)), want_r)
    assert np.array_equal(host(ops.linear_gate_residual(ad, wd, to_dev(res, dev), **args)), want_r)


# ---- the reference GPU linear test's geometries ------------------------------
# tests/parity/parity_wp11_gpu_linear.mojo:105-111: rows, out_features,
# in_features, bias, and that test's absolute bar for the case.
REF_SHAPES = [
    (4096, 3072, 1024, True, 2e-4),
    (1029, 1024, 1024, True, 2e-4),
    (2369, 4096, 1024, True, 2e-4),
    (2369, 1024, 4096, True, 4e-4),
    (600, 6144, 1024, False, 2e-4),
]


def _ref_fill(seed, shape, scale):
    """Operands distributed as the reference test's fill
    (parity_wp11_gpu_linear.mojo:33-50): uniform in [-scale, scale)."""
    return np.random.default_rng(seed).uniform(-scale, scale, shape).astype(np.float32)


def _ref_case(seed, rows, co, ci, dtype, w_scale=0.03, b_scale=0.5):
    """make_case (parity_wp11_gpu_linear.mojo:43-50) with x and w stored in
    `dtype`, the way a 16-bit checkpoint and a 16-bit activation arrive."""
    a = storage_round(_ref_fill(seed, (rows, ci), 1.0), dtype)
    w = storage_round(_ref_fill(seed + 1, (co, ci), w_scale), dtype)
    return a, w, _ref_fill(seed + 2, (co,), b_scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(REF_SHAPES)))
def test_reference_linear_shapes(dev, dtype, case):
    """DiT qkv / out / mlp / adaLN GEMMs at the reference test's shapes, odd
    token counts (ragged last token tile) and k = 4096 among them: the f32
    output is within the reference test's absolute bar of the oracle on the
    same 16-bit operands, and within the summation-order bound."""
    rows, co, ci, has_bias, atol = REF_SHAPES[case]
    a, w, b = _ref_case(11 + case, rows, co, ci, dtype)
    bias = b if has_bias else None
    want = orc.linear(a, w, bias=bias)
    got = host(ops.linear(to_dev(a, dev, dtype), to_dev(w, dev, dtype),
                          bias=to_dev(b, dev) if has_bias else None, out_dtype=torch.float32))
    err = np.abs(got - want)
    assert err.max() <= atol, f"{rows}x{co}x{ci}: max |diff| {err.max():.3e} > {atol:g}"
    assert np.all(err <= _sum_bound(a, w) + 2.0 ** -23 * np.abs(want))


def test_reference_linear_3d_input(dev):
    """A [1, 1500, 1024] dense-DiT activation to 3072 features
    (parity_wp11_gpu_linear.mojo:113-126): output [1, 1500, 3072] within
    2e-4 of the oracle."""
    a, w, b = _ref_case(21, 1500, 3072, 1024, torch.float16)
    got = ops.linear(to_dev(a, dev, torch.float16).reshape(1, 1500, 1024), to_dev(w, dev, torch.float16),
                     bias=to_dev(b, dev), out_dtype=torch.float32)
    assert got.shape == (1, 1500, 3072)
    assert np.abs(host(got).reshape(1500, 3072) - orc.linear(a, w, bias=b)).max() <= 2e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_mlp_chain(dev, dtype):
    """The feed-forward chain lin2(gelu_tanh(lin0(x))) at 1500 x 1024 -> 4096
    -> 1024 (parity_wp11_gpu_linear.mojo:166-194): the first GEMM's bias and
    GELU in its store, the 4096-wide hidden stored in `dtype`, the second GEMM
    with its bias; within the reference test's 5e-4 of the oracle's chain
    (which rounds the hidden to `dtype` the same way)."""
    rows, ci, hid = 1500, 1024, 4096
    x = storage_round(_ref_fill(91, (rows, ci), 1.0), dtype)
    w0 = storage_round(_ref_fill(92, (hid, ci), 0.03), dtype)
    b0 = _ref_fill(93, (hid,), 0.1)
    w2 = storage_round(_ref_fill(94, (ci, hid), 0.015), dtype)
    b2 = _ref_fill(95, (ci,), 0.1)
    mid = ops.linear(to_dev(x, dev, dtype), to_dev(w0, dev, dtype), bias=to_dev(b0, dev), act=ops.ACT_GELU_TANH)
    assert mid.dtype == dtype
    got = host(ops.linear(mid, to_dev(w2, dev, dtype), bias=to_dev(b2, dev), out_dtype=torch.float32))
    want_mid = orc.linear(x, w0, bias=b0, act=ops.ACT_GELU_TANH)
    assert_close(mid, storage_round(want_mid, dtype), dtype, "mlp hidden")
    want = orc.linear(storage_round(want_mid, dtype), w2, bias=b2)
    assert np.abs(got - want).max() <= 5e-4
