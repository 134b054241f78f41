"""GPU: non-finite inputs (NaN, +-inf, f32 overflow) propagate as in the
reference's f32 arithmetic, checked against the C oracle. The oracle is the
reference's CPU code restated in C with IEEE f32 semantics (no fast-math),
so its NaN / inf positions are the reference's:
- LayerNorm (modules/nn.mojo:314-369): a row with a NaN, or with +inf and
  -inf, is NaN throughout; a row with one +inf is NaN (inf - inf in the
  centring); a row whose squares overflow has variance inf, so its normalised
  values are 0 and the output is the shift.
- MultiHeadRMSNorm (sparse/attention/modules.mojo:75-95): `if norm < 1e-12`
  is false for a NaN norm, so a head with a NaN is NaN throughout; an inf
  element gives norm inf, finite elements / inf = 0 and inf / inf = NaN; the
  RoPE rotation then mixes each pair (re*c - im*s).
- GELU-tanh (nn.mojo:576-579): +inf -> +inf, -inf -> NaN (-inf * 0),
  NaN -> NaN, and the f32 overflow of v^3 saturates.
- The gated residual (modulated.mojo:22-33): IEEE adds and multiplies.
The comparison: identical NaN / +inf / -inf masks, and the finite values to
the op's usual bar (err = |got - want| / max(|want|, 1), bit-exact for the
gated residual)."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import TOL, host, storage_round, to_dev
from t2h import ops

pytestmark = pytest.mark.gpu


def same_nonfinite(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, what
    for name, f in (("NaN", np.isnan), ("+inf", np.isposinf), ("-inf", np.isneginf)):
        g, w = f(got), f(want)
        assert np.array_equal(g, w), f"{what}: {name} at {np.argwhere(g != w)[:4].tolist()}"
    return np.isfinite(want)


def close_where_finite(got, want, tol, what):
    fin = same_nonfinite(got, want, what)
    g = np.asarray(got, np.float64)[fin]
    w = np.asarray(want, np.float64)[fin]
    e = float(np.max(np.abs(g - w) / np.maximum(np.abs(w), 1.0))) if g.size else 0.0
    assert e <= tol, f"{what}: finite values max err {e:.3e} > {tol}"
    return int(fin.size - fin.sum())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_layernorm_modulate_nonfinite_rows(dev, dtype):
    rows, c = 16, 1536
    x = orc.randn(901, (rows, c))
    x[2, 5] = np.nan
    x[4, 100] = np.inf
    x[6, 7] = -np.inf
    x[8, 9], x[8, 10] = np.inf, -np.inf
    if dtype == torch.float32:
        x[10, 0] = 3e38   # (x - mean)^2 overflows: variance inf, normalised values 0
    shift = orc.randn(902, (c,), std=0.1)
    scale = orc.randn(903, (c,), std=0.1)
    xin = storage_round(x, dtype)
    want = storage_round(orc.ln_modulate(xin, shift, scale, eps=1e-6), dtype)
    got = host(ops.ln_modulate(to_dev(x, dev, dtype), 1e-6, shift=to_dev(shift, dev), scale=to_dev(scale, dev)))
    n = close_where_finite(got, want, TOL[dtype], "LN + modulate")
    assert n == 4 * c   # rows 2, 4, 6, 8
    if dtype == torch.float32:
        assert np.array_equal(got[10], want[10])
        assert np.array_equal(want[10], storage_round(shift, dtype))   # the shift alone
    finite_rows = [r for r in range(rows) if r not in (2, 4, 6, 8, 10)]
    assert np.all(np.isfinite(got[finite_rows]))


def test_qk_rmsnorm_rope_nonfinite_heads(dev):
    rows, h, d = 8, 12, 128
    q = orc.randn(911, (rows, h, d))
    k = orc.randn(912, (rows, h, d))
    q[1, 3, 5] = np.nan
    q[2, 0, :] = 0.0            # zero head: the 1e-12 clamp keeps it 0
    q[3, 7, 9] = np.inf
    k[4, 2, 0] = -np.inf
    k[5, 11, 127] = np.inf
    gq = orc.randn(913, (h, d), mean=1.0, std=0.02)
    gk = orc.randn(914, (h, d), mean=1.0, std=0.02)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = orc.Rng(915).uniform((rows, 3), 0.0, 64.0).astype(np.int32)
    freqs = orc.rope_freqs(d)
    phases = orc.rope_phases_from_coords(coords, d, freqs)
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    gq_out, gk_out = ops.qk_rmsnorm_rope(q=to_dev(q, dev), k=to_dev(k, dev), gamma_q=to_dev(gq, dev),
                                         gamma_k=to_dev(gk, dev), freqs=freqs, coords=to_dev(coords, dev))
    nq = close_where_finite(host(gq_out), wq, TOL[torch.float32], "q")
    nk = close_where_finite(host(gk_out), wk, TOL[torch.float32], "k")
    assert np.all(np.isnan(wq[1, 3]))                     # NaN head: NaN throughout
    assert np.all(host(gq_out)[2, 0] == 0.0)              # zero head stays 0
    assert nq == d + 2 and nk == 2 * 2                    # inf: its RoPE pair only
    assert np.all(np.isfinite(wq[[0, 4, 5, 6, 7]])) and np.all(np.isfinite(wk[[0, 1, 2, 3, 6, 7]]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_gelu_tanh_bias_nonfinite(dev, dtype):
    specials = [np.nan, np.inf, -np.inf, 0.0, -0.0, 20.0, -20.0, 88.0, -88.0]
    if dtype == torch.float32:
        specials += [1e30, -1e30, 3e38, -3e38]   # v^3 overflows f32
    else:
        specials += [65504.0, -65504.0]
    rows, c = 4, 1024
    x = orc.randn(921, (rows, c))
    x[0, :len(specials)] = specials
    x[3, -len(specials):] = specials
    bias = orc.randn(922, (c,), std=0.02)
    bias[:len(specials)] = 0.0
    bias[-len(specials):] = 0.0
    xin = storage_round(x, dtype)
    want = storage_round(orc.gelu_tanh_bias(xin, bias), dtype)
    got = host(ops.activation(to_dev(x, dev, dtype), ops.ACT_GELU_TANH, bias=to_dev(bias, dev)))
    n = close_where_finite(got, want, TOL[dtype], "GELU-tanh + bias")
    assert n == 2 * 3            # NaN, +inf, -inf (-> NaN) in two rows
    assert np.isposinf(got[0, 1]) and np.isnan(got[0, 2])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_gated_residual_nonfinite(dev, dtype):
    rows, c = 8, 1536
    x = orc.randn(931, (rows, c))
    h = orc.randn(932, (rows, c))
    gate = orc.randn(933, (c,), std=0.1)
    x[0, :4] = [np.inf, -np.inf, np.nan, np.inf]
    h[0, :4] = [-np.inf, 1.0, 1.0, 2.0]
    h[1, :3] = [np.inf, -np.inf, np.nan]
    gate[5] = 0.0
    h[2, 5] = np.inf             # inf * 0 gate = NaN
    gate[6] = np.inf
    xin, hin = storage_round(x, dtype), storage_round(h, dtype)
    want = storage_round(orc.gate_residual(xin, hin, gate), dtype)
    got = host(ops.gate_residual(to_dev(x, dev, dtype), to_dev(h, dev, dtype), gate=to_dev(gate, dev)))
    fin = same_nonfinite(got, want, "gated residual")
    assert np.array_equal(got[fin].view(np.int32), want[fin].view(np.int32))   # finite values bit for bit
    assert np.isnan(got[0, 0]) and np.isneginf(got[0, 1]) and np.isnan(got[2, 5])
