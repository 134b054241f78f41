"""GPU parity of the host-pointer wrappers (t2h_h_*), called through ctypes
with numpy buffers exactly as the reference's unchanged Tensor[F32] APIs
would call them: LayerNorm32.forward / modulate / _mod_shift_scale
(modules/nn.mojo:314-369, 660-689; sparse/transformer/modulated.mojo:60-65),
MultiHeadRMSNorm + SparseRotaryPositionEmbedder.embed
(sparse/attention/modules.mojo:49-102, sparse/attention/rope.mojo:128-134),
activation after a linear (modules/nn.mojo:588-647), y + _gate(h, g)
(modules/transformer/modulated.mojo:22-33, 60-69), TimestepEmbedder
(models/sparse_structure_flow.mojo:60-76) and SparseTensor._cal_offsets
(sparse/basic.mojo:321-339). Metric and tolerances: tests/_parity.py.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close
from t2h import _lib, workloads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L(dev):
    return _lib.load()


def _p(a):
    return None if a is None else a.ctypes.data


def test_h_ln_modulate_sparse(L):
    """_mod_shift_scale(norm1(h)) on config-4 rows: host offsets, [2, C] chunks."""
    coords, offsets = workloads.config4()
    t, c = coords.shape[0], 1536
    x = orc.randn(4000, (t, c))
    shift, scale = orc.randn(4001, (2, c), std=0.1), orc.randn(4002, (2, c), std=0.1)
    out = np.empty_like(x)
    rc = L.t2h_h_ln_modulate(_p(x), _p(out), t, c, ctypes.c_float(1e-6), _lib.LN_MODULATE, _p(shift), _p(scale),
                             _p(offsets), 2, 0)
    assert rc == 0, L.t2h_last_error()
    assert_close(out, orc.ln_modulate(x, shift, scale, offsets, 1e-6), torch.float32, "t2h_h_ln_modulate")


def test_h_qk_rmsnorm_rope_coords(L):
    """MultiHeadRMSNorm then the sparse RoPE from int coords, host buffers."""
    coords, _ = workloads.config4()
    coords = np.ascontiguousarray(coords[:5000])
    t, h, d = coords.shape[0], 12, 128
    q, k = orc.randn(4100, (t, h, d)), orc.randn(4101, (t, h, d))
    gq, gk = orc.randn(4102, (h, d), mean=1.0, std=0.02), orc.randn(4103, (h, d), mean=1.0, std=0.02)
    freqs = orc.rope_freqs(d)
    qo, ko = np.empty_like(q), np.empty_like(k)
    rc = L.t2h_h_qk_rmsnorm_rope(_p(q), _p(k), _p(qo), _p(ko), t, h, d, _p(gq), _p(gk), 1, _p(freqs), freqs.size,
                                 3, None, 0, _p(coords), 4, 0)
    assert rc == 0, L.t2h_last_error()
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, orc.rope_phases_from_coords(coords, d, freqs))
    assert_close(qo, wq, torch.float32, "host q")
    assert_close(ko, wk, torch.float32, "host k")


@pytest.mark.parametrize("kind", [orc.ACT_RELU, orc.ACT_SILU, orc.ACT_GELU, orc.ACT_GELU_TANH])
def test_h_activation_with_bias(L, kind):
    x = orc.randn(4200 + kind, (333, 6144), std=2.0)
    bias = orc.randn(4210, (6144,), std=0.1)
    out = np.empty_like(x)
    rc = L.t2h_h_activation(_p(x), _p(out), _p(bias), 333, 6144, kind)
    assert rc == 0, L.t2h_last_error()
    assert_close(out, orc.activation(orc.add_bias(x, bias), kind), torch.float32, f"t2h_h_activation {kind}")


def test_h_gate_residual_dense_batches(L):
    """y + _gate(h, g) over [N, L, C] with N = 3: gate rows by r / L; bit-exact."""
    n, l, c = 3, 500, 1536
    x, hh = orc.randn(4300, (n * l, c)), orc.randn(4301, (n * l, c))
    g = orc.randn(4302, (n, c), std=0.1)
    out = np.empty_like(x)
    rc = L.t2h_h_gate_residual(_p(x), _p(hh), _p(out), None, _p(g), n * l, c, None, n, l)
    assert rc == 0, L.t2h_last_error()
    want = orc.binop_flat(x.reshape(n, l, c), orc.gate(hh.reshape(n, l, c), g), orc.OP_ADD).reshape(n * l, c)
    assert np.array_equal(out, want)


def test_h_timestep_embedding(L):
    t = (orc.Rng(4400).uniform((7,)) * 1000.0).astype(np.float32)
    out = np.empty((7, 256), np.float32)
    rc = L.t2h_h_timestep_embedding(_p(t), _p(out), 7, 256, 10000.0)
    assert rc == 0, L.t2h_last_error()
    assert_close(out, orc.timestep_embedding(t, 256), torch.float32, "t2h_h_timestep_embedding")


def test_h_wrappers_reject_bad_shapes(L):
    x = np.zeros((4, 8), np.float32)
    assert L.t2h_h_activation(_p(x), _p(x), None, 4, 8, 9) == _lib.T2H_EINVAL
    assert L.t2h_h_gate_residual(_p(x), _p(x), _p(x), None, None, -1, 8, None, 1, 0) == _lib.T2H_EINVAL
    assert L.t2h_h_timestep_embedding(_p(x), _p(x), 4, 0, 10000.0) == _lib.T2H_EINVAL
    rc = L.t2h_h_qk_rmsnorm_rope(_p(x), None, _p(x), None, 4, 1, 7, None, None, 0, None, 0, 3, None, 0, None, 0, 0)
    assert rc == _lib.T2H_EINVAL and b"even" in L.t2h_last_error()
