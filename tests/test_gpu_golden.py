"""GPU kernels against the committed golden fixtures (tests/golden/
oracle_golden.npz): the same inputs and oracle outputs pinned on the CPU.
Metric and tolerances: tests/_parity.py."""
import os

import numpy as np
import pytest
import torch

from _parity import assert_close, host, to_dev
from t2h import nn, ops, sparse

pytestmark = pytest.mark.gpu
G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_golden.npz"), allow_pickle=False)


def test_golden_layernorm(dev):
    assert_close(ops.ln_modulate(to_dev(G["ln_x"], dev), 1e-6), G["ln_eps1e-6"], torch.float32, "ln")
    got = ops.ln_modulate(to_dev(G["ln_x"], dev), 1e-5, weight=to_dev(G["ln_w"], dev), bias=to_dev(G["ln_b"], dev))
    assert_close(got, G["ln_affine_eps1e-5"], torch.float32, "ln affine")


def test_golden_modulate_and_gather(dev):
    got = nn.modulate(to_dev(G["mod_x"], dev), to_dev(G["mod_shift"], dev), to_dev(G["mod_scale"], dev))
    assert np.array_equal(host(got), G["mod_out"])
    st = sparse.SparseTensor(to_dev(G["sp_h"], dev), to_dev(G["sp_coords"], dev), 3)
    assert np.array_equal(host(st.offsets).astype(np.int64), G["sp_offsets"])
    got = sparse._mod_shift_scale(st, to_dev(G["sp_shift"], dev), to_dev(G["sp_scale"], dev))
    assert np.array_equal(host(got.feats), G["sp_mod_out"])
    gr = ops.gate_residual(to_dev(G["gr_x"], dev), to_dev(G["gr_y"], dev), gate=to_dev(G["gr_gate"], dev),
                           offsets=st.offsets)
    assert np.array_equal(host(gr), G["gr_out"])
    gr = ops.gate_residual(to_dev(G["gr_x"], dev), to_dev(G["gr_y"], dev), gate=to_dev(G["gr_gate"], dev),
                           bias=to_dev(G["gr_bias"], dev), offsets=st.offsets)
    assert np.array_equal(host(gr), G["gr_out_bias"])


def test_golden_rms_rope(dev):
    rms = nn.MultiHeadRMSNorm(128, 12)
    rms.gamma = to_dev(G["rms_gamma"], dev)
    assert_close(rms.forward(to_dev(G["rms_x"], dev)), G["rms_out"], torch.float32, "rms")
    assert np.array_equal(nn.rope_freqs(128), G["rope_freqs128"]), "host frequency table must be bit-exact"
    assert np.array_equal(nn.rope_freqs(64), G["rope_freqs64"])
    ph = ops.rope_phases(5, 128, G["rope_freqs128"], coords=to_dev(G["sp_coords"], dev))
    assert_close(ph, G["rope_phases_coords"], torch.float32, "phases")
    q, _ = ops.qk_rmsnorm_rope(q=to_dev(G["rms_x"], dev), gamma_q=to_dev(G["rms_gamma"], dev),
                               freqs=G["rope_freqs128"], coords=to_dev(G["sp_coords"], dev))
    assert_close(q, G["rope_rotate_out"], torch.float32, "rms+rope")


def test_golden_activations_and_timestep(dev):
    for k, name in enumerate(["relu", "silu", "gelu", "gelu_tanh"]):
        assert_close(nn.activation(to_dev(G["act_x"], dev), k), G[f"act_{name}"], torch.float32, name)
    got = ops.activation(to_dev(G["gelu_bias_h"], dev), ops.ACT_GELU_TANH, bias=to_dev(G["gelu_bias_b"], dev))
    assert_close(got, G["gelu_bias_out"], torch.float32, "gelu+bias")
    for dim in (256, 255):
        got = nn.TimestepEmbedder(dim).timestep_embedding(to_dev(G["ts_t"], dev))
        assert_close(got, G[f"ts_{dim}"], torch.float32, f"timestep {dim}")
