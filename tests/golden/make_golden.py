"""Writes tests/golden/oracle_golden.npz: small seeded inputs and the C
oracle's outputs for every hot-path function (rows H1-H18 of the reference's
per-token ops). The fixtures pin the oracle across sessions: test_golden.py
recomputes them and requires identical bits (integer outputs) or agreement to
1 ulp-level tolerance (libm transcendentals).

Run: python tests/golden/make_golden.py   (CPU only)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as orc  # noqa: E402


def build() -> dict:
    g = {}
    r = orc.Rng(1337)
    g["rng_u64_seed1337"] = np.array([r.next_u64() for _ in range(8)], np.uint64)
    g["randn_seed42"] = orc.randn(42, (16,))
    # LayerNorm (+ affine) and modulate
    x = orc.randn(1, (6, 1536), mean=0.3, std=1.7)
    g["ln_x"] = x
    g["ln_eps1e-6"] = orc.layernorm(x, 1e-6)
    w, b = orc.randn(2, (1536,), mean=1.0, std=0.1), orc.randn(3, (1536,), std=0.1)
    g["ln_w"], g["ln_b"] = w, b
    g["ln_affine_eps1e-5"] = orc.layernorm(x, 1e-5, True, w, b)
    xm = orc.randn(4, (2, 5, 64))
    sh, sc = orc.randn(5, (2, 64), std=0.1), orc.randn(6, (2, 64), std=0.1)
    g["mod_x"], g["mod_shift"], g["mod_scale"] = xm, sh, sc
    g["mod_out"] = orc.modulate(xm, sh, sc)
    # sparse layout + gathered modulate
    coords = np.array([[0, 1, 2, 3], [0, 4, 5, 6], [2, 0, 0, 0], [2, 1, 1, 1], [2, 7, 8, 9]], np.int32)
    g["sp_coords"] = coords
    g["sp_offsets"] = orc.cal_offsets(coords, 3)
    hs = orc.randn(7, (5, 64))
    g["sp_h"] = hs
    shs, scs = orc.randn(8, (3, 64), std=0.1), orc.randn(9, (3, 64), std=0.1)
    g["sp_shift"], g["sp_scale"] = shs, scs
    g["sp_mod_out"] = orc.mod_shift_scale(hs, shs, scs, g["sp_offsets"])
    # RMSNorm + RoPE
    q = orc.randn(10, (5, 12, 128), std=2.0)
    gq = orc.randn(11, (12, 128), mean=1.0, std=0.02)
    g["rms_x"], g["rms_gamma"] = q, gq
    g["rms_out"] = orc.multihead_rmsnorm(q, gq)
    f = orc.rope_freqs(128)
    g["rope_freqs128"] = f
    g["rope_freqs64"] = orc.rope_freqs(64)
    g["rope_phases_coords"] = orc.rope_phases_from_coords(coords, 128, f)
    g["rope_phases_grid4"] = orc.rope_phases_from_positions(orc.grid_positions(4), 128, f)
    g["rope_rotate_out"] = orc.rope_rotate(g["rms_out"], g["rope_phases_coords"])
    # activations
    a = orc.randn(12, (1024,), std=4.0)
    g["act_x"] = a
    for k, name in enumerate(["relu", "silu", "gelu", "gelu_tanh"]):
        g[f"act_{name}"] = orc.activation(a, k)
    hb = orc.randn(13, (4, 256))
    bb = orc.randn(14, (256,), std=0.02)
    g["gelu_bias_h"], g["gelu_bias_b"] = hb, bb
    g["gelu_bias_out"] = orc.gelu_tanh_bias(hb, bb)
    # gated residual
    xr, yr = orc.randn(15, (5, 64)), orc.randn(16, (5, 64))
    gt = orc.randn(17, (3, 64), std=0.1)
    g["gr_x"], g["gr_y"], g["gr_gate"] = xr, yr, gt
    g["gr_out"] = orc.gate_residual(xr, yr, gt, offsets=g["sp_offsets"])
    g["gr_bias"] = orc.randn(18, (64,), std=0.05)
    g["gr_out_bias"] = orc.gate_residual(xr, yr, gt, offsets=g["sp_offsets"], bias=g["gr_bias"])
    # timestep embedding
    t = np.array([0.0, 0.25, 1.0, 999.0], np.float32)
    g["ts_t"] = t
    g["ts_256"] = orc.timestep_embedding(t, 256)
    g["ts_255"] = orc.timestep_embedding(t, 255)
    return g


if __name__ == "__main__":
    out = os.path.join(HERE, "oracle_golden.npz")
    np.savez(out, **build())
    print("wrote", out, os.path.getsize(out), "bytes")
