"""GPU parity at sizes past 2^31 elements: every kernel indexes rows and
elements in 64 bits. Each test fills a device tensor of more than 2^31
elements, runs the op, and checks sampled rows (first, middle, last, and
rows straddling the 2^31-element mark) against the C oracle on the same
rows. Metric and tolerances: tests/_parity.py.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, bits_equal, host, storage_round
from t2h import nn, ops

pytestmark = pytest.mark.gpu
BIG = 1 << 31


def _rows(n_rows, cols):
    """Sample rows: ends, middle, and those around element 2^31."""
    mark = BIG // cols
    cand = [0, 1, n_rows // 2, mark - 1, mark, mark + 1, n_rows - 2, n_rows - 1]
    return np.array(sorted({r for r in cand if 0 <= r < n_rows}), np.int64)


def _fill(shape, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)


def test_gelu_bias_past_2g_elements(dev):
    rows, cols = (BIG // 6144) + 4099, 6144          # 2.17e9 elements, 4.3 GB f16
    x = _fill((rows, cols), torch.float16, dev, 1)
    assert x.numel() > BIG
    bias = torch.randn(cols, device=dev) * 0.02
    out = ops.activation(x, ops.ACT_GELU_TANH, bias=bias)
    idx = _rows(rows, cols)
    xi = host(x[idx])
    want = orc.gelu_tanh_bias(xi, host(bias))
    assert_close(out[idx], want, torch.float16, "GELU rows past 2^31 elements")
    del x, out
    torch.cuda.empty_cache()


def test_ln_modulate_and_gated_residual_past_2g_elements(dev):
    rows, cols = (BIG // 1536) + 777, 1536           # 1.4M rows, 4.3 GB f16
    x = _fill((rows, cols), torch.float16, dev, 2)
    assert x.numel() > BIG
    shift, scale = torch.randn(cols, device=dev) * 0.1, torch.randn(cols, device=dev) * 0.1
    y = ops.ln_modulate(x, 1e-6, shift=shift, scale=scale)
    idx = _rows(rows, cols)
    xi = host(x[idx])
    assert_close(y[idx], orc.ln_modulate(xi, host(shift), host(scale), eps=1e-6), torch.float16, "LN rows")
    gate = torch.randn(cols, device=dev) * 0.1
    out = ops.gate_residual(x, y, gate=gate)
    want = orc.gate_residual(xi, host(y[idx]), host(gate))
    assert bits_equal(out[idx], storage_round(want, torch.float16), torch.float16)
    del x, y, out
    torch.cuda.empty_cache()


def test_qk_rmsnorm_rope_past_2g_elements(dev):
    rows, h, d = (BIG // 1536) + 333, 12, 128
    q = _fill((rows, h, d), torch.float16, dev, 3)
    assert q.numel() > BIG
    coords = torch.zeros((rows, 4), dtype=torch.int32, device=dev)
    coords[:, 1:] = (torch.arange(rows, device=dev, dtype=torch.int64).unsqueeze(1) //
                     torch.tensor([16384, 128, 1], device=dev) % 128).to(torch.int32)
    gq = torch.ones((h, d), device=dev) + torch.randn((h, d), device=dev) * 0.02
    qo, _ = ops.qk_rmsnorm_rope(q=q, gamma_q=gq, freqs=nn.rope_freqs(d), coords=coords)
    idx = _rows(rows, h * d)
    qi, ci = host(q[idx]), coords[idx].cpu().numpy()
    phases = orc.rope_phases_from_coords(ci, d, orc.rope_freqs(d))
    want, _ = orc.qk_rms_rope(qi, qi, host(gq), host(gq), phases)
    assert_close(qo[idx], want, torch.float16, "QK rows past 2^31 elements")
    del q, qo, coords
    torch.cuda.empty_cache()


# ---- launches past 2^20 blocks take a 2-D grid (block_linear) -----------------
GRID_X = 1 << 20


def test_two_d_grid_ln_and_gelu(dev):
    """LN with 8 rows per block and GELU with 4 rows per block, both at
    512 columns, with more than 2^20 blocks."""
    rows = 8 * GRID_X + 13
    x = _fill((rows, 512), torch.float16, dev, 11)
    shift, scale = torch.randn(512, device=dev) * 0.1, torch.randn(512, device=dev) * 0.1
    y = ops.ln_modulate(x, 1e-6, shift=shift, scale=scale)
    idx = np.array([0, GRID_X * 8 - 1, GRID_X * 8, rows - 9, rows - 1])
    assert_close(y[idx], orc.ln_modulate(host(x[idx]), host(shift), host(scale), eps=1e-6), torch.float16,
                 "LN on a 2-D grid")
    g = ops.activation(x, ops.ACT_GELU_TANH)
    idx = np.array([0, 4 * GRID_X - 1, 4 * GRID_X, rows - 1])
    assert_close(g[idx], orc.activation(host(x[idx]), orc.ACT_GELU_TANH), torch.float16, "GELU on a 2-D grid")
    del x, y, g
    torch.cuda.empty_cache()


def test_two_d_grid_qk_and_pack(dev):
    """QK (8 rows per block, q only) and the attention pack (8 rows per block
    and tensor) past 2^20 blocks, 4 heads x 64."""
    h, d = 4, 64
    rows = 8 * GRID_X + 9
    q = _fill((rows, h, d), torch.float16, dev, 12)
    coords = torch.zeros((rows, 4), dtype=torch.int32, device=dev)
    coords[:, 1:] = (torch.arange(rows, device=dev).unsqueeze(1) // torch.tensor([4096, 64, 1], device=dev)
                     % 64).to(torch.int32)
    gq = torch.ones((h, d), device=dev)
    fr = nn.rope_freqs(d)
    qo, _ = ops.qk_rmsnorm_rope(q=q, gamma_q=gq, freqs=fr, coords=coords)
    idx = np.array([0, 8 * GRID_X - 1, 8 * GRID_X, rows - 1])
    ph = orc.rope_phases_from_coords(coords[idx].cpu().numpy(), d, orc.rope_freqs(d))
    want, _ = orc.qk_rms_rope(host(q[idx]), host(q[idx]), host(gq), host(gq), ph)
    assert_close(qo[idx], want, torch.float16, "QK on a 2-D grid")
    del qo
    # pack: q, k, v views of [n, 3, h, d] with n such that ceil(n / 8) * 3 > 2^20
    n = (GRID_X // 3 + 1000) * 8 + 5
    qkv = _fill((n, 3, h, d), torch.float16, dev, 13)
    mp = (n + 63) // 64 * 64
    qh, kt, vh = ops.attn_pack(qkv[:, 0], qkv[:, 1], qkv[:, 2], mp=mp, lp=mp, use_rope=False, k_transposed=False)
    for t in (n - 1, n - 2, 0):
        src = host(qkv[t])
        assert np.array_equal(host(vh[:, t]), src[2])
        assert np.array_equal(host(kt[:, t]), src[1])
    assert not host(qh[:, n:]).any()
    del q, coords, qkv, qh, kt, vh
    torch.cuda.empty_cache()


def test_two_d_grid_sampler_rescale(dev):
    """Dense CFG rescale with one segment per row and more than 2^20 rows:
    the per-segment ratio pass and the two block passes use 2-D grids."""
    rows, rs = GRID_X + 7, 4
    x = _fill((rows, rs), torch.float32, dev, 14)
    pos = _fill((rows, rs), torch.float32, dev, 15)
    neg = _fill((rows, rs), torch.float32, dev, 16)
    xp, _ = ops.flow_euler_step(x, pos, 0.8, 0.7, 1e-5, v_neg=neg, guidance_strength=3.0, guidance_rescale=0.7,
                                pred_x0=False)
    idx = np.array([0, GRID_X - 1, GRID_X, rows - 1])
    xs, ps, ns = host(x[idx]), host(pos[idx]), host(neg[idx])
    pred = orc.flow_rescale(xs, orc.flow_cfg(ps, ns, 3.0), ps, 0.8, 1e-5, 0.7)
    want = orc.flow_step(xs, pred, 0.8, 0.7)
    assert_close(xp[idx], want, torch.float32, "sampler on a 2-D grid")


def test_linear_output_past_2g_elements(dev):
    """The MFMA GEMM with an output of more than 2^31 elements ([466,000+,
    4608] f16, 4.3 GB): sampled rows, including those straddling element 2^31,
    match the oracle's GEMM on the same rows (to the f16 storage bar)."""
    n, k = 4608, 256
    rows = BIG // n + 517
    x = _fill((rows, k), torch.float16, dev, 21)
    w = (torch.randn((n, k), device=dev) * 0.05).to(torch.float16)
    out = ops.linear(x, w)
    assert out.numel() > BIG
    idx = _rows(rows, n)
    want = orc.linear(host(x[idx]), host(w))
    assert_close(out[idx], want, torch.float16, "linear rows past 2^31 output elements")
    del x, out
    torch.cuda.empty_cache()


def test_qkv_linear_pack_past_2g_elements(dev):
    """The fused qkv linear + pack with qh/kt/vh of more than 2^31 elements
    each (rows x 12 heads x 128 > 2^31): sampled tokens match the oracle's
    GEMM followed by the attention epilogue and packs."""
    h, d, k = 12, 128, 64
    rows = BIG // (h * d) + 333
    x = _fill((rows, k), torch.float16, dev, 22)
    w = (torch.randn((3 * h * d, k), device=dev) * 0.1).to(torch.float16)
    mp = (rows + 63) // 64 * 64
    qh, kt, vh = ops.qkv_linear_pack(x, w, h, mp=mp, lp=mp, use_rope=False, k_transposed=True)
    assert qh.numel() > BIG and kt.numel() > BIG
    idx = _rows(rows, h * d)
    qkv = orc.linear(host(x[idx]), host(w)).reshape(-1, 3, h, d)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    assert_close(qh[:, idx], (qkv[:, 0] * scale).transpose(1, 0, 2), torch.float16, "qh")
    assert_close(kt[:, :, idx], qkv[:, 1].transpose(1, 2, 0), torch.float16, "kt")
    assert_close(vh[:, idx], qkv[:, 2].transpose(1, 0, 2), torch.float16, "vh")
    del x, qh, kt, vh
    torch.cuda.empty_cache()
