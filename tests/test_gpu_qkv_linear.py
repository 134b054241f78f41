"""GPU parity: the qkv linear fused with the self-attention epilogue and the
head-major pack (t2h_qkv_linear_pack), through the C ABI, against the C
oracle's composition of the reference's chain: the qkv GEMM
(gpu/linear.mojo:326-388, f16 operands, f32 sums), bias_rms_rope_qkv,
pack_q_z and pack_kv_z (gpu/attention.mojo:507-563, 566-594, 634-662, order
983-1013).

head_dim 128 (12 heads at width 1536, config 5's geometry) and head_dim 64
(16 heads at width 1024, the reference's sparse SLat geometry).

Bar: the f16 (bf16) storage tolerance of tests/_parity.py. The GEMM sums the
same exact products in another order and the head's sum of squares is
reduced in another order, both far below the storage rounding; pads are
exact zeros."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, host, storage_round, to_dev
from t2h import nn, ops, workloads
from t2h._lib import T2HError

pytestmark = pytest.mark.gpu
H, D, C = 12, 128, 1536


def _case(seed, rows, dtype, k=C):
    x = storage_round(orc.randn(seed, (rows, k)), dtype)
    w = storage_round(orc.randn(seed + 1, (3 * H * D, k), std=0.02), dtype)
    bias = orc.randn(seed + 2, (3 * H * D,), std=0.05)
    gq = orc.randn(seed + 3, (H, D), mean=1.0, std=0.02)
    gk = orc.randn(seed + 4, (H, D), mean=1.0, std=0.02)
    return x, w, bias, gq, gk


def _want(x, w, bias, gq, gk, phases, mp, lp):
    qkv = orc.linear(x, w)
    return orc.attn_pack(qkv, H, D, mp, lp, bias, gq, gk, phases)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sparse_coords_padded(dev, dtype):
    """Config-4 voxel rows (the first 3000 of the 64^3 shells) with RoPE from
    int coords, padded to a multiple of 64 as the reference chain does."""
    coords, _ = workloads.config4()
    coords = np.ascontiguousarray(coords[:3000])
    rows = coords.shape[0]
    mp = (rows + 63) // 64 * 64
    x, w, bias, gq, gk = _case(5000, rows, dtype)
    phases = orc.rope_phases_from_coords(coords, D, orc.rope_freqs(D))
    wq, wk, wv = _want(x, w, bias, gq, gk, phases, mp, mp)
    qh, kt, vh = ops.qkv_linear_pack(to_dev(x, dev, dtype), to_dev(w, dev, dtype), H, bias=to_dev(bias, dev),
                                     gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), mp=mp, lp=mp,
                                     freqs=nn.rope_freqs(D), coords=to_dev(coords, dev))
    assert qh.shape == (H, mp, D) and kt.shape == (H, D, mp) and vh.shape == (H, mp, D)
    assert_close(qh, wq, dtype, "qh")
    assert_close(kt, wk, dtype, "kt")
    assert_close(vh, wv, dtype, "vh")
    assert not host(qh)[:, rows:].any() and not host(kt)[:, :, rows:].any() and not host(vh)[:, rows:].any()


def test_dense_grid_phase_table_and_k_layouts(dev):
    """Config-2 tokens (16^3 grid, 4096 rows) with the reference's uploaded
    phase table; k row-major [H, lp, D] is the transpose of the [H, D, lp] k."""
    rows = 4096
    x, w, bias, gq, gk = _case(5100, rows, torch.float16)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16), D, orc.rope_freqs(D))
    wq, wk, wv = _want(x, w, bias, gq, gk, phases, rows, rows)
    args = dict(bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(D),
                phases=to_dev(phases, dev))
    xd, wd = to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16)
    qh, kt, vh = ops.qkv_linear_pack(xd, wd, H, **args)
    assert_close(qh, wq, torch.float16, "qh")
    assert_close(kt, wk, torch.float16, "kt")
    assert_close(vh, wv, torch.float16, "vh")
    qh2, kr, vh2 = ops.qkv_linear_pack(xd, wd, H, k_transposed=False, **args)
    assert torch.equal(qh2, qh) and torch.equal(vh2, vh)
    assert torch.equal(kr, kt.transpose(1, 2).contiguous())


def test_grid_positions_match_phase_table(dev):
    """Positions from the dense grid index (no table) give the result of a
    phase table built on the device from the same grid (same sincos)."""
    rows = 1000
    x, w, bias, gq, gk = _case(5200, rows, torch.float16)
    xd, wd = to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16)
    phases = ops.rope_phases(rows, D, nn.rope_freqs(D), grid_res=16, device=dev)
    kw = dict(bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(D))
    a = ops.qkv_linear_pack(xd, wd, H, grid_res=16, **kw)
    b = ops.qkv_linear_pack(xd, wd, H, phases=phases, **kw)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_no_rms_no_rope_no_bias_is_gemm_plus_pack(dev):
    """Without bias, RMS and RoPE the op is the GEMM followed by the packs:
    every output equals t2h_linear's f32 sums rounded once, permuted (bit
    exact), q scaled by 1/sqrt(D) in f32."""
    rows = 700
    x, w, _, _, _ = _case(5300, rows, torch.float16)
    xd, wd = to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16)
    qh, kt, vh = ops.qkv_linear_pack(xd, wd, H, use_rope=False, mp=768, lp=768)
    qkv = host(ops.linear(xd, wd, out_dtype=torch.float32)).reshape(rows, 3, H, D)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    assert np.array_equal(host(qh)[:, :rows], storage_round((qkv[:, 0] * scale).transpose(1, 0, 2), torch.float16))
    assert np.array_equal(host(kt)[:, :, :rows], storage_round(qkv[:, 1].transpose(1, 2, 0), torch.float16))
    assert np.array_equal(host(vh)[:, :rows], storage_round(qkv[:, 2].transpose(1, 0, 2), torch.float16))
    assert not host(qh)[:, rows:].any() and not host(vh)[:, rows:].any()


def test_pads_beyond_the_last_token_tile(dev):
    """mp and lp past the token tiles of the rows (rows = 300, pads to 1000):
    tiles with no rows skip the GEMM and write zeros; mp != lp."""
    rows = 300
    x, w, bias, gq, gk = _case(5400, rows, torch.float16)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16)[:rows], D, orc.rope_freqs(D))
    wq, wk, wv = _want(x, w, bias, gq, gk, phases, 1000, 1024)
    qh, kt, vh = ops.qkv_linear_pack(to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16), H,
                                     bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                                     mp=1000, lp=1024, freqs=nn.rope_freqs(D), phases=to_dev(phases, dev))
    assert qh.shape == (H, 1000, D) and kt.shape == (H, D, 1024)
    assert_close(qh, wq, torch.float16, "qh")
    assert_close(kt, wk, torch.float16, "kt")
    assert_close(vh, wv, torch.float16, "vh")


@pytest.mark.parametrize("heads", [2, 4, 16])
def test_other_head_counts(dev, heads):
    """H = 2, 4 and 16: q, k and v start at feature tiles 0, H/2 and H, so
    every wave finds its tensor and head from its feature tile (with H = 2
    each tensor is one tile). Ragged rows (700), phase table, pads to 704."""
    rows, k, mp = 700, 256, 704
    n = 3 * heads * D
    x = storage_round(orc.randn(5500 + heads, (rows, k)), torch.float16)
    w = storage_round(orc.randn(5501 + heads, (n, k), std=0.05), torch.float16)
    bias = orc.randn(5502 + heads, (n,), std=0.05)
    gq = orc.randn(5503 + heads, (heads, D), mean=1.0, std=0.02)
    gk = orc.randn(5504 + heads, (heads, D), mean=1.0, std=0.02)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16)[:rows], D, orc.rope_freqs(D))
    wq, wk, wv = orc.attn_pack(orc.linear(x, w), heads, D, mp, mp, bias, gq, gk, phases)
    qh, kt, vh = ops.qkv_linear_pack(to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16), heads,
                                     bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                                     mp=mp, lp=mp, freqs=nn.rope_freqs(D), phases=to_dev(phases, dev))
    assert qh.shape == (heads, mp, D) and kt.shape == (heads, D, mp) and vh.shape == (heads, mp, D)
    assert_close(qh, wq, torch.float16, f"qh H={heads}")
    assert_close(kt, wk, torch.float16, f"kt H={heads}")
    assert_close(vh, wv, torch.float16, f"vh H={heads}")


def _case_hd(seed, rows, heads, hd, k, dtype):
    n = 3 * heads * hd
    x = storage_round(orc.randn(seed, (rows, k)), dtype)
    w = storage_round(orc.randn(seed + 1, (n, k), std=0.02), dtype)
    bias = orc.randn(seed + 2, (n,), std=0.05)
    gq = orc.randn(seed + 3, (heads, hd), mean=1.0, std=0.02)
    gk = orc.randn(seed + 4, (heads, hd), mean=1.0, std=0.02)
    return x, w, bias, gq, gk


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_head_dim_64_slat_sparse_coords(dev, dtype, k_transposed):
    """The reference's sparse SLat geometry: width 1024 as 16 heads of 64
    (gpu/attention.mojo:983-1013; tests/parity/parity_wp11_gpu_attn.mojo's
    whole-block case), 2,369 sparse tokens with RoPE from their int coords,
    padded to a multiple of 64. A wave's 128 features are two heads: each
    head's sum of squares is 32 values per lane and one lane ^ 32 shuffle."""
    heads, hd, k = 16, 64, 1024
    coords, _ = workloads.config4()
    coords = np.ascontiguousarray(coords[:2369])
    rows = coords.shape[0]
    mp = (rows + 63) // 64 * 64
    x, w, bias, gq, gk = _case_hd(5600, rows, heads, hd, k, dtype)
    phases = orc.rope_phases_from_coords(coords, hd, orc.rope_freqs(hd))
    wq, wk, wv = orc.attn_pack(orc.linear(x, w), heads, hd, mp, mp, bias, gq, gk, phases)
    qh, ko, vh = ops.qkv_linear_pack(to_dev(x, dev, dtype), to_dev(w, dev, dtype), heads, bias=to_dev(bias, dev),
                                     gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), mp=mp, lp=mp,
                                     freqs=nn.rope_freqs(hd), coords=to_dev(coords, dev),
                                     k_transposed=k_transposed)
    assert qh.shape == (heads, mp, hd) and vh.shape == (heads, mp, hd)
    assert ko.shape == ((heads, hd, mp) if k_transposed else (heads, mp, hd))
    assert_close(qh, wq, dtype, "qh")
    assert_close(ko, wk if k_transposed else wk.transpose(0, 2, 1), dtype, "k")
    assert_close(vh, wv, dtype, "vh")
    assert not host(qh)[:, rows:].any() and not host(vh)[:, rows:].any()


def test_head_dim_64_dense_grid(dev):
    """16 x 64 heads at width 1024 on 2,048 dense tokens (the reference's L =
    2048 whole-block case) with the uploaded phase table, and the same tokens
    with positions from the grid index: both equal the oracle's chain, and
    the grid path equals a device-built phase table bit for bit."""
    heads, hd, k, rows = 16, 64, 1024, 2048
    x, w, bias, gq, gk = _case_hd(5700, rows, heads, hd, k, torch.float16)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16)[:rows], hd, orc.rope_freqs(hd))
    wq, wk, wv = orc.attn_pack(orc.linear(x, w), heads, hd, rows, rows, bias, gq, gk, phases)
    xd, wd = to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16)
    kw = dict(bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(hd))
    qh, kt, vh = ops.qkv_linear_pack(xd, wd, heads, phases=to_dev(phases, dev), **kw)
    assert_close(qh, wq, torch.float16, "qh")
    assert_close(kt, wk, torch.float16, "kt")
    assert_close(vh, wv, torch.float16, "vh")
    a = ops.qkv_linear_pack(xd, wd, heads, grid_res=16, **kw)
    b = ops.qkv_linear_pack(xd, wd, heads, phases=ops.rope_phases(rows, hd, nn.rope_freqs(hd), grid_res=16,
                                                                   device=dev), **kw)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_head_dim_64_is_gemm_plus_pack(dev):
    """head_dim 64 without bias, RMS and RoPE: the GEMM's f32 sums rounded
    once and permuted into the two heads of each wave's features (bit
    exact), both k layouts; 8 heads, ragged rows, pads."""
    heads, hd, k, rows = 8, 64, 512, 700
    x, w, _, _, _ = _case_hd(5800, rows, heads, hd, k, torch.float16)
    xd, wd = to_dev(x, dev, torch.float16), to_dev(w, dev, torch.float16)
    qkv = host(ops.linear(xd, wd, out_dtype=torch.float32)).reshape(rows, 3, heads, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    for kt_layout in (True, False):
        qh, ko, vh = ops.qkv_linear_pack(xd, wd, heads, use_rope=False, mp=768, lp=712, k_transposed=kt_layout)
        assert np.array_equal(host(qh)[:, :rows],
                              storage_round((qkv[:, 0] * scale).transpose(1, 0, 2), torch.float16))
        kw = qkv[:, 1].transpose(1, 2, 0) if kt_layout else qkv[:, 1].transpose(1, 0, 2)
        got_k = host(ko)[:, :, :rows] if kt_layout else host(ko)[:, :rows]
        assert np.array_equal(got_k, storage_round(kw, torch.float16))
        assert np.array_equal(host(vh)[:, :rows], storage_round(qkv[:, 2].transpose(1, 0, 2), torch.float16))
        assert not host(qh)[:, rows:].any() and not host(vh)[:, rows:].any()
        assert not (host(ko)[:, :, rows:] if kt_layout else host(ko)[:, rows:]).any()


def test_zero_rows_and_errors(dev):
    w = torch.zeros((3 * H * D, C), dtype=torch.float16, device=dev)
    qh, kt, vh = ops.qkv_linear_pack(torch.zeros((0, C), dtype=torch.float16, device=dev), w, H, mp=64, lp=64,
                                     use_rope=False)
    assert not host(qh).any() and not host(kt).any() and not host(vh).any()
    with pytest.raises(T2HError, match="head_dim must be 64 or 128"):
        ops.qkv_linear_pack(torch.zeros((4, C), dtype=torch.float16, device=dev),
                            torch.zeros((3 * H * 32, C), dtype=torch.float16, device=dev), H, use_rope=False)
    with pytest.raises(T2HError, match="even for head_dim 128"):
        ops.qkv_linear_pack(torch.zeros((4, C), dtype=torch.float16, device=dev),
                            torch.zeros((3 * 3 * D, C), dtype=torch.float16, device=dev), 3, use_rope=False)
    with pytest.raises(T2HError, match="a multiple of 4 for 64"):
        ops.qkv_linear_pack(torch.zeros((4, C), dtype=torch.float16, device=dev),
                            torch.zeros((3 * 6 * 64, C), dtype=torch.float16, device=dev), 6, use_rope=False)
    with pytest.raises(ValueError, match="lp % 8"):
        ops.qkv_linear_pack(torch.zeros((4, C), dtype=torch.float16, device=dev), w, H, mp=4, lp=4,
                            use_rope=False)
