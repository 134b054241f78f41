"""GPU parity: the self-attention epilogue fused with the head-major packing
of the attention operands (t2h_attn_pack), through the C ABI, against the C
oracle's bias_rms_rope_qkv + pack_q_z + pack_kv_z sequence
(gpu/attention.mojo:507-563, 566-594, 634-662, order 987-1013) and the cross
chain's bias_rms_q + pack_q_z (596-631, 1223-1234).
Metric and tolerances: tests/_parity.py; index work (packing, transposition,
pads) is compared bit for bit."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, host, storage_round, to_dev
from t2h import nn, ops, workloads
from t2h._lib import T2HError

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def pad64(n):
    return (n + 63) // 64 * 64


def _params(h, d, seed):
    bias = orc.randn(seed, (3, h, d), std=0.05)
    gq = orc.randn(seed + 1, (h, d), mean=1.0, std=0.02)
    gk = orc.randn(seed + 2, (h, d), mean=1.0, std=0.02)
    return bias, gq, gk


def _views(qkv_dev, h, d):
    q3 = qkv_dev.reshape(qkv_dev.shape[0], 3, h, d)
    return q3[:, 0], q3[:, 1], q3[:, 2]


def test_config2_dense_grid_f32(dev):
    """Config-2 shape: qkv [4096, 3, 12, 128] f32, 16^3 grid positions, mp = lp = 4096."""
    rows, h, d = 4096, 12, 128
    qkv = orc.randn(2100, (rows, 3, h, d))
    bias, gq, gk = _params(h, d, 2101)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16), d, orc.rope_freqs(d))
    wq, wk, wv = orc.attn_pack(qkv, h, d, rows, rows, bias.reshape(-1), gq, gk, phases)
    q, k, v = _views(to_dev(qkv, dev), h, d)
    b = to_dev(bias, dev)
    qh, kt, vh = ops.attn_pack(q, k, v, bias_q=b[0], bias_k=b[1], bias_v=b[2], gamma_q=to_dev(gq, dev),
                               gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d), grid_res=16)
    assert qh.shape == (h, rows, d) and kt.shape == (h, d, rows) and vh.shape == (h, rows, d)
    assert_close(qh, wq, torch.float32, "qh")
    assert_close(kt, wk, torch.float32, "kt")
    assert_close(vh, wv, torch.float32, "vh")


@pytest.mark.parametrize("dtype", DTYPES)
def test_config4_sparse_coords_padded(dev, dtype):
    """Sparse rows (config 4, T = 39,804) with RoPE from int coords, padded to
    the next multiple of 64 as the reference chain does (mp = lp)."""
    coords, _ = workloads.config4()
    rows, h, d = coords.shape[0], 12, 128
    mp = pad64(rows)
    assert mp > rows
    qkv = storage_round(orc.randn(2200, (rows, 3, h, d)), dtype)
    bias, gq, gk = _params(h, d, 2201)
    phases = orc.rope_phases_from_coords(coords, d, orc.rope_freqs(d))
    wq, wk, wv = orc.attn_pack(qkv, h, d, mp, mp, bias.reshape(-1), gq, gk, phases)
    q, k, v = _views(to_dev(qkv, dev, dtype), h, d)
    b = to_dev(bias, dev)
    qh, kt, vh = ops.attn_pack(q, k, v, mp=mp, lp=mp, bias_q=b[0], bias_k=b[1], bias_v=b[2],
                               gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d),
                               coords=to_dev(coords, dev))
    assert_close(qh, wq, dtype, f"qh {dtype}")
    assert_close(kt, wk, dtype, f"kt {dtype}")
    assert_close(vh, wv, dtype, f"vh {dtype}")
    # the pads are exact zeros and v is bias-add only (bit-exact)
    assert not host(qh)[:, rows:].any() and not host(kt)[:, :, rows:].any() and not host(vh)[:, rows:].any()
    assert torch.equal(vh.cpu(), torch.from_numpy(storage_round(wv, dtype)).to(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [64, 128])
def test_k_layouts_agree(dev, dtype, d):
    """k [H, D, lp] (the reference's kt) is the exact transpose of [H, lp, D]."""
    rows, h = 1000, 8
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = orc.Rng(5).uniform((rows, 3), 0, 64).astype(np.int32)
    qkv = to_dev(orc.randn(2300 + d, (rows, 3, h, d)), dev, dtype)
    q, k, v = _views(qkv, h, d)
    gq, gk = [to_dev(g, dev) for g in _params(h, d, 2301)[1:]]
    kw = dict(gamma_q=gq, gamma_k=gk, freqs=nn.rope_freqs(d), coords=to_dev(coords, dev), mp=1024, lp=1024)
    _, kt, _ = ops.attn_pack(None, k, None, k_transposed=True, **kw)
    _, kn, _ = ops.attn_pack(None, k, None, k_transposed=False, **kw)
    assert kt.shape == (h, d, 1024) and kn.shape == (h, 1024, d)
    assert torch.equal(kt, kn.transpose(1, 2))
    # and the same k through the row-major QK kernel (no packing) agrees to tolerance
    _, kr = ops.qk_rmsnorm_rope(k=k, gamma_k=gk, freqs=nn.rope_freqs(d), coords=to_dev(coords, dev))
    assert_close(kn[:, :rows].transpose(0, 1), host(kr), dtype, "packed k vs qk_rmsnorm_rope")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows", [25_000, 39_804, 100_000, 140_000])
def test_k_transposed_head_groups(dev, dtype, rows):
    """The transposed-k tile kernel walks a group of heads per block, the
    16-bit tiles alternating between two LDS buffers from head to head. On
    256 CUs these row counts give 2, 3, 6 and 12 heads per block; each must
    equal the row-major layout (another kernel) exactly."""
    h, d = 12, 128
    g = torch.Generator(device=dev).manual_seed(rows)
    qkv = torch.randn((rows, 3, h, d), generator=g, device=dev).to(dtype)
    coords = torch.randint(0, 64, (rows, 4), generator=g, device=dev, dtype=torch.int32)
    gq, gk = [torch.randn((h, d), generator=g, device=dev) * 0.05 + 1 for _ in range(2)]
    bk = torch.randn((h, d), generator=g, device=dev) * 0.02
    mp = pad64(rows)
    kw = dict(bias_k=bk, gamma_q=gq, gamma_k=gk, freqs=nn.rope_freqs(d), coords=coords, mp=mp, lp=mp)
    _, kt, _ = ops.attn_pack(None, qkv[:, 1], None, k_transposed=True, **kw)
    _, kn, _ = ops.attn_pack(None, qkv[:, 1], None, k_transposed=False, **kw)
    assert torch.equal(kt, kn.transpose(1, 2)), rows


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_cross_chain_q_only(dev, dtype):
    """Cross chain: q [rows, H, D] rows H*D apart, + bias, RMS, no RoPE, packed
    into qh [H, mp, D] (bias_rms_q + pack_q_z with stride H*D)."""
    rows, h, d = 1234, 12, 128
    mp = pad64(rows)
    q = storage_round(orc.randn(2400, (rows, h, d)), dtype)
    bias, gq, _ = _params(h, d, 2401)
    e, _ = orc.qk_rms_rope(q, q, gq, gq, None, bias_q=bias[0], bias_k=bias[0], use_rope=False)
    want = orc.pack_q(e.reshape(rows, -1), rows, h, d, mp, h * d)
    qh, ko, vh = ops.attn_pack(to_dev(q, dev, dtype), mp=mp, bias_q=to_dev(bias[0], dev), gamma_q=to_dev(gq, dev),
                               use_rope=False)
    assert ko is None and vh is None
    assert_close(qh, want, dtype, f"cross qh {dtype}")


def test_pack_only_bit_exact(dev):
    """Without bias, RMS and RoPE the pack is pure data movement plus the
    1/sqrt(D) product: bit-exact with pack_q_z / pack_kv_z in f32."""
    rows, h, d = 777, 12, 64
    qkv = orc.randn(2500, (rows, 3, h, d))
    mp = pad64(rows)
    wq = orc.pack_q(qkv.reshape(rows, -1), rows, h, d, mp, 3 * h * d)
    wk, wv = orc.pack_kv(qkv, rows, h, d, mp)
    q, k, v = _views(to_dev(qkv, dev), h, d)
    qh, kt, vh = ops.attn_pack(q, k, v, mp=mp, lp=mp, use_rope=False)
    assert np.array_equal(host(qh), wq)
    assert np.array_equal(host(kt), wk)
    assert np.array_equal(host(vh), wv)


def test_empty_rows_zero_pads(dev):
    """rows = 0 with mp = lp = 64: every output row is a pad row."""
    h, d = 4, 128
    qkv = torch.empty((0, 3 * h * d), device=dev)
    q, k, v = _views(qkv, h, d)
    qh, kt, vh = ops.attn_pack(q, k, v, mp=64, lp=64, use_rope=False)
    for t in (qh, kt, vh):
        assert t.numel() == h * 64 * d and not t.any()


@pytest.mark.parametrize("k_transposed", [1, 0])
def test_empty_rows_with_rope_sources(dev, k_transposed):
    """rows = 0 with RoPE on and a non-NULL coords pointer (a caller's
    buffer of other rows) or a phase table, through the C ABI: no coordinate,
    phase or row is read, and every output row is a zero pad. (A zero-row
    torch view has a NULL data pointer, so the call is made directly.)"""
    from t2h._lib import call

    h, d, lp = 4, 128, 64
    freqs, fp, fd = ops._host_freqs(nn.rope_freqs(d))
    coords = torch.zeros((16, 4), dtype=torch.int32, device=dev)
    phases = torch.ones((1, d // 2, 2), device=dev)
    src = torch.zeros((1, 3 * h * d), device=dev)   # input pointers (never read)
    for ph, ph_rows, co, cc in ((None, 0, coords.data_ptr(), 4), (phases.data_ptr(), 1, None, 0)):
        qh = torch.full((h, lp, d), 7.0, device=dev)
        ko = torch.full((h, lp, d), 7.0, device=dev)
        vh = torch.full((h, lp, d), 7.0, device=dev)
        call("t2h_attn_pack", src.data_ptr(), src.data_ptr(), src.data_ptr(), 3 * h * d, 0, h, d, 0, None, None,
             None, None, None, 1, fp, fd, 3, ph, ph_rows, co, cc, 0, qh.data_ptr(), lp, ko.data_ptr(),
             vh.data_ptr(), lp, k_transposed, ops._stream())
        for t in (qh, ko, vh):
            assert not t.any()
    del freqs


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_many_heads_and_table_phases(dev, dtype):
    """20 heads x 64 (beyond the one-wave-per-row kernel's 16) with a phase
    table as the position source; mp != lp."""
    rows, h, d = 999, 20, 64
    qkv = storage_round(orc.randn(2600, (rows, 3, h, d)), dtype)
    bias, gq, gk = _params(h, d, 2601)
    pos = orc.Rng(2602).uniform((rows, 3), 0, 100).astype(np.float32)
    phases = orc.rope_phases_from_positions(pos, d, orc.rope_freqs(d))
    mp, lp = pad64(rows), pad64(rows) + 64
    wq, wk, wv = orc.attn_pack(qkv, h, d, mp, lp, bias.reshape(-1), gq, gk, phases)
    q, k, v = _views(to_dev(qkv, dev, dtype), h, d)
    b = to_dev(bias, dev)
    for kt in (True, False):
        qh, ko, vh = ops.attn_pack(q, k, v, mp=mp, lp=lp, bias_q=b[0], bias_k=b[1], bias_v=b[2],
                                   gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d),
                                   phases=to_dev(phases, dev), k_transposed=kt)
        assert_close(qh, wq, dtype, f"qh {dtype}")
        assert_close(ko if kt else ko.transpose(1, 2), wk, dtype, f"k transposed={kt} {dtype}")
        assert_close(vh, wv, dtype, f"vh {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_row_major_staged_mp_ne_lp(dev, dtype):
    """16-bit head_dim 128 (the rows staged in LDS and written per head run)
    with mp != lp, a ragged last tile and pads, both k layouts, against the
    oracle; v bit-exact."""
    rows, h, d = 1001, 12, 128
    qkv = storage_round(orc.randn(2800, (rows, 3, h, d)), dtype)
    bias, gq, gk = _params(h, d, 2801)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = orc.Rng(2802).uniform((rows, 3), 0, 64).astype(np.int32)
    phases = orc.rope_phases_from_coords(coords, d, orc.rope_freqs(d))
    mp, lp = pad64(rows), pad64(rows) + 64
    wq, wk, wv = orc.attn_pack(qkv, h, d, mp, lp, bias.reshape(-1), gq, gk, phases)
    q, k, v = _views(to_dev(qkv, dev, dtype), h, d)
    b = to_dev(bias, dev)
    for kt in (False, True):
        qh, ko, vh = ops.attn_pack(q, k, v, mp=mp, lp=lp, bias_q=b[0], bias_k=b[1], bias_v=b[2],
                                   gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d),
                                   coords=to_dev(coords, dev), k_transposed=kt)
        assert_close(qh, wq, dtype, f"qh {dtype}")
        assert_close(ko if kt else ko.transpose(1, 2), wk, dtype, f"k transposed={kt} {dtype}")
        assert torch.equal(vh.cpu(), torch.from_numpy(storage_round(wv, dtype)).to(dtype))
        assert not host(qh)[:, rows:].any() and not host(vh)[:, rows:].any()


def test_attn_pack_errors(dev):
    h, d = 4, 96
    x = torch.zeros((8, 3, h, d), device=dev)
    with pytest.raises(T2HError, match="head_dim must be 64 or 128"):
        ops.attn_pack(x[:, 0], use_rope=False)
    x = torch.zeros((8, 3, h, 128), device=dev)
    with pytest.raises(ValueError, match="lp % 8"):
        ops.attn_pack(None, x[:, 1], None, lp=12, use_rope=False)
    with pytest.raises(ValueError, match="mp < rows"):
        ops.attn_pack(x[:, 0], mp=4, use_rope=False)
    with pytest.raises(ValueError, match="gamma_q and gamma_k"):
        ops.attn_pack(x[:, 0], x[:, 1], gamma_q=torch.ones(h, 128, device=dev), use_rope=False)
    with pytest.raises(ValueError, match="needs phases, coords or grid_res"):
        ops.attn_pack(x[:, 0], freqs=nn.rope_freqs(128))


@pytest.mark.parametrize("rows,h", [(2048, 4), (2369, 4), (2113, 4), (4096, 2), (4160, 16)])
def test_reference_attention_shapes(dev, rows, h):
    """The geometries of the reference's GPU attention parity test
    (tests/parity/parity_wp11_gpu_attn.mojo:261-279: DiT self-attention,
    the odd slat lengths 2369 and 2113, 2 heads at 4096 and 16 heads at 4160,
    head_dim 64), through the epilogue + pack with a dense phase table, in f32
    against the oracle, both k layouts."""
    d = 64
    qkv = orc.randn(2700 + rows + h, (rows, 3, h, d))
    bias, gq, gk = _params(h, d, 2701)
    pos = orc.Rng(2702 + rows).uniform((rows, 3), 0, 16).astype(np.float32)
    phases = orc.rope_phases_from_positions(pos, d, orc.rope_freqs(d))
    mp, lp = pad64(rows), pad64(rows)
    wq, wk, wv = orc.attn_pack(qkv, h, d, mp, lp, bias.reshape(-1), gq, gk, phases)
    q, k, v = _views(to_dev(qkv, dev), h, d)
    b = to_dev(bias, dev)
    for kt in (True, False):
        qh, ko, vh = ops.attn_pack(q, k, v, mp=mp, lp=lp, bias_q=b[0], bias_k=b[1], bias_v=b[2],
                                   gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d),
                                   phases=to_dev(phases, dev), k_transposed=kt)
        assert_close(qh, wq, torch.float32, f"qh rows={rows} h={h}")
        assert_close(ko if kt else ko.transpose(1, 2), wk, torch.float32, f"k transposed={kt} rows={rows} h={h}")
        assert np.array_equal(host(vh), wv), "v: bias add and pack are exact"
