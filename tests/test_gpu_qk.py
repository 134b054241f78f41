"""GPU parity: multi-head QK RMSNorm + 3D RoPE (+ qkv bias) and the phase
builder, through the C ABI, against the C oracle
(sparse/attention/modules.mojo:37-102; modules/rope.mojo:17-88;
sparse/attention/rope.mojo:20-134; gpu/attention.mojo:507-631).
Metric and tolerances: tests/_parity.py."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, bits_equal, host, max_err, storage_round, to_dev
from t2h import nn, ops, sparse, workloads

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _gammas(h, d, seed):
    return orc.randn(seed, (h, d), mean=1.0, std=0.02), orc.randn(seed + 1, (h, d), mean=1.0, std=0.02)


def test_config2_dense_grid_f32(dev):
    """fp32 Q,K [4096,12,128], gamma 1+N(0,0.02), 16^3 grid
    positions, base 10000, 21 freqs/axis + identity pad slot 63."""
    rows, h, d = 4096, 12, 128
    q, k = orc.randn(1, (rows, h, d)), orc.randn(2, (rows, h, d))
    gq, gk = _gammas(h, d, 3)
    freqs = orc.rope_freqs(d)
    assert freqs.size == 21
    phases = orc.rope_phases_from_positions(orc.grid_positions(16), d, freqs)
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    qo, ko = ops.qk_rmsnorm_rope(q=to_dev(q, dev), k=to_dev(k, dev), gamma_q=to_dev(gq, dev),
                                 gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d), grid_res=16)
    assert_close(qo, wq, torch.float32, "config2 q")
    assert_close(ko, wk, torch.float32, "config2 k")


def test_config2_mojo_api(dev):
    """MultiHeadRMSNorm.forward then apply_rotary_embedding(x [N,L,H,D], phases)
    with RotaryPositionEmbedder.forward(grid) — the dense MHA order
    (modules/attention.mojo:122-130)."""
    l, h, d = 4096, 12, 128
    q = orc.randn(11, (1, l, h, d))
    gq, _ = _gammas(h, d, 12)
    rms = nn.MultiHeadRMSNorm(d, h)
    rms.gamma = to_dev(gq, dev)
    emb = nn.RotaryPositionEmbedder(d)
    pos = to_dev(orc.grid_positions(16), dev)
    phases = emb.forward(pos)
    ph_want = orc.rope_phases_from_positions(orc.grid_positions(16), d, orc.rope_freqs(d))
    assert max_err(phases, ph_want) <= 2e-7, "phase table"
    got = nn.apply_rotary_embedding(rms.forward(to_dev(q, dev)), phases)
    want = orc.apply_rotary(orc.multihead_rmsnorm(q, gq), ph_want)
    assert_close(got, want, torch.float32, "MultiHeadRMSNorm + apply_rotary_embedding")
    # the grid source and the phase-table source agree
    g2 = emb.grid_phases(16)
    assert torch.equal(g2, phases)


@pytest.mark.parametrize("dtype", DTYPES)
def test_config4_sparse_coords(dev, dtype):
    """Sparse positions from int coords (config 4 shells, coords up to 63)."""
    coords, offsets = workloads.config4()
    t, h, d = coords.shape[0], 12, 128
    q = storage_round(orc.randn(21, (t, h, d)), dtype)
    k = storage_round(orc.randn(22, (t, h, d)), dtype)
    gq, gk = _gammas(h, d, 23)
    phases = orc.rope_phases_from_coords(coords, d, orc.rope_freqs(d))
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    qo, ko = ops.qk_rmsnorm_rope(q=to_dev(q, dev, dtype), k=to_dev(k, dev, dtype), gamma_q=to_dev(gq, dev),
                                 gamma_k=to_dev(gk, dev), freqs=nn.rope_freqs(d), coords=to_dev(coords, dev))
    assert_close(qo, wq, dtype, f"sparse q {dtype}")
    assert_close(ko, wk, dtype, f"sparse k {dtype}")


def test_sparse_embedder_api(dev):
    """SparseRotaryPositionEmbedder.embed(q, k) after MultiHeadRMSNorm on a
    128^3 shell (coords up to 127, angles up to 127 rad)."""
    coords, offsets = workloads.shell_coords(128, 1, 60.0, 1.0, 2.0, seed=9)
    t, h, d = coords.shape[0], 12, 128
    q, k = orc.randn(31, (t, h, d)), orc.randn(32, (t, h, d))
    dq, dk = to_dev(q, dev), to_dev(k, dev)
    dco = to_dev(coords, dev)
    emb = sparse.SparseRotaryPositionEmbedder(d)
    sq = sparse.SparseTensor(dq, dco, 1)
    sk = sparse.SparseTensor(dk, dco, 1)
    rq, rk = emb.embed(sq, sk)
    phases = orc.rope_phases_from_coords(coords, d, orc.rope_freqs(d))
    assert_close(rq.feats, orc.rope_rotate(q, phases), torch.float32, "embed q")
    assert_close(rk.feats, orc.rope_rotate(k, phases), torch.float32, "embed k")
    assert_close(emb._compute_phases(sq), phases, torch.float32, "_compute_phases")


def test_packed_qkv_bias(dev):
    """bias_rms_rope_qkv semantics in place on [rows, 3, H, D]."""
    rows, h, d = 2048, 12, 128
    qkv = orc.randn(41, (rows, 3, h, d))
    bias = orc.randn(42, (3 * h * d,), std=0.1)
    gq, gk = _gammas(h, d, 43)
    freqs = orc.rope_freqs(d)
    phases = orc.rope_phases_from_positions(orc.grid_positions(16)[:rows], d, freqs)
    b3 = bias.reshape(3, h, d)
    wq, wk = orc.qk_rms_rope(qkv[:, 0], qkv[:, 1], gq, gk, phases, bias_q=b3[0], bias_k=b3[1])
    wv = (qkv[:, 2] + b3[2]).astype(np.float32)
    dq = to_dev(qkv.reshape(rows, -1), dev)
    ops.qkv_bias_rmsnorm_rope(dq, h, d, bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                              freqs=freqs, grid_res=16)
    got = host(dq).reshape(rows, 3, h, d)
    assert_close(got[:, 0], wq, torch.float32, "packed q")
    assert_close(got[:, 1], wk, torch.float32, "packed k")
    assert np.array_equal(got[:, 2], wv), "v bias must be bit-exact"


def test_views_into_packed_qkv(dev):
    """q and k as strided views of a packed qkv buffer, separate outputs."""
    rows, h, d = 1000, 12, 128
    qkv = orc.randn(51, (rows, 3, h, d))
    gq, gk = _gammas(h, d, 52)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = np.stack([np.arange(rows) % 17, (np.arange(rows) // 17) % 13, np.arange(rows) % 5], 1)
    dq = to_dev(qkv, dev)
    qo, ko = ops.qk_rmsnorm_rope(q=dq[:, 0], k=dq[:, 1], gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                                 freqs=orc.rope_freqs(d), coords=to_dev(coords, dev))
    phases = orc.rope_phases_from_coords(coords, d, orc.rope_freqs(d))
    wq, wk = orc.qk_rms_rope(qkv[:, 0], qkv[:, 1], gq, gk, phases)
    assert_close(qo, wq, torch.float32, "view q")
    assert_close(ko, wk, torch.float32, "view k")
    assert np.array_equal(host(dq), qkv), "inputs must be untouched"


@pytest.mark.parametrize("h,d", [(16, 64), (4, 128), (8, 64), (20, 128), (6, 96), (2, 32), (12, 256)])
def test_head_shapes(dev, h, d):
    """Fast path (D 64/128, H <= 16) and the generic per-(row, head) kernel."""
    rows = 300
    q, k = orc.randn(61, (rows, h, d)), orc.randn(62, (rows, h, d))
    gq, gk = _gammas(h, d, 63)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = (np.arange(rows * 3).reshape(rows, 3) * 5) % 31
    freqs = orc.rope_freqs(d)
    phases = orc.rope_phases_from_coords(coords, d, freqs)
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    qo, ko = ops.qk_rmsnorm_rope(q=to_dev(q, dev), k=to_dev(k, dev), gamma_q=to_dev(gq, dev),
                                 gamma_k=to_dev(gk, dev), freqs=freqs, coords=to_dev(coords, dev))
    assert_close(qo, wq, torch.float32, f"q H={h} D={d}")
    assert_close(ko, wk, torch.float32, f"k H={h} D={d}")


def test_rms_only_and_rope_only(dev):
    rows, h, d = 512, 12, 128
    q = orc.randn(71, (rows, h, d))
    gq, _ = _gammas(h, d, 72)
    got = nn.MultiHeadRMSNorm(d, h)
    got.gamma = to_dev(gq, dev)
    assert_close(got.forward(to_dev(q, dev)), orc.multihead_rmsnorm(q, gq), torch.float32, "rms only")
    z = np.zeros((4, h, d), np.float32)  # zero heads: the 1e-12 clamp keeps them 0
    assert np.all(host(got.forward(to_dev(z, dev))) == 0.0)
    ph = orc.rope_phases_from_positions(orc.grid_positions(8), d, orc.rope_freqs(d))
    x = orc.randn(73, (1, 512, h, d))
    out = nn.apply_rotary_embedding(to_dev(x, dev), to_dev(ph, dev))
    assert_close(out, orc.apply_rotary(x, ph), torch.float32, "rope only")


def test_rope_identity_and_norm(dev):
    """Position 0 is the identity; every pair keeps its norm."""
    rows, h, d = 256, 12, 128
    x = orc.randn(81, (rows, h, d))
    coords = np.zeros((rows, 4), np.int32)
    out, _ = ops.qk_rmsnorm_rope(q=to_dev(x, dev), freqs=orc.rope_freqs(d), coords=to_dev(coords, dev))
    assert np.array_equal(host(out), x)
    coords[:, 1:] = np.random.default_rng(0).integers(0, 128, (rows, 3))
    out, _ = ops.qk_rmsnorm_rope(q=to_dev(x, dev), freqs=orc.rope_freqs(d), coords=to_dev(coords, dev))
    o = host(out).reshape(rows, h, d // 2, 2).astype(np.float64)
    xi = x.reshape(rows, h, d // 2, 2).astype(np.float64)
    np.testing.assert_allclose(np.hypot(o[..., 0], o[..., 1]), np.hypot(xi[..., 0], xi[..., 1]), rtol=2e-6, atol=1e-6)
    # pad slot 63 (head_dim 128, 3 x 21 rotated slots) passes through untouched
    assert np.array_equal(host(out).reshape(rows, h, 64, 2)[:, :, 63], x.reshape(rows, h, 64, 2)[:, :, 63])


def test_phase_builder_sources(dev):
    d = 128
    freqs = orc.rope_freqs(d)
    coords, _ = workloads.config4()
    got = ops.rope_phases(coords.shape[0], d, freqs, coords=to_dev(coords, dev))
    want = orc.rope_phases_from_coords(coords, d, freqs)
    assert max_err(got, want) <= 2e-7
    assert np.array_equal(host(got)[:, 63], np.tile([1.0, 0.0], (coords.shape[0], 1)).astype(np.float32))
    pos = orc.randn(91, (500, 3), std=30.0)
    got = ops.rope_phases(500, d, freqs, positions=to_dev(pos, dev))
    assert max_err(got, orc.rope_phases_from_positions(pos, d, freqs)) <= 2e-7


def test_qk_errors(dev):
    with pytest.raises(ValueError):
        nn.apply_rotary_embedding(torch.zeros((1, 8, 12, 128), device=dev), torch.zeros((4, 64, 2), device=dev))
    with pytest.raises(ValueError, match="head_dim must be even"):
        nn.RotaryPositionEmbedder(127)
    with pytest.raises(ValueError):  # RoPE without a position source
        ops.qk_rmsnorm_rope(q=torch.zeros((4, 12, 128), device=dev), freqs=orc.rope_freqs(128))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("h", [4, 6, 8, 12, 16])
@pytest.mark.parametrize("source", ["coords", "grid", "table"])
@pytest.mark.parametrize("d", [128, 64])
def test_16bit_head_groups_and_sources(dev, dtype, h, source, d):
    """16-bit rows: head_dim 128 (config 5's storage) in 1-4 groups of 4
    heads per wave instruction (16 lanes a head), head_dim 64 (the SLat
    DiT's) in 1-2 groups of 8 (8 lanes a head), with idle tails (6 or 12
    heads), 301 rows (a partial last tile), the three position sources (int
    coords, the dense grid index, a phase table), q and k biases, against
    the oracle; then q alone in place, and the packed qkv with its v bias
    (bit-exact after one rounding)."""
    rows = 301
    q = storage_round(orc.randn(1000 + h, (rows, h, d)), dtype)
    k = storage_round(orc.randn(1001 + h, (rows, h, d)), dtype)
    gq, gk = _gammas(h, d, 1002 + h)
    bq, bk = orc.randn(1004 + h, (h, d), std=0.1), orc.randn(1005 + h, (h, d), std=0.1)
    freqs = orc.rope_freqs(d)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = np.random.default_rng(h).integers(0, 128, (rows, 3))
    src = {}
    if source == "coords":
        phases = orc.rope_phases_from_coords(coords, d, freqs)
        src = dict(coords=to_dev(coords, dev))
    elif source == "grid":
        phases = orc.rope_phases_from_positions(np.tile(orc.grid_positions(8), (2, 1))[:rows], d, freqs)
        src = dict(grid_res=8)
    else:
        phases = orc.rope_phases_from_positions(orc.randn(1006, (rows, 3), std=40.0), d, freqs)
        src = dict(phases=to_dev(phases, dev))
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases, bias_q=bq, bias_k=bk)
    dq, dk = to_dev(q, dev, dtype), to_dev(k, dev, dtype)
    qo, ko = ops.qk_rmsnorm_rope(q=dq, k=dk, gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                                 bias_q=to_dev(bq, dev), bias_k=to_dev(bk, dev), freqs=freqs, **src)
    assert_close(qo, wq, dtype, f"q {dtype} H={h} {source}")
    assert_close(ko, wk, dtype, f"k {dtype} H={h} {source}")
    ops.qk_rmsnorm_rope(q=dq, gamma_q=to_dev(gq, dev), freqs=freqs, in_place=True, **src)
    wq1, _ = orc.qk_rms_rope(q, k, gq, gk, phases)
    assert_close(dq, wq1, dtype, f"q in place {dtype} H={h} {source}")
    qkv = storage_round(orc.randn(1007 + h, (rows, 3, h, d)), dtype)
    bias = orc.randn(1008 + h, (3 * h * d,), std=0.1)
    b3 = bias.reshape(3, h, d)
    dqkv = to_dev(qkv.reshape(rows, -1), dev, dtype)
    ops.qkv_bias_rmsnorm_rope(dqkv, h, d, bias=to_dev(bias, dev), gamma_q=to_dev(gq, dev), gamma_k=to_dev(gk, dev),
                              freqs=freqs, **src)
    got = dqkv.reshape(rows, 3, h, d)
    pq, pk = orc.qk_rms_rope(qkv[:, 0], qkv[:, 1], gq, gk, phases, bias_q=b3[0], bias_k=b3[1])
    assert_close(got[:, 0], pq, dtype, "packed q")
    assert_close(got[:, 1], pk, dtype, "packed k")
    assert bits_equal(got[:, 2].contiguous(), (qkv[:, 2] + b3[2]).astype(np.float32), dtype), "v bias"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("res", [5, 12, 16, 1500])
def test_dense_grid_sizes(dev, dtype, res):
    """The dense-grid position source for grid sizes that are and are not
    powers of two, one past 2^31 when cubed (R = 1500), over 3000 rows, so
    the smaller grids wrap (row r sits at l = r % R^3), against the oracle
    with the positions written out here (the oracle's grid for R <= 16 is
    checked against them first)."""
    rows, h, d = 3000, 12, 128
    r = np.arange(rows, dtype=np.int64)
    l = r % res ** 3
    pos = np.stack([l // (res * res), (l // res) % res, l % res], axis=1).astype(np.float32)
    if res <= 16:
        assert np.array_equal(np.tile(orc.grid_positions(res), (rows // res ** 3 + 1, 1))[:rows], pos)
    q = storage_round(orc.randn(1200 + res, (rows, h, d)), dtype)
    k = storage_round(orc.randn(1201 + res, (rows, h, d)), dtype)
    gq, gk = _gammas(h, d, 1202)
    freqs = orc.rope_freqs(d)
    phases = orc.rope_phases_from_positions(pos, d, freqs)
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    qo, ko = ops.qk_rmsnorm_rope(q=to_dev(q, dev, dtype), k=to_dev(k, dev, dtype), gamma_q=to_dev(gq, dev),
                                 gamma_k=to_dev(gk, dev), freqs=freqs, grid_res=res)
    assert_close(qo, wq, dtype, f"q {dtype} R={res}")
    assert_close(ko, wk, dtype, f"k {dtype} R={res}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [2048, 2369])
def test_reference_block_geometry(dev, dtype, rows):
    """QK RMSNorm + RoPE at the attention geometry of the reference's
    whole-block GPU cases (tests/parity/parity_wp11_gpu_attn.mojo:495-536:
    width 1024 as 16 heads of 64, L = 2048 dense on the 16^3 grid's first
    rows, T = 2369 sparse from coords) against the oracle."""
    h, d = 16, 64
    q = storage_round(orc.randn(1100 + rows, (rows, h, d)), dtype)
    k = storage_round(orc.randn(1101 + rows, (rows, h, d)), dtype)
    gq, gk = _gammas(h, d, 1102)
    freqs = orc.rope_freqs(d)
    if rows == 2048:
        phases = orc.rope_phases_from_positions(orc.grid_positions(16)[:rows], d, freqs)
        src = dict(grid_res=16)
    else:
        coords = np.zeros((rows, 4), np.int32)
        coords[:, 1:] = np.random.default_rng(rows).integers(0, 64, (rows, 3))
        phases = orc.rope_phases_from_coords(coords, d, freqs)
        src = dict(coords=to_dev(coords, dev))
    wq, wk = orc.qk_rms_rope(q, k, gq, gk, phases)
    qo, ko = ops.qk_rmsnorm_rope(q=to_dev(q, dev, dtype), k=to_dev(k, dev, dtype), gamma_q=to_dev(gq, dev),
                                 gamma_k=to_dev(gk, dev), freqs=freqs, **src)
    assert_close(qo, wq, dtype, f"q {dtype} rows={rows}")
    assert_close(ko, wk, dtype, f"k {dtype} rows={rows}")
