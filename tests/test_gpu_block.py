"""GPU parity: the per-token glue of one DiT cross block, end to end, through
the C ABI.

* Resident form (gpu/block.mojo:217-397): the const buffer `bk`, the Metal
  kernels' mirrors t2h_ln_mod_rows / t2h_gate_add_bias_rows, and the fused
  join + norm t2h_block_join_ln.
* CPU-order form for dense [N, L, C] and sparse feats with B batches
  (modules/transformer/modulated.mojo:177-200,
  sparse/transformer/modulated.mojo:187-226).

The attention / MLP chains are GEMM and SDPA work outside this library; the
tests pass stand-ins that the device and the oracle compute identically (a
row roll times 0.5, a column flip times -0.25: exact in every storage type)
or to tolerance (GELU-tanh through t2h vs the oracle). Metric and tolerances:
tests/_parity.py.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, host, storage_round, to_dev
from t2h import block, ops, sparse, workloads

pytestmark = pytest.mark.gpu


def dev_chains():
    return (lambda h: torch.roll(h, 1, 0) * 0.5,
            lambda h: torch.flip(h, [1]) * -0.25,
            lambda h: ops.activation(h, ops.ACT_GELU_TANH))


def orc_chains():
    return (lambda h: (np.roll(h, 1, axis=0) * np.float32(0.5)).astype(np.float32),
            lambda h: (h[:, ::-1] * np.float32(-0.25)).astype(np.float32),
            lambda h: orc.activation(h, orc.ACT_GELU_TANH))


def block_params(seed, c, nb=1):
    m = [orc.randn(seed + i, (nb, c), std=0.1) for i in range(6)]
    w2 = orc.randn(seed + 6, (c,), mean=1.0, std=0.1)
    b2 = orc.randn(seed + 7, (c,), std=0.05)
    biases = [orc.randn(seed + 8 + i, (c,), std=0.02) for i in range(3)]
    return m, w2, b2, biases


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("fused", [True, False])
def test_resident_block_glue(dev, dtype, fused):
    """One resident block at width 1536 over 4096 rows (config-1 shape)."""
    rows, c = 4096, 1536
    x = orc.randn(1100, (rows, c))
    m, w2, b2, biases = block_params(1101, c)
    bk = block.pack_block_consts([to_dev(mm, dev) for mm in m], to_dev(w2, dev), to_dev(b2, dev),
                                 *[to_dev(b, dev) for b in biases])
    xs = to_dev(x, dev, dtype)
    out = block.cross_block_enqueue(xs, bk, *dev_chains(), fused=fused)
    assert out.data_ptr() == xs.data_ptr(), "the block must update x in place"
    rnd = lambda a: storage_round(a, dtype)
    want = orc.cross_block_resident(rnd(x), host(bk), *orc_chains(), store=rnd)
    assert_close(out, want, dtype, f"resident block {dtype} fused={fused}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_resident_fused_equals_unfused(dev, dtype):
    """Fusing a join with the next norm changes no bit: the norm reads the
    join's stored value either way."""
    rows, c = 2048, 1536
    x = orc.randn(1200, (rows, c))
    m, w2, b2, biases = block_params(1201, c)
    bk = block.pack_block_consts([to_dev(mm, dev) for mm in m], to_dev(w2, dev), to_dev(b2, dev),
                                 *[to_dev(b, dev) for b in biases])
    a = block.cross_block_enqueue(to_dev(x, dev, dtype), bk, *dev_chains(), fused=True)
    b = block.cross_block_enqueue(to_dev(x, dev, dtype), bk, *dev_chains(), fused=False)
    assert torch.equal(a, b)


def test_resident_mirrors_in_place_and_aliasing(dev):
    """ln_mod_rows may write over its input (the Metal kernel's thread reads
    its row before writing it); the chains may work in place on hs."""
    rows, c = 1000, 1536
    x = orc.randn(1300, (rows, c))
    m, w2, b2, biases = block_params(1301, c)
    bk = block.pack_block_consts([to_dev(mm, dev) for mm in m], to_dev(w2, dev), to_dev(b2, dev),
                                 *[to_dev(b, dev) for b in biases])
    xd = to_dev(x, dev)
    y = ops.ln_mod_rows(xd, torch.empty_like(xd), bk, 4 * c, 2)
    ops.ln_mod_rows(xd, xd, bk, 4 * c, 2)
    assert torch.equal(xd, y)
    assert_close(y, orc.layernorm(x, 1e-6, True, w2, b2), torch.float32, "ln_mod_rows affine")

    def self_in_place(h):
        return h.mul_(0.5)
    sc, cc, mc = dev_chains()
    xs = to_dev(x, dev)
    block.cross_block_enqueue(xs, bk, self_in_place, cc, mc)
    want = orc.cross_block_resident(x, host(bk), lambda h: (h * np.float32(0.5)).astype(np.float32),
                                    *orc_chains()[1:])
    assert_close(xs, want, torch.float32, "in-place chain")


def test_resident_errors(dev):
    c = 256
    x = torch.zeros(8, c, device=dev)
    bk = torch.zeros(12 * c, device=dev)
    with pytest.raises(ValueError, match="bad mode 3"):
        ops.ln_mod_rows(x, torch.empty_like(x), bk, 0, 3)
    with pytest.raises(ValueError, match="outside a buffer"):
        ops.gate_add_bias_rows(x, x.clone(), bk, 11 * c, 1)
    with pytest.raises(ValueError, match="must not alias"):
        ops.block_join_ln(x, x.clone(), x, bk, 2 * c, 1, 4 * c, 2)
    with pytest.raises(ValueError, match="consts must hold"):
        block.cross_block_enqueue(x, bk[:11 * c], *dev_chains())
    with pytest.raises(ValueError, match="self chain returned"):
        block.cross_block_enqueue(x, bk, lambda h: h[:4], *dev_chains()[1:])


def test_dense_cross_block_batches(dev):
    """Dense [N, L, C] with N = 2: each batch row uses its own chunk row
    (share_mod Modulation: mod [2, 6C] + modulation [6C])."""
    n, l, c = 2, 777, 1536
    x = orc.randn(1400, (n, l, c))
    mod = orc.randn(1401, (n, 6 * c), std=0.1)
    modulation = orc.randn(1402, (6 * c,), std=0.1)
    w2 = orc.randn(1403, (c,), mean=1.0, std=0.1)
    b2 = orc.randn(1404, (c,), std=0.05)
    blk = block.ModulatedCrossBlock(c, to_dev(w2, dev), to_dev(b2, dev), modulation=to_dev(modulation, dev))
    sc, cc, mc = dev_chains()
    got = blk(to_dev(x, dev), to_dev(mod, dev), lambda h: sc(h.reshape(n * l, c)), cc, mc)
    assert got.shape == (n, l, c)
    mm = orc.modulation_add(mod, modulation)
    chunks = [mm[:, i * c:(i + 1) * c] for i in range(6)]
    osc, occ, omc = orc_chains()
    want = orc.cross_block(x.reshape(n * l, c), chunks, w2, b2, osc, occ, omc,
                           offsets=np.array([0, l, 2 * l], np.int64))
    assert_close(got.reshape(n * l, c), want, torch.float32, "dense block N=2")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_sparse_cross_block_config4(dev, dtype):
    """Sparse feats on the config-4 layout (B = 2 shells on 64^3, T = 39,804):
    the chunk row of each token follows its batch through the offsets."""
    coords, offsets = workloads.config4()
    t, c = coords.shape[0], 1536
    x = orc.randn(1500, (t, c))
    mod = orc.randn(1501, (2, 6 * c), std=0.1)
    w2 = orc.randn(1502, (c,), mean=1.0, std=0.1)
    b2 = orc.randn(1503, (c,), std=0.05)
    st = sparse.SparseTensor(to_dev(x, dev, dtype), to_dev(coords, dev), 2)
    blk = block.ModulatedCrossBlock(c, to_dev(w2, dev), to_dev(b2, dev))
    got = blk(st, to_dev(mod, dev), *dev_chains())
    assert isinstance(got, sparse.SparseTensor) and got.feats.dtype == dtype
    chunks = [mod[:, i * c:(i + 1) * c] for i in range(6)]
    rnd = lambda a: storage_round(a, dtype)
    want = orc.cross_block(rnd(x), chunks, w2, b2, *orc_chains(), offsets=offsets, store=rnd)
    assert_close(got.feats, want, dtype, f"sparse block {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("form", ["resident", "dense", "sparse"])
def test_reference_block_geometry(dev, dtype, form):
    """The per-token glue at the geometry of the reference's whole-block GPU
    parity cases (tests/parity/parity_wp11_gpu_attn.mojo:495-536: width
    1024, a dense block of L = 2048 and a sparse block of T = 2369 tokens):
    the resident form over the const buffer, the dense [1, L, C] block and
    the sparse feats, against the oracle."""
    c = 1024
    rows = 2369 if form == "sparse" else 2048
    x = orc.randn(1600 + rows, (rows, c))
    rnd = lambda a: storage_round(a, dtype)
    m, w2, b2, biases = block_params(1601, c)
    if form == "resident":
        bk = block.pack_block_consts([to_dev(mm, dev) for mm in m], to_dev(w2, dev), to_dev(b2, dev),
                                     *[to_dev(b, dev) for b in biases])
        got = block.cross_block_enqueue(to_dev(x, dev, dtype), bk, *dev_chains(), fused=True)
        want = orc.cross_block_resident(rnd(x), host(bk), *orc_chains(), store=rnd)
        assert_close(got, want, dtype, f"resident block C=1024 {dtype}")
        return
    mod = np.concatenate(m, axis=1)   # [1, 6C]: the six chunks in adaLN order
    blk = block.ModulatedCrossBlock(c, to_dev(w2, dev), to_dev(b2, dev))
    if form == "dense":
        got = blk(to_dev(x, dev, dtype).reshape(1, rows, c), to_dev(mod, dev),
                  lambda h: dev_chains()[0](h.reshape(rows, c)), *dev_chains()[1:]).reshape(rows, c)
    else:
        coords = np.zeros((rows, 4), np.int32)
        coords[:, 1:] = np.stack([np.arange(rows) // 256, (np.arange(rows) // 16) % 16, np.arange(rows) % 16], 1)
        st = sparse.SparseTensor(to_dev(x, dev, dtype), to_dev(coords, dev), 1)
        got = blk(st, to_dev(mod, dev), *dev_chains()).feats
    want = orc.cross_block(rnd(x), m, w2, b2, *orc_chains(), offsets=np.array([0, rows], np.int64), store=rnd)
    assert_close(got, want, dtype, f"{form} block C=1024 {dtype}")
