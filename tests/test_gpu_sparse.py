"""GPU: SparseTensor layout and batch-id gather, bit-exact. The hand-computed
cases are those of the reference's tests/parity/test_sparse_basic.mojo
(make_sparse 28-43; elemwise_batch 73-91, 261-268; layout 149-158;
contiguity 161-171), here run through libt2h's offsets and gather kernels."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import host, to_dev
from t2h import _lib, ops, sparse, workloads

pytestmark = pytest.mark.gpu


def make_sparse(dev):
    feats = np.arange(1, 11, dtype=np.float32).reshape(5, 2)
    coords = np.array([[0, 0, 0, 0], [0, 1, 0, 1], [1, 0, 1, 0], [1, 1, 1, 1], [1, 1, 0, 0]], np.int32)
    return sparse.SparseTensor(to_dev(feats, dev), to_dev(coords, dev))


def test_sparse_layout_from_coords(dev):
    x = make_sparse(dev)
    assert x.batch_size() == 2
    assert x.seqlen(0) == 2 and x.seqlen(1) == 3
    assert host(x.offsets).astype(np.int64).tolist() == [0, 2, 5]


def test_sparse_elemwise_batch(dev):
    x = make_sparse(dev)
    b = to_dev(np.array([[10, 20], [100, 200]], np.float32), dev)
    y = x.elemwise_batch(b, sparse.OP_ADD)
    assert host(y.feats).reshape(-1)[0] == 11.0
    assert host(y.feats).reshape(-1)[9] == 210.0
    m = x.elemwise_batch(b, sparse.OP_MUL)
    assert host(m.feats).reshape(-1)[1] == 40.0
    # per-batch scalar [B, 1]
    s = x.elemwise_batch(to_dev(np.array([[10], [100]], np.float32), dev), sparse.OP_ADD)
    assert host(s.feats).reshape(-1)[0] == 11.0
    assert host(s.feats).reshape(-1)[4] == 105.0
    s2 = x.elemwise_batch(to_dev(np.array([[10, 20], [100, 200]], np.float32), dev), sparse.OP_ADD)
    assert host(s2.feats).reshape(-1)[1] == 22.0


def test_sparse_contiguity_enforced(dev):
    coords = np.zeros((2, 4), np.int32)
    coords[0, 0] = 1  # batch 1 before batch 0 -> must raise
    with pytest.raises(ValueError, match="ordered/contiguous"):
        sparse.SparseTensor(torch.zeros((2, 1), device=dev), to_dev(coords, dev), 2)
    coords = np.zeros((3, 4), np.int32)
    coords[2, 0] = 5
    with pytest.raises(ValueError, match="out of range"):
        sparse.SparseTensor(torch.zeros((3, 1), device=dev), to_dev(coords, dev), 2)


def test_first_bad_row_order(dev):
    """The first offending row decides the error, order checked before range
    (sparse/basic.mojo:327-332)."""
    coords = np.zeros((6, 4), np.int32)
    coords[:, 0] = [0, 0, 1, 9, 0, 1]   # row 3 out of range comes before row 4 unordered
    off, bad = ops.coords_to_offsets_async(to_dev(coords, dev), 2)
    assert int(bad.item()) == (3 << 1) | 1
    coords[:, 0] = [0, 1, 0, 9, 0, 1]   # row 2 unordered first
    off, bad = ops.coords_to_offsets_async(to_dev(coords, dev), 2)
    assert int(bad.item()) == (2 << 1) | 0


@pytest.mark.parametrize("batches", [[5], [0, 3], [3, 0], [2, 0, 0, 4, 0], [0, 0, 0], [1, 1, 1, 1, 1, 1, 1]])
def test_offsets_and_gather_with_empty_batches(dev, batches):
    nb = len(batches)
    coords = np.zeros((sum(batches), 4), np.int32)
    coords[:, 0] = np.repeat(np.arange(nb), batches)
    want = orc.cal_offsets(coords, nb)
    got = ops.coords_to_offsets(to_dev(coords, dev), nb)
    assert np.array_equal(host(got).astype(np.int64), want)
    if coords.shape[0]:
        x = orc.randn(1, (coords.shape[0], 1536))
        sh = orc.randn(2, (nb, 1536))
        sc = orc.randn(3, (nb, 1536))
        g = ops.modulate(to_dev(x, dev), to_dev(sh, dev), to_dev(sc, dev), offsets=got)
        assert np.array_equal(host(g), orc.mod_shift_scale(x, sh, sc, want))


def test_gather_config4_bit_exact(dev):
    coords, offsets = workloads.config4()
    got = ops.coords_to_offsets(to_dev(coords, dev), 2)
    assert np.array_equal(host(got).astype(np.int64), offsets)
    assert np.array_equal(offsets, orc.cal_offsets(coords, 2))
    x = orc.randn(11, (coords.shape[0], 1536))
    other = orc.randn(12, (2, 1536))
    rm = orc.batch_broadcast_map(offsets)
    for op in (sparse.OP_ADD, sparse.OP_SUB, sparse.OP_MUL, sparse.OP_DIV):
        g = ops.binop_rows(to_dev(x, dev), to_dev(other, dev), op, offsets=got)
        assert np.array_equal(host(g), orc.binop_rows(x, other, rm, op)), f"op {op}"


def test_host_wrapper_errors(dev):
    import ctypes

    L = _lib.load()
    coords = np.zeros((2, 4), np.int32)
    coords[0, 0] = 1
    off = np.zeros(3, np.int64)
    rc = L.t2h_h_coords_to_offsets(coords.ctypes.data, 2, 4, 2, off.ctypes.data)
    assert rc == _lib.T2H_EBATCH_ORDER
    assert b"ordered/contiguous" in L.t2h_last_error()
    coords[0, 0] = 0
    coords[1, 0] = 1
    rc = L.t2h_h_coords_to_offsets(coords.ctypes.data, 2, 4, 2, off.ctypes.data)
    assert rc == 0 and off.tolist() == [0, 1, 2]
    x = orc.randn(5, (16, 1536))
    out = np.empty_like(x)
    rc = L.t2h_h_ln_modulate(x.ctypes.data, out.ctypes.data, 16, 1536, ctypes.c_float(1e-6), 0, None, None, None,
                             1, 0)
    assert rc == 0
    assert np.max(np.abs(out - orc.layernorm(x, 1e-6))) < 1e-5


def test_varlen_elemwise_reference_cases(dev):
    """tests/parity/test_sparse_basic.mojo:73-91 on the device: scalar ops,
    flat add, negation, per-batch [B, 1] and [B, C] broadcasts; plus the
    reverse scalar forms (value - x, value / x)."""
    feats = torch.arange(1, 11, dtype=torch.float32, device=dev).reshape(5, 2)
    x = sparse.VarLenTensor(feats, [0, 2, 5])
    y = (x + 1.0) * 2.0
    assert y.feats.reshape(-1)[0].item() == 4.0 and y.feats.reshape(-1)[9].item() == 22.0
    z = x + x
    assert z.feats.reshape(-1)[3].item() == 8.0
    n = -x
    assert n.feats.reshape(-1)[0].item() == -1.0
    b = torch.tensor([[10.0], [100.0]], device=dev)
    w = x.elemwise_batch(b, sparse.OP_ADD)
    assert w.feats.reshape(-1)[0].item() == 11.0 and w.feats.reshape(-1)[4].item() == 105.0
    b2 = torch.tensor([[10.0, 20.0], [100.0, 200.0]], device=dev)
    w2 = x.elemwise_batch(b2, sparse.OP_ADD)
    assert w2.feats.reshape(-1)[1].item() == 22.0 and w2.feats.reshape(-1)[9].item() == 210.0
    f = host(feats)
    assert np.array_equal(host(x.elemwise_scalar(1.0, sparse.OP_SUB, reverse=True).feats), np.float32(1.0) - f)
    assert np.array_equal(host(x.elemwise_scalar(3.0, sparse.OP_DIV, reverse=True).feats), np.float32(3.0) / f)
    assert np.array_equal(host((x / 3.0).feats), f / np.float32(3.0))
    assert np.array_equal(host((x - 0.5).feats), f - np.float32(0.5))
    with pytest.raises(ValueError, match="batch size mismatch"):
        x.elemwise_batch(torch.ones((3, 1), device=dev), sparse.OP_ADD)


def test_sparse_vl_view(dev):
    coords, offsets = workloads.config4()
    st = sparse.SparseTensor(torch.zeros((coords.shape[0], 4), device=dev), to_dev(coords, dev), 2)
    v = st.vl
    assert v.offsets == [int(o) for o in offsets] and v.feats is st.feats
    assert v.batch_size() == 2
