"""Host-side logic of the t2h package that needs no GPU (CPU torch tensors):
the VarLenTensor layout against the reference's own expectations
(tests/parity/test_sparse_basic.mojo:22-27, 47-71)."""
import pytest
import torch

from t2h.sparse import VarLenTensor


def make_varlen():
    # batch 0: 2 rows, batch 1: 3 rows; C = 2 (test_sparse_basic.mojo:22-27)
    feats = torch.arange(1, 11, dtype=torch.float32).reshape(5, 2)
    return VarLenTensor(feats, [0, 2, 5])


def test_varlen_shape_and_layout():
    x = make_varlen()
    assert x.batch_size() == 2 and len(x) == 2
    assert x.shape() == [2, 2]
    assert x.seqlen(0) == 2 and x.seqlen(1) == 3 and x.seqlen_list() == [2, 3]
    assert x.batch_broadcast_map() == [0, 0, 1, 1, 1]


def test_varlen_roundtrip():
    x = make_varlen()
    parts = x.to_tensor_list()
    assert len(parts) == 2 and parts[1].shape[0] == 3 and parts[1].reshape(-1)[0].item() == 5.0
    y = VarLenTensor.from_tensor_list(parts)
    assert torch.equal(y.feats, x.feats) and y.offsets[2] == 5
    assert VarLenTensor.offsets_from_seqlen([2, 0, 3]) == [0, 2, 2, 5]


@pytest.mark.parametrize("offsets", [[1, 2, 5], [0, 3, 2, 5], [0, 2, 4], []])
def test_varlen_invalid_offsets(offsets):
    with pytest.raises(ValueError, match="VarLenTensor: invalid offsets"):
        VarLenTensor(torch.zeros(5, 2), offsets)


def test_varlen_replace_checks_rows():
    x = make_varlen()
    with pytest.raises(ValueError, match="row count mismatch"):
        x.replace(torch.zeros(4, 2))
    assert x.replace(torch.ones(5, 3)).offsets == [0, 2, 5]
