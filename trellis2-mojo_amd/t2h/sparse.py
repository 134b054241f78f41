"""SparseTensor feature rows on the MI355X path.

Mirror of the reference's SparseTensor data model (sparse/basic.mojo:296-339):
feats [N, *tail] + int32 coords [N, 4] = (batch, x, y, z), rows of a batch
contiguous and batches ordered; offsets [B+1] computed on the device from
coords[:, 0] with the reference's two errors. The per-batch ops gather the
[B, C] parameter row of each token row through the offsets.

Reference: sparse/basic.mojo (VarLenTensor 89-155, SparseTensor 296-339,
elemwise_batch 433-439), sparse/transformer/modulated.mojo (Modulation.chunks
24-57, _mod_shift_scale 60-65), sparse/attention/rope.mojo (embedder 20-134).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .nn import rope_freqs

OP_ADD, OP_SUB, OP_MUL, OP_DIV = ops.OP_ADD, ops.OP_SUB, ops.OP_MUL, ops.OP_DIV
_REVERSE = {OP_SUB: ops.OP_RSUB, OP_DIV: ops.OP_RDIV, OP_ADD: OP_ADD, OP_MUL: OP_MUL}


def _offsets_ok(offsets, total_rows: int) -> bool:
    """sparse/basic.mojo:76-82."""
    if len(offsets) < 1 or offsets[0] != 0:
        return False
    if any(b < a for a, b in zip(offsets, offsets[1:])):
        return False
    return offsets[-1] == total_rows


class VarLenTensor:
    """feats [T, *tail] with host offsets [B+1]: batch b owns rows
    [offsets[b], offsets[b+1]) (sparse/basic.mojo:89-247). The tensor math
    runs in libt2h kernels (bit-exact f32 sequences); the offsets also live on
    the device, once, for the per-batch gathers."""

    def __init__(self, feats: torch.Tensor, offsets):
        offsets = [int(o) for o in offsets]
        if not _offsets_ok(offsets, feats.shape[0]):
            raise ValueError("VarLenTensor: invalid offsets")
        self.feats = feats
        self.offsets = offsets
        self._dev_offsets: Optional[torch.Tensor] = None

    @staticmethod
    def offsets_from_seqlen(seqlen):
        out, start = [0], 0
        for n in seqlen:
            start += int(n)
            out.append(start)
        return out

    @classmethod
    def from_tensor_list(cls, tensors) -> "VarLenTensor":
        return cls(torch.cat(list(tensors), dim=0), cls.offsets_from_seqlen([t.shape[0] for t in tensors]))

    def to_tensor_list(self):
        return [self.feats[self.offsets[b]:self.offsets[b + 1]] for b in range(self.batch_size())]

    def batch_size(self) -> int:
        return len(self.offsets) - 1

    __len__ = batch_size

    def shape(self):
        return [self.batch_size(), *self.feats.shape[1:]]

    def seqlen(self, b: int) -> int:
        return self.offsets[b + 1] - self.offsets[b]

    def seqlen_list(self):
        return [self.seqlen(b) for b in range(self.batch_size())]

    def batch_broadcast_map(self):
        """Row -> batch index, on the host (sparse/basic.mojo:149-155)."""
        return [b for b in range(self.batch_size()) for _ in range(self.seqlen(b))]

    def device_offsets(self) -> torch.Tensor:
        if self._dev_offsets is None or self._dev_offsets.device != self.feats.device:
            self._dev_offsets = torch.tensor(self.offsets, dtype=torch.int64, device=self.feats.device)
        return self._dev_offsets

    def replace(self, feats: torch.Tensor) -> "VarLenTensor":
        if feats.shape[0] != self.feats.shape[0]:
            raise ValueError("VarLenTensor.replace: row count mismatch")
        out = VarLenTensor.__new__(VarLenTensor)
        out.feats, out.offsets, out._dev_offsets = feats, self.offsets, self._dev_offsets
        return out

    def _rows2d(self):
        f = self.feats.contiguous()
        t = f.shape[0]
        return f, f.reshape(t, f.numel() // t if t else 1)

    def elemwise_batch(self, other: torch.Tensor, op: int) -> "VarLenTensor":
        """feats[r] OP other[b(r)], other [B, row] or [B, 1] (sparse/basic.mojo:204-207)."""
        if other.shape[0] != self.batch_size():
            raise ValueError("VarLenTensor.elemwise_batch: batch size mismatch")
        f, f2 = self._rows2d()
        oth = other.reshape(other.shape[0], -1).to(device=f.device, dtype=torch.float32).contiguous()
        return self.replace(ops.binop_rows(f2, oth, op, offsets=self.device_offsets()).reshape(f.shape))

    def elemwise_scalar(self, value: float, op: int, reverse: bool = False) -> "VarLenTensor":
        """feats OP value (or value OP feats), one f32 rounding (sparse/basic.mojo:201-202)."""
        f, f2 = self._rows2d()
        s = torch.full((1, 1), float(value), dtype=torch.float32, device=f.device)
        return self.replace(ops.binop_rows(f2, s, _REVERSE[op] if reverse else op).reshape(f.shape))

    def __add__(self, other):
        if isinstance(other, VarLenTensor):
            if other.feats.numel() != self.feats.numel():
                raise ValueError("Tensor binop: size mismatch")
            f, f2 = self._rows2d()
            _, o2 = other._rows2d()
            return self.replace(ops.gate_residual(f2, o2).reshape(f.shape))
        return self.elemwise_scalar(other, OP_ADD)

    def __sub__(self, value: float):
        return self.elemwise_scalar(value, OP_SUB)

    def __mul__(self, value: float):
        return self.elemwise_scalar(value, OP_MUL)

    def __truediv__(self, value: float):
        return self.elemwise_scalar(value, OP_DIV)

    def __neg__(self):
        return self.elemwise_scalar(-1.0, OP_MUL)


class SparseTensor:
    def __init__(self, feats: torch.Tensor, coords: torch.Tensor, batch_size: int = -1,
                 offsets: Optional[torch.Tensor] = None):
        if feats.shape[0] != coords.shape[0]:
            raise ValueError("SparseTensor: feats/coords row mismatch")
        if coords.dtype != torch.int32 or coords.dim() != 2:
            raise ValueError("SparseTensor: coords must be int32 [N, 4]")
        self.feats = feats
        self.coords = coords.contiguous()
        b = batch_size
        if b < 0:
            if coords.shape[0] == 0:
                raise ValueError("IntMatrix.col_max: empty matrix")
            b = int(self.coords[:, 0].max().item()) + 1
        self._batch_size = b
        self.offsets = offsets if offsets is not None else ops.coords_to_offsets(self.coords, b)

    def batch_size(self) -> int:
        return self._batch_size

    @property
    def vl(self) -> VarLenTensor:
        """The reference's `x.vl` (feats + offsets, sparse/basic.mojo:296-319);
        the offsets come to the host once."""
        v = VarLenTensor(self.feats, self.offsets.cpu().tolist())
        v._dev_offsets = self.offsets
        return v

    def seqlen(self, b: int) -> int:
        return int(self.offsets[b + 1].item() - self.offsets[b].item())

    def replace(self, feats: torch.Tensor) -> "SparseTensor":
        if feats.shape[0] != self.feats.shape[0]:
            raise ValueError("VarLenTensor.replace: row count mismatch")
        return SparseTensor(feats, self.coords, self._batch_size, self.offsets)

    def elemwise_batch(self, other: torch.Tensor, op: int) -> "SparseTensor":
        """feats[r] OP other[b(r)] with other [B, C] or [B, 1] (basic.mojo:433-436)."""
        if other.shape[0] != self._batch_size:
            raise ValueError("SparseTensor.elemwise_batch: batch size mismatch")
        f = self.feats.contiguous()
        c = f.numel() // f.shape[0] if f.shape[0] else 0
        oth = other.reshape(other.shape[0], -1).to(torch.float32).contiguous()
        out = ops.binop_rows(f.reshape(-1, c), oth, op, offsets=self.offsets)
        return self.replace(out.reshape(f.shape))

    def __add__(self, other: "SparseTensor") -> "SparseTensor":
        """Elementwise feats add (sparse/basic.mojo:438-439)."""
        if other.feats.numel() != self.feats.numel():
            raise ValueError("Tensor binop: size mismatch")
        c = self.feats.shape[-1]
        out = ops.gate_residual(self.feats.contiguous().reshape(-1, c), other.feats.contiguous().reshape(-1, c))
        return self.replace(out.reshape(self.feats.shape))


def _mod_shift_scale(h: SparseTensor, shift: torch.Tensor, scale: torch.Tensor) -> SparseTensor:
    """h * (1 + scale) + shift with [B, C] batch broadcast
    (sparse/transformer/modulated.mojo:60-65)."""
    if shift.shape[0] != h.batch_size() or scale.shape[0] != h.batch_size():
        raise ValueError("SparseTensor.elemwise_batch: batch size mismatch")
    f = h.feats.contiguous()
    return h.replace(ops.modulate(f, shift, scale, offsets=h.offsets))


def norm_mod_shift_scale(h: SparseTensor, eps: float, shift: torch.Tensor, scale: torch.Tensor) -> SparseTensor:
    """`_mod_shift_scale(norm(h), shift, scale)` with a non-affine norm
    (sparse/transformer/modulated.mojo:210-211) as one fused kernel."""
    if shift.shape[0] != h.batch_size() or scale.shape[0] != h.batch_size():
        raise ValueError("SparseTensor.elemwise_batch: batch size mismatch")
    return h.replace(ops.ln_modulate(h.feats.contiguous(), eps, shift=shift, scale=scale, offsets=h.offsets))


def gated_residual(x: SparseTensor, h: SparseTensor, gate: torch.Tensor) -> SparseTensor:
    """`x + h.elemwise_batch(gate, OP_MUL)` (sparse/transformer/modulated.mojo:214-215)."""
    if gate.shape[0] != x.batch_size():
        raise ValueError("SparseTensor.elemwise_batch: batch size mismatch")
    return x.replace(ops.gate_residual(x.feats.contiguous(), h.feats.contiguous(), gate=gate, offsets=x.offsets))


class Modulation:
    """Modulation.chunks (sparse/transformer/modulated.mojo:24-57): the six
    [N, C] chunks shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp,
    gate_mlp of m, where m = mod + modulation (share_mod: the [6C] parameter
    row-broadcast), or m = lin(SiLU(mod)) with `lin` the adaLN linear
    [C -> 6C] as a callable (a GEMM, outside this library). The chunks are
    strided views of m; every t2h op reads them in place."""

    def __init__(self, modulation: Optional[torch.Tensor] = None, lin=None):
        if (modulation is None) == (lin is None):
            raise ValueError("Modulation: give the share_mod parameter or the linear, not both")
        self.share_mod = modulation is not None
        self.modulation = modulation.to(torch.float32).contiguous() if modulation is not None else None
        self.lin = lin

    def chunks(self, mod: torch.Tensor, channels: int):
        mod = mod.to(torch.float32).contiguous()
        if self.share_mod:
            m = ops.modulation_add(mod, self.modulation)
        else:
            m = self.lin(ops.activation(mod, ops.ACT_SILU)).to(torch.float32).contiguous()
        if m.dim() != 2 or m.shape[1] != 6 * channels:
            raise ValueError("Modulation: expected [N, 6C] modulation rows")
        return [m[:, i * channels:(i + 1) * channels] for i in range(6)]


class SparseRotaryPositionEmbedder:
    """RoPE from int voxel coords (sparse/attention/rope.mojo:20-134). embed()
    rotates q and k in one kernel; phases are computed in-kernel from coords
    (no phase tensor is built or cached)."""

    def __init__(self, head_dim: int, dim: int = 3, freq_lo: float = 1.0, freq_hi: float = 10000.0):
        if head_dim % 2 != 0:
            raise ValueError("SparseRotaryPositionEmbedder: head_dim must be even")
        self.head_dim, self.dim = int(head_dim), int(dim)
        self.freq_dim = head_dim // 2 // dim
        self.freqs = rope_freqs(head_dim, dim, freq_lo, freq_hi)

    def _compute_phases(self, x: SparseTensor) -> torch.Tensor:
        """-> [N, head_dim/2, 2] (sparse/attention/rope.mojo:48-66)."""
        return ops.rope_phases(x.coords.shape[0], self.head_dim, self.freqs, self.dim, coords=x.coords)

    def embed(self, q: SparseTensor, k: SparseTensor):
        if q.coords.shape[1] != self.dim + 1:
            raise ValueError("rope: coords must have dim+1 columns")
        if q.feats.shape[-1] != self.head_dim:
            raise ValueError("rope: feats last dim != head_dim")
        qf, kf = q.feats.contiguous(), k.feats.contiguous()
        qo, ko = ops.qk_rmsnorm_rope(q=qf.reshape(qf.shape[0], -1, self.head_dim),
                                     k=kf.reshape(kf.shape[0], -1, self.head_dim), freqs=self.freqs,
                                     pos_dim=self.dim, coords=q.coords, use_rope=True)
        return q.replace(qo.reshape(qf.shape)), k.replace(ko.reshape(kf.shape))
