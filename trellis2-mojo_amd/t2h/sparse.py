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
    """share_mod path of Modulation.chunks (sparse/transformer/modulated.mojo:24-57):
    m = mod + modulation (row-broadcast), sliced into the six [N, C] chunks
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp. The chunks
    are strided views of m; every t2h op reads them in place."""

    def __init__(self, modulation: torch.Tensor):
        self.share_mod = True
        self.modulation = modulation.to(torch.float32).contiguous()

    def chunks(self, mod: torch.Tensor, channels: int):
        m = ops.modulation_add(mod.to(torch.float32).contiguous(), self.modulation)
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
