"""Per-token glue of the DiT cross block on the MI355X path.

Two mirrors of the reference's block, with the attention / cross-attention /
MLP chains passed in as callables (those are GEMM and SDPA work outside this
library):

* `pack_block_consts` + `cross_block_enqueue`: the device-resident block
  (trellis2_mojo/gpu/block.mojo:217-397). One f32 const buffer `bk` [12C]
  carries the six glue pairs; the running x stays resident and is updated in
  place. The chains receive the normed rows and return their output WITHOUT
  the out-linear bias, which the reference folds into the residual join.
  With fused=True each join is merged with the next norm
  (t2h_block_join_ln): 4 instead of 6 row-passes of HBM traffic per pair.
* `ModulatedCrossBlock.forward`: the CPU block order for dense [N, L, C]
  (modules/transformer/modulated.mojo:177-200) and sparse feats with any
  batch count (sparse/transformer/modulated.mojo:187-226), gathering each
  row's adaLN chunk row through the batch map. Chains return complete
  outputs (bias included), as the reference's attention modules do.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence

import torch

from . import ops
from .sparse import Modulation, SparseTensor

Chain = Callable[[torch.Tensor], torch.Tensor]

# const-buffer pair offsets, in units of C (gpu/block.mojo:255-262)
BK_NORM1 = 0        # shift1, scale1           (norm1 modulate)
BK_SELF_JOIN = 2    # self_out bias, gate1     (self residual join)
BK_NORM2 = 4        # norm2 weight, bias       (affine norm2)
BK_CROSS_JOIN = 6   # cross_out bias, 0        (ungated cross join)
BK_NORM3 = 8        # shift3, scale3           (norm3 modulate)
BK_MLP_JOIN = 10    # mlp2 bias, gate3         (mlp residual join)
BK_FLOATS = 12      # buffer size in units of C


def _vec(t: Optional[torch.Tensor], c: int, device, what: str) -> torch.Tensor:
    if t is None:
        return torch.zeros(c, dtype=torch.float32, device=device)
    v = t.reshape(-1)
    if v.numel() != c:
        raise ValueError(f"pack_block_consts: {what} must have {c} values")
    return v.to(device=device, dtype=torch.float32)


def pack_block_consts(m: Sequence[torch.Tensor], norm2_weight: torch.Tensor, norm2_bias: torch.Tensor,
                      self_out_bias: Optional[torch.Tensor] = None, cross_out_bias: Optional[torch.Tensor] = None,
                      mlp2_bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The block's glue consts [12C] f32 on the device of m[0], in the
    reference's layout (gpu/block.mojo:255-289). m = the six adaLN chunks of a
    single batch row (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp,
    gate_mlp); a missing out bias is zeros, as in the reference."""
    if len(m) != 6:
        raise ValueError("gpu_cross_block_enqueue: expected 6 mod chunks")
    c = m[0].shape[-1]
    dev = m[0].device
    parts = [
        _vec(m[0], c, dev, "shift1"), _vec(m[1], c, dev, "scale1"),
        _vec(self_out_bias, c, dev, "self_out bias"), _vec(m[2], c, dev, "gate1"),
        _vec(norm2_weight, c, dev, "norm2 weight"), _vec(norm2_bias, c, dev, "norm2 bias"),
        _vec(cross_out_bias, c, dev, "cross_out bias"), torch.zeros(c, dtype=torch.float32, device=dev),
        _vec(m[3], c, dev, "shift3"), _vec(m[4], c, dev, "scale3"),
        _vec(mlp2_bias, c, dev, "mlp2 bias"), _vec(m[5], c, dev, "gate3"),
    ]
    return torch.cat(parts).contiguous()


def _spare(h: torch.Tensor, bufs) -> torch.Tensor:
    """A scratch buffer that does not alias the chain output h."""
    for b in bufs:
        if b.data_ptr() != h.data_ptr():
            return b
    raise AssertionError("unreachable: two distinct buffers")


def _check_chain_out(h: torch.Tensor, xs: torch.Tensor, what: str) -> torch.Tensor:
    if h.shape != xs.shape or h.dtype != xs.dtype:
        raise ValueError(f"cross_block_enqueue: {what} chain returned {tuple(h.shape)} {h.dtype}, "
                         f"expected {tuple(xs.shape)} {xs.dtype}")
    return h.contiguous()


def cross_block_enqueue(xs: torch.Tensor, bk: torch.Tensor, self_chain: Chain, cross_chain: Chain,
                        mlp_chain: Chain, fused: bool = True) -> torch.Tensor:
    """One block against the resident rows xs [rows, C] (updated in place and
    returned), in the order of gpu/block.mojo:304-397:

        hs = LN(xs)*(1+scale1)+shift1;        h = self_chain(hs)
        xs += (h + self_out_bias) * gate1;    hs = LN(xs)*w2 + b2
        h = cross_chain(hs);                  xs += h + cross_out_bias
        hs = LN(xs)*(1+scale3)+shift3;        h = mlp_chain(hs)
        xs += (h + mlp2_bias) * gate3
    """
    if xs.dim() != 2:
        raise ValueError("cross_block_enqueue: xs must be [rows, C]")
    c = xs.shape[1]
    if bk.numel() != BK_FLOATS * c:
        raise ValueError(f"cross_block_enqueue: consts must hold {BK_FLOATS * c} floats")
    bufs = (torch.empty_like(xs), torch.empty_like(xs))
    hs = ops.ln_mod_rows(xs, bufs[0], bk, BK_NORM1 * c, 1)
    h = _check_chain_out(self_chain(hs), xs, "self")
    if fused:
        hs = ops.block_join_ln(xs, h, _spare(h, bufs), bk, BK_SELF_JOIN * c, 1, BK_NORM2 * c, 2)
    else:
        ops.gate_add_bias_rows(xs, h, bk, BK_SELF_JOIN * c, 1)
        hs = ops.ln_mod_rows(xs, _spare(h, bufs), bk, BK_NORM2 * c, 2)
    h = _check_chain_out(cross_chain(hs), xs, "cross")
    if fused:
        hs = ops.block_join_ln(xs, h, _spare(h, bufs), bk, BK_CROSS_JOIN * c, 0, BK_NORM3 * c, 1)
    else:
        ops.gate_add_bias_rows(xs, h, bk, BK_CROSS_JOIN * c, 0)
        hs = ops.ln_mod_rows(xs, _spare(h, bufs), bk, BK_NORM3 * c, 1)
    h = _check_chain_out(mlp_chain(hs), xs, "mlp")
    ops.gate_add_bias_rows(xs, h, bk, BK_MLP_JOIN * c, 1)
    return xs


class ModulatedCrossBlock:
    """Glue of ModulatedTransformerCrossBlock / ModulatedSparseTransformerCrossBlock:
    norm1 and norm3 non-affine, norm2 affine, all with eps (1e-6 in the DiT
    blocks, loaders.mojo:53-60). `modulation` is the share_mod parameter
    [6C] (Modulation), or None when `mod` already holds the chunks [B, 6C]."""

    def __init__(self, channels: int, norm2_weight: torch.Tensor, norm2_bias: torch.Tensor,
                 modulation: Optional[torch.Tensor] = None, eps: float = 1e-6):
        self.channels = int(channels)
        self.eps = float(eps)
        self.norm2_weight = norm2_weight.to(torch.float32).contiguous()
        self.norm2_bias = norm2_bias.to(torch.float32).contiguous()
        self.modulation = Modulation(modulation) if modulation is not None else None

    def _chunks(self, mod: torch.Tensor):
        c = self.channels
        if self.modulation is not None:
            return self.modulation.chunks(mod, c)
        m = mod.to(torch.float32).contiguous()
        if m.dim() != 2 or m.shape[1] != 6 * c:
            raise ValueError("ModulatedCrossBlock: mod must be [B, 6C]")
        return [m[:, i * c:(i + 1) * c] for i in range(6)]

    def forward(self, x, mod: torch.Tensor, self_attn: Chain, cross_attn: Chain, mlp: Chain):
        """x: dense [N, L, C] or SparseTensor with feats [T, C]. Returns a new
        tensor of the same kind (value semantics)."""
        m = self._chunks(mod)
        c = self.channels
        if isinstance(x, SparseTensor):
            feats = x.feats.contiguous()
            if feats.dim() != 2 or feats.shape[1] != c:
                raise ValueError("LayerNorm32: last dim mismatch")
            if m[0].shape[0] != x.batch_size():
                raise ValueError("SparseTensor.elemwise_batch: batch size mismatch")
            batch = dict(offsets=x.offsets)
        else:
            if x.dim() != 3 or x.shape[2] != c:
                raise ValueError("LayerNorm32: last dim mismatch")
            if m[0].shape[0] != x.shape[0]:
                raise ValueError("modulate: shift/scale shape mismatch")
            feats = x.contiguous().reshape(-1, c)
            batch = dict(rows_per_batch=x.shape[1])
        h = ops.ln_modulate(feats, self.eps, shift=m[0], scale=m[1], **batch)
        h = self_attn(h)
        # y = x + h * gate_msa[b];  h2 = norm2(y)
        y, h2 = ops.gate_residual_ln_modulate(feats, h.contiguous(), gate=m[2], eps=self.eps,
                                              weight=self.norm2_weight, norm_bias=self.norm2_bias, **batch)
        h2 = cross_attn(h2)
        # y = y + h2;  h3 = norm3(y) * (1 + scale_mlp[b]) + shift_mlp[b]
        y, h3 = ops.gate_residual_ln_modulate(y, h2.contiguous(), eps=self.eps, shift=m[3], scale=m[4],
                                              x_out=y, **batch)
        h3 = mlp(h3)
        out = ops.gate_residual(y, h3.contiguous(), gate=m[5], out=y, **batch)
        if isinstance(x, SparseTensor):
            return x.replace(out)
        return out.reshape(x.shape)

    __call__ = forward
