"""Mirror of the reference's per-token op interface on the MI355X path.

Same names, argument meaning and errors as the Mojo originals (value
semantics: inputs borrowed, a fresh output tensor returned), on device
tensors, every op a libt2h kernel. Sparse tensors live in t2h.sparse.

Reference: trellis2_mojo/modules/nn.mojo (LayerNorm32 297-375, activation
588-655, modulate 660-689), modules/rope.mojo, sparse/attention/modules.mojo
(MultiHeadRMSNorm 37-102), modules/transformer/modulated.mojo (_gate 22-33),
models/sparse_structure_flow.mojo (TimestepEmbedder 40-80).
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops

ACT_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH = ops.ACT_RELU, ops.ACT_SILU, ops.ACT_GELU, ops.ACT_GELU_TANH


def _is_sparse(x) -> bool:
    return hasattr(x, "feats") and hasattr(x, "replace")


class LayerNorm32:
    """nn.LayerNorm over the last dim (modules/nn.mojo:297-369): ctor defaults
    eps 1e-5, affine True; weight ones / bias zeros."""

    def __init__(self, num_channels: int, eps: float = 1e-5, affine: bool = True, device="cuda"):
        self.num_channels = int(num_channels)
        self.eps = float(eps)
        self.affine = bool(affine)
        self.weight = torch.ones(num_channels, dtype=torch.float32, device=device)
        self.bias = torch.zeros(num_channels, dtype=torch.float32, device=device)

    def forward(self, x):
        if _is_sparse(x):
            return x.replace(self.forward(x.feats))
        if x.shape[-1] != self.num_channels:
            raise ValueError("LayerNorm32: last dim mismatch")
        if self.affine:
            return ops.ln_modulate(x.contiguous(), self.eps, weight=self.weight, bias=self.bias)
        return ops.ln_modulate(x.contiguous(), self.eps)

    __call__ = forward


def modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1); x [N, L, C], shift/scale
    [N, C] (modules/nn.mojo:660-689)."""
    n, l, c = x.shape
    if shift.numel() != n * c or scale.numel() != n * c:
        raise ValueError("modulate: shift/scale shape mismatch")
    return ops.modulate(x.contiguous(), shift.reshape(n, c), scale.reshape(n, c), rows_per_batch=l)


def layernorm_modulate(norm: LayerNorm32, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """`modulate(norm.forward(x), shift, scale)` (modules/transformer/modulated.mojo:185)
    as one fused kernel (ln_mod_rows mode 1, gpu/block.mojo:47-83)."""
    if norm.affine:
        raise ValueError("layernorm_modulate: the fused path needs a non-affine norm")
    n, l, c = x.shape
    if c != norm.num_channels:
        raise ValueError("LayerNorm32: last dim mismatch")
    if shift.numel() != n * c or scale.numel() != n * c:
        raise ValueError("modulate: shift/scale shape mismatch")
    return ops.ln_modulate(x.contiguous(), norm.eps, shift=shift.reshape(n, c), scale=scale.reshape(n, c),
                           rows_per_batch=l)


def activation(x, kind: int):
    """Elementwise activation (modules/nn.mojo:588-647)."""
    if _is_sparse(x):
        return x.replace(activation(x.feats, kind))
    if kind not in (ACT_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH):
        raise ValueError("unknown activation")
    return ops.activation(x.contiguous(), kind)


def linear_bias_activation(h: torch.Tensor, bias: torch.Tensor, kind: int = ACT_GELU_TANH) -> torch.Tensor:
    """`activation(linear(x) + bias)` epilogue: the FFN's lin1 bias folded into
    the activation (gpu/linear.mojo:662-684 gelu_tanh_bias)."""
    return ops.activation(h.contiguous(), kind, bias=bias)


class MultiHeadRMSNorm:
    """F.normalize(x, dim=-1) * gamma * sqrt(dim) over x [..., H, D]
    (sparse/attention/modules.mojo:37-102)."""

    def __init__(self, dim: int, heads: int, device="cuda"):
        self.gamma = torch.ones((heads, dim), dtype=torch.float32, device=device)
        self.scale = float(np.float32(float(dim) ** 0.5))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h, d = x.shape[-2], x.shape[-1]
        if self.gamma.shape != (h, d):
            raise ValueError("MultiHeadRMSNorm: gamma shape mismatch")
        x3 = x.contiguous().reshape(-1, h, d)
        q, _ = ops.qk_rmsnorm_rope(q=x3, gamma_q=self.gamma, use_rope=False)
        return q.reshape(x.shape)

    __call__ = forward


def rope_freqs(head_dim: int, dim: int = 3, freq_lo: float = 1.0, freq_hi: float = 10000.0) -> np.ndarray:
    """freqs = freq_lo / freq_hi ** (arange(freq_dim) / freq_dim) in f32
    (modules/rope.mojo:33-37), computed by libt2h's host code with libm powf."""
    out = np.zeros(max(head_dim // 2, 1), np.float32)
    from ._lib import load, check
    fd = load().t2h_rope_freqs(int(head_dim), int(dim), float(freq_lo), float(freq_hi), out.ctypes.data, out.size)
    if fd < 0:
        check(fd)
    return out[:fd].copy()


class RotaryPositionEmbedder:
    """Dense-path RoPE (modules/rope.mojo:17-61): forward(positions [L, dim]) ->
    phases [L, head_dim/2, 2] (cos, sin), axis-major slots, unit pad slots."""

    def __init__(self, head_dim: int, dim: int = 3, freq_lo: float = 1.0, freq_hi: float = 10000.0):
        if head_dim % 2 != 0:
            raise ValueError("RotaryPositionEmbedder: head_dim must be even")
        self.head_dim, self.dim = int(head_dim), int(dim)
        self.freq_lo, self.freq_hi = float(freq_lo), float(freq_hi)
        self.freq_dim = head_dim // 2 // dim
        self.freqs = rope_freqs(head_dim, dim, freq_lo, freq_hi)

    def forward(self, positions: torch.Tensor) -> torch.Tensor:
        if positions.shape[-1] != self.dim:
            raise ValueError("RotaryPositionEmbedder: last dim of positions must be dim")
        pos = positions.to(torch.float32).contiguous()
        return ops.rope_phases(pos.shape[0], self.head_dim, self.freqs, self.dim, positions=pos)

    def grid_phases(self, resolution: int, device="cuda") -> torch.Tensor:
        """Phases of the 'ij' meshgrid over resolution^3 (sparse_structure_flow.mojo:132-151)."""
        return ops.rope_phases(resolution ** 3, self.head_dim, self.freqs, 3, grid_res=resolution, device=device)

    __call__ = forward


def apply_rotary_embedding(x: torch.Tensor, phases: torch.Tensor) -> torch.Tensor:
    """x [N, L, H, D] (adjacent re/im pairs), phases [L, D/2, 2] broadcast over
    N and H (modules/rope.mojo:64-88)."""
    if x.dim() != 4:
        raise ValueError("apply_rotary_embedding: expected [N, L, H, D]")
    n, l, h, d = x.shape
    if phases.shape[0] != l or phases.shape[1] != d // 2:
        raise ValueError("apply_rotary_embedding: phases shape mismatch")
    x3 = x.contiguous().reshape(n * l, h, d)
    q, _ = ops.qk_rmsnorm_rope(q=x3, phases=phases.contiguous(), use_rope=True)
    return q.reshape(x.shape)


def _gate(x: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """x [N, L, C] * g [N, C] broadcast over L (modules/transformer/modulated.mojo:22-33)."""
    n, l, c = x.shape
    return ops.gate_residual(None, x.contiguous(), gate=g.reshape(n, c), rows_per_batch=l)


def gate_residual(y: torch.Tensor, h: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """`y._binop_flat(_gate(h, g), OP_ADD)` (modulated.mojo:60-69, 192-200) in one pass."""
    n, l, c = h.shape
    return ops.gate_residual(y.contiguous(), h.contiguous(), gate=g.reshape(n, c), rows_per_batch=l)


class TimestepEmbedder:
    """Sinusoidal timestep embedding (models/sparse_structure_flow.mojo:40-80).
    Only timestep_embedding is on this path (the MLP after it is a GEMM)."""

    def __init__(self, frequency_embedding_size: int = 256, max_period: float = 10000.0):
        self.frequency_embedding_size = int(frequency_embedding_size)
        self.max_period = float(max_period)

    def timestep_embedding(self, t: torch.Tensor) -> torch.Tensor:
        return ops.timestep_embedding(t.reshape(-1).to(torch.float32).contiguous(), self.frequency_embedding_size,
                                      self.max_period)
