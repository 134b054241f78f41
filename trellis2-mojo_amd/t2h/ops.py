"""Tensor-level wrappers of the libt2h C ABI (device tensors in, device
tensors out, enqueued on torch's current stream).

Every function validates shapes/dtypes/devices on the host, then calls the
HIP entry point. There is no CPU or PyTorch fallback: a missing library or a
CPU tensor raises.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import BF16, F16, F32, LN_AFFINE, LN_MODULATE, LN_PLAIN, call

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

ACT_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH = 0, 1, 2, 3
ACT_NONE = -1
OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_RSUB, OP_RDIV = 0, 1, 2, 3, 4, 5


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what}: expected a device (cuda) tensor")


def _dtype(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {t.dtype}") from None


def _rows_view(x: torch.Tensor, what: str):
    """x [..., C] contiguous -> (rows, C)."""
    _dev(x, what)
    if not x.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    c = x.shape[-1]
    rows = x.numel() // c if c else 0
    return rows, c


def _param_rows(p: Optional[torch.Tensor], cols: int, what: str):
    """f32 parameter rows [B, C] (row stride >= C, unit column stride) or [C].
    Returns (ptr, row_stride, nrows)."""
    if p is None:
        return None, 0, 0
    _dev(p, what)
    if p.dtype != torch.float32:
        raise ValueError(f"{what}: parameters must be float32")
    if p.dim() == 1:
        if p.numel() != cols or p.stride(0) != 1:
            raise ValueError(f"{what}: expected [{cols}] parameters")
        return p.data_ptr(), cols, 1
    p2 = p.reshape(-1, p.shape[-1]) if p.dim() > 2 else p
    if p2.shape[-1] != cols or p2.stride(-1) != 1 or p2.stride(0) < cols:
        raise ValueError(f"{what}: expected [B, {cols}] parameters with unit column stride")
    return p2.data_ptr(), p2.stride(0), p2.shape[0]


def _batch(offsets: Optional[torch.Tensor], rows_per_batch: int, nparam_rows: int, rows: int, what: str):
    """Batch-map arguments + a host-side check that every row maps to an
    existing parameter row."""
    if offsets is not None:
        _dev(offsets, what)
        if offsets.dtype != torch.int64 or offsets.dim() != 1 or offsets.numel() < 2:
            raise ValueError(f"{what}: offsets must be int64 [B+1]")
        nb = offsets.numel() - 1
        if nparam_rows and nparam_rows < nb:
            raise ValueError(f"{what}: batch size mismatch")
        return offsets.data_ptr(), nb, 0
    if rows_per_batch > 0:
        need = (rows + rows_per_batch - 1) // rows_per_batch
        if nparam_rows and nparam_rows < need:
            raise ValueError(f"{what}: batch size mismatch")
        return None, max(need, 1), rows_per_batch
    return None, 1, 0


# ---- LayerNorm (+ modulate / affine) ------------------------------------------
def ln_modulate(x: torch.Tensor, eps: float = 1e-6, shift=None, scale=None, weight=None, bias=None,
                offsets=None, rows_per_batch: int = 0, out=None) -> torch.Tensor:
    """LN(x) [* (1 + scale[b]) + shift[b]] or [* weight + bias]."""
    rows, c = _rows_view(x, "ln_modulate")
    dt = _dtype(x, "ln_modulate")
    if (shift is None) != (scale is None) or (weight is None) != (bias is None):
        raise ValueError("ln_modulate: shift/scale and weight/bias come in pairs")
    if shift is not None and weight is not None:
        raise ValueError("ln_modulate: modulate and affine are exclusive")
    mode = LN_MODULATE if shift is not None else (LN_AFFINE if weight is not None else LN_PLAIN)
    p0, p1 = (shift, scale) if mode == LN_MODULATE else (weight, bias)
    p0p, s0, n0 = _param_rows(p0, c, "ln_modulate")
    p1p, s1, n1 = _param_rows(p1, c, "ln_modulate")
    if s0 != s1:
        raise ValueError("ln_modulate: p0/p1 row strides differ")
    off, nb, rpb = _batch(offsets, rows_per_batch, min(n0, n1) if mode == LN_MODULATE else 0, rows, "ln_modulate")
    out = torch.empty_like(x) if out is None else out
    if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("ln_modulate: bad out tensor")
    call("t2h_ln_modulate", x.data_ptr(), out.data_ptr(), rows, c, dt, float(eps), mode, p0p, p1p, s0, off, nb,
         rpb, _stream())
    return out


def gate_residual_ln_modulate(x, h, gate=None, bias=None, eps: float = 1e-6, shift=None, scale=None,
                              weight=None, norm_bias=None, offsets=None, rows_per_batch: int = 0,
                              x_out=None, y_out=None):
    """x_out = x + (h + bias) * gate[b];  y_out = LN(x_out) epilogue."""
    rows, c = _rows_view(x, "gate_residual_ln_modulate")
    dt = _dtype(x, "gate_residual_ln_modulate")
    if h.shape != x.shape or h.dtype != x.dtype or not h.is_contiguous():
        raise ValueError("gate_residual_ln_modulate: h must match x")
    mode = LN_MODULATE if shift is not None else (LN_AFFINE if weight is not None else LN_PLAIN)
    p0, p1 = (shift, scale) if mode == LN_MODULATE else (weight, norm_bias)
    p0p, s0, n0 = _param_rows(p0, c, "gate_residual_ln_modulate")
    p1p, _, n1 = _param_rows(p1, c, "gate_residual_ln_modulate")
    gp, gs, ng = _param_rows(gate, c, "gate_residual_ln_modulate")
    bp, _, _ = _param_rows(bias, c, "gate_residual_ln_modulate")
    need = max(min(n0, n1) if mode == LN_MODULATE else 0, ng)
    off, nb, rpb = _batch(offsets, rows_per_batch, need, rows, "gate_residual_ln_modulate")
    x_out = torch.empty_like(x) if x_out is None else x_out
    y_out = torch.empty_like(x) if y_out is None else y_out
    call("t2h_gate_residual_ln_modulate", x.data_ptr(), h.data_ptr(), x_out.data_ptr(), y_out.data_ptr(), bp, gp,
         gs, float(eps), mode, p0p, p1p, s0, rows, c, dt, off, nb, rpb, _stream())
    return x_out, y_out


def modulate(x, shift, scale, offsets=None, rows_per_batch: int = 0, out=None) -> torch.Tensor:
    """fl(fl(x * fl(1 + scale[b])) + shift[b]) — bit-exact."""
    rows, c = _rows_view(x, "modulate")
    dt = _dtype(x, "modulate")
    sp, s0, n0 = _param_rows(shift, c, "modulate")
    cp, s1, n1 = _param_rows(scale, c, "modulate")
    if s0 != s1:
        raise ValueError("modulate: shift/scale row strides differ")
    off, nb, rpb = _batch(offsets, rows_per_batch, min(n0, n1), rows, "modulate")
    out = torch.empty_like(x) if out is None else out
    call("t2h_modulate", x.data_ptr(), out.data_ptr(), rows, c, dt, sp, cp, s0, off, nb, rpb, _stream())
    return out


def binop_rows(x, other, op: int, offsets=None, rows_per_batch: int = 0, out=None) -> torch.Tensor:
    """x[r, :] OP other[b(r), :] (other [B, C] or [B, 1]) — bit-exact."""
    rows, c = _rows_view(x, "binop_rows")
    dt = _dtype(x, "binop_rows")
    _dev(other, "binop_rows")
    if other.dtype != torch.float32 or not other.is_contiguous():
        raise ValueError("binop_rows: other must be contiguous float32")
    oc = other.shape[-1] if other.dim() > 1 else 1
    if oc != c and oc != 1:
        raise ValueError("Tensor._binop_rows: incompatible row size")
    off, nb, rpb = _batch(offsets, rows_per_batch, other.numel() // oc, rows, "binop_rows")
    out = torch.empty_like(x) if out is None else out
    call("t2h_binop_rows", x.data_ptr(), other.data_ptr(), out.data_ptr(), rows, c, oc, dt, int(op), off, nb, rpb,
         _stream())
    return out


# ---- QK RMSNorm + RoPE -----------------------------------------------------------
def _heads_view(t: torch.Tensor, what: str):
    """[rows, H, D] with unit stride on D and contiguous heads -> (rows, H, D, row_stride)."""
    _dev(t, what)
    if t.dim() < 3:
        raise ValueError(f"{what}: expected [..., H, D]")
    h, d = t.shape[-2], t.shape[-1]
    if t.stride(-1) != 1 or t.stride(-2) != d:
        raise ValueError(f"{what}: heads must be contiguous [H, D]")
    lead = t.shape[:-2]
    rows = int(np.prod(lead)) if len(lead) else 1
    if t.dim() == 3:
        stride = t.stride(0)
    else:  # leading dims must collapse to one row stride
        stride = h * d
        if not t.is_contiguous():
            raise ValueError(f"{what}: leading dims must be contiguous")
    return rows, h, d, stride


def _host_freqs(freqs) -> tuple:
    f = np.ascontiguousarray(np.asarray(freqs, dtype=np.float32))
    return f, (f.ctypes.data if f.size else None), int(f.size)


def qk_rmsnorm_rope(q=None, k=None, gamma_q=None, gamma_k=None, bias_q=None, bias_k=None, freqs=None,
                    pos_dim: int = 3, phases=None, coords=None, grid_res: int = 0, use_rope: bool = True,
                    q_out=None, k_out=None, in_place: bool = False):
    """bias -> RMS (if gammas) -> RoPE on q/k [rows, H, D] (views allowed).
    Returns (q_out, k_out)."""
    ref = q if q is not None else k
    if ref is None:
        raise ValueError("qk_rmsnorm_rope: q and k are both None")
    rows, h, d, in_stride = _heads_view(ref, "qk_rmsnorm_rope")
    dt = _dtype(ref, "qk_rmsnorm_rope")
    for t in (q, k):
        if t is not None:
            r2, h2, d2, s2 = _heads_view(t, "qk_rmsnorm_rope")
            if (r2, h2, d2, s2) != (rows, h, d, in_stride) or t.dtype != ref.dtype:
                raise ValueError("qk_rmsnorm_rope: q/k layouts differ")
    if in_place:
        q_out, k_out = q, k
    else:
        if q is not None and q_out is None:
            q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        if k is not None and k_out is None:
            k_out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    out_ref = q_out if q_out is not None else k_out
    _, _, _, out_stride = _heads_view(out_ref, "qk_rmsnorm_rope")
    for g in (gamma_q, gamma_k, bias_q, bias_k):
        if g is not None:
            _dev(g, "qk_rmsnorm_rope")
            if g.dtype != torch.float32 or g.numel() != h * d or not g.is_contiguous():
                raise ValueError("qk_rmsnorm_rope: gamma/bias must be contiguous float32 [H, D]")
    hold, fp, fd = _host_freqs(freqs if freqs is not None else [])
    ph_rows = 0
    if phases is not None:
        _dev(phases, "qk_rmsnorm_rope")
        if phases.dtype != torch.float32 or not phases.is_contiguous() or phases.shape[-2:] != (d // 2, 2):
            raise ValueError("apply_rotary_embedding: phases shape mismatch")
        ph_rows = phases.numel() // d
    cc = 0
    if coords is not None:
        _dev(coords, "qk_rmsnorm_rope")
        if coords.dtype != torch.int32 or not coords.is_contiguous() or coords.shape[0] != rows:
            raise ValueError("qk_rmsnorm_rope: coords must be contiguous int32 [rows, 1+pos_dim]")
        cc = coords.shape[1]
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_qk_rmsnorm_rope", p(q), p(k), p(q_out), p(k_out), rows, in_stride, out_stride, h, d, dt,
         p(bias_q), p(bias_k), p(gamma_q), p(gamma_k), int(bool(use_rope)), fp, fd, int(pos_dim), p(phases),
         ph_rows, p(coords), cc, int(grid_res), _stream())
    del hold
    return q_out, k_out


def qkv_bias_rmsnorm_rope(qkv, heads: int, head_dim: int, bias=None, gamma_q=None, gamma_k=None, freqs=None,
                          pos_dim: int = 3, phases=None, coords=None, grid_res: int = 0, use_rope: bool = True):
    """In place on a packed qkv [rows, 3*H*D] (bias_rms_rope_qkv)."""
    rows, c3 = _rows_view(qkv, "qkv_bias_rmsnorm_rope")
    if c3 != 3 * heads * head_dim:
        raise ValueError("qkv_bias_rmsnorm_rope: last dim must be 3*H*D")
    dt = _dtype(qkv, "qkv_bias_rmsnorm_rope")
    hold, fp, fd = _host_freqs(freqs if freqs is not None else [])
    ph_rows = phases.numel() // head_dim if phases is not None else 0
    cc = coords.shape[1] if coords is not None else 0
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_qkv_bias_rmsnorm_rope", qkv.data_ptr(), rows, heads, head_dim, dt, p(bias), p(gamma_q), p(gamma_k),
         int(bool(use_rope)), fp, fd, int(pos_dim), p(phases), ph_rows, p(coords), cc, int(grid_res), _stream())
    del hold
    return qkv


def attn_pack(q=None, k=None, v=None, mp: int = 0, lp: int = 0, bias_q=None, bias_k=None, bias_v=None, gamma_q=None,
              gamma_k=None, freqs=None, pos_dim: int = 3, phases=None, coords=None, grid_res: int = 0,
              use_rope: bool = True, k_transposed: bool = True):
    """Attention epilogue + head-major packing: q/k/v [rows, H, D] (views of
    a packed qkv allowed) -> qh [H, mp, D] (scaled by 1/sqrt(D)), k [H, D, lp]
    (k_transposed) or [H, lp, D], vh [H, lp, D]; pads zero. mp/lp 0 = rows.
    Returns (qh, k_out, vh), None for an absent input."""
    ref = next((t for t in (q, k, v) if t is not None), None)
    if ref is None:
        raise ValueError("attn_pack: q, k and v are all None")
    rows, h, d, in_stride = _heads_view(ref, "attn_pack")
    dt = _dtype(ref, "attn_pack")
    for t in (q, k, v):
        if t is not None:
            if _heads_view(t, "attn_pack") != (rows, h, d, in_stride) or t.dtype != ref.dtype:
                raise ValueError("attn_pack: q/k/v layouts differ")
    for g in (gamma_q, gamma_k, bias_q, bias_k, bias_v):
        if g is not None:
            _dev(g, "attn_pack")
            if g.dtype != torch.float32 or g.numel() != h * d or not g.is_contiguous():
                raise ValueError("attn_pack: gamma/bias must be contiguous float32 [H, D]")
    mp = mp or rows
    lp = lp or rows
    mk = lambda shape: torch.empty(shape, dtype=ref.dtype, device=ref.device)
    qh = mk((h, mp, d)) if q is not None else None
    ko = (mk((h, d, lp)) if k_transposed else mk((h, lp, d))) if k is not None else None
    vh = mk((h, lp, d)) if v is not None else None
    hold, fp, fd = _host_freqs(freqs if freqs is not None else [])
    ph_rows = 0
    if phases is not None:
        _dev(phases, "attn_pack")
        if phases.dtype != torch.float32 or not phases.is_contiguous() or phases.shape[-2:] != (d // 2, 2):
            raise ValueError("apply_rotary_embedding: phases shape mismatch")
        ph_rows = phases.numel() // d
    cc = 0
    if coords is not None:
        _dev(coords, "attn_pack")
        if coords.dtype != torch.int32 or not coords.is_contiguous() or coords.shape[0] != rows:
            raise ValueError("attn_pack: coords must be contiguous int32 [rows, 1+pos_dim]")
        cc = coords.shape[1]
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_attn_pack", p(q), p(k), p(v), in_stride, rows, h, d, dt, p(bias_q), p(bias_k), p(bias_v), p(gamma_q),
         p(gamma_k), int(bool(use_rope)), fp, fd, int(pos_dim), p(phases), ph_rows, p(coords), cc, int(grid_res),
         p(qh), mp, p(ko), p(vh), lp, int(bool(k_transposed)), _stream())
    del hold
    return qh, ko, vh


def qkv_linear_pack(x, weight, heads: int, bias=None, gamma_q=None, gamma_k=None, mp: int = 0, lp: int = 0,
                    freqs=None, pos_dim: int = 3, phases=None, coords=None, grid_res: int = 0, use_rope: bool = True,
                    k_transposed: bool = True):
    """The qkv linear fused with the attention epilogue and the head-major
    pack: x [rows, K] (float16/bfloat16, rows may be strided), weight
    [3*H*D, K] of x's dtype, bias [3*H*D] float32 (or None), gammas [H, D]
    float32 -> (qh [H, mp, D] scaled by 1/sqrt(D), k [H, D, lp] (k_transposed)
    or [H, lp, D], vh [H, lp, D]); pads zero; mp/lp 0 = rows. D = 128 (H
    even) or 64 (H a multiple of 4)."""
    _dev(x, "qkv_linear_pack")
    _dev(weight, "qkv_linear_pack")
    dt = _dtype(x, "qkv_linear_pack")
    if weight.dtype != x.dtype or weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("qkv_linear_pack: weight must be a contiguous [3*H*D, K] tensor of x's dtype")
    n, k = weight.shape
    if n % (3 * heads) != 0:
        raise ValueError("qkv_linear_pack: weight rows must be 3 * heads * head_dim")
    d = n // (3 * heads)
    if x.dim() != 2 or x.shape[1] != k or x.stride(1) != 1:
        raise ValueError("qkv_linear_pack: x must be [rows, K] with unit column stride")
    rows, ldx = x.shape[0], (x.stride(0) if x.shape[0] > 1 else k)
    bq = bk = bv = None
    if bias is not None:
        _dev(bias, "qkv_linear_pack")
        if bias.dtype != torch.float32 or bias.numel() != n or not bias.is_contiguous():
            raise ValueError("qkv_linear_pack: bias must be a contiguous float32 [3*H*D] tensor")
        bq, bk, bv = bias.reshape(3, heads * d).unbind(0)
    for g in (gamma_q, gamma_k):
        if g is not None:
            _dev(g, "qkv_linear_pack")
            if g.dtype != torch.float32 or g.numel() != heads * d or not g.is_contiguous():
                raise ValueError("qkv_linear_pack: gammas must be contiguous float32 [H, D]")
    mp = mp or rows
    lp = lp or rows
    mk = lambda shape: torch.empty(shape, dtype=x.dtype, device=x.device)
    qh = mk((heads, mp, d))
    ko = mk((heads, d, lp)) if k_transposed else mk((heads, lp, d))
    vh = mk((heads, lp, d))
    hold, fp, fd = _host_freqs(freqs if freqs is not None else [])
    ph_rows = 0
    if phases is not None:
        _dev(phases, "qkv_linear_pack")
        if phases.dtype != torch.float32 or not phases.is_contiguous() or phases.shape[-2:] != (d // 2, 2):
            raise ValueError("apply_rotary_embedding: phases shape mismatch")
        ph_rows = phases.numel() // d
    cc = 0
    if coords is not None:
        _dev(coords, "qkv_linear_pack")
        if coords.dtype != torch.int32 or not coords.is_contiguous() or coords.shape[0] != rows:
            raise ValueError("qkv_linear_pack: coords must be contiguous int32 [rows, 1+pos_dim]")
        cc = coords.shape[1]
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_qkv_linear_pack", x.data_ptr(), ldx, weight.data_ptr(), rows, k, heads, d, dt, p(bq), p(bk), p(bv),
         p(gamma_q), p(gamma_k), int(bool(use_rope)), fp, fd, int(pos_dim), p(phases), ph_rows, p(coords), cc,
         int(grid_res), qh.data_ptr(), mp, ko.data_ptr(), vh.data_ptr(), lp, int(bool(k_transposed)), _stream())
    del hold
    return qh, ko, vh


def rope_phases(rows: int, head_dim: int, freqs, pos_dim: int = 3, positions=None, coords=None, grid_res: int = 0,
                device=None) -> torch.Tensor:
    """Phase table [rows, head_dim/2, 2] (cos, sin) f32."""
    dev = device
    for t in (positions, coords):
        if t is not None:
            _dev(t, "rope_phases")
            dev = t.device
    if dev is None:
        dev = torch.device("cuda")
    out = torch.empty((rows, head_dim // 2, 2), dtype=torch.float32, device=dev)
    hold, fp, fd = _host_freqs(freqs)
    if positions is not None and (positions.dtype != torch.float32 or not positions.is_contiguous()):
        raise ValueError("rope_phases: positions must be contiguous float32")
    cc = coords.shape[1] if coords is not None else 0
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_rope_phases", out.data_ptr(), rows, head_dim, fp, fd, int(pos_dim), p(positions), p(coords), cc,
         int(grid_res), _stream())
    del hold
    return out


# ---- activation / residual -------------------------------------------------------
def activation(x, kind: int = ACT_GELU_TANH, bias=None, out=None) -> torch.Tensor:
    """act(x + bias[col]) elementwise over [..., C]."""
    rows, c = _rows_view(x, "activation")
    dt = _dtype(x, "activation")
    bp, _, _ = _param_rows(bias, c, "activation")
    out = torch.empty_like(x) if out is None else out
    call("t2h_activation", x.data_ptr(), out.data_ptr(), bp, rows, c, dt, int(kind), _stream())
    return out


def linear(x, weight, bias=None, act: int = ACT_NONE, out_dtype=None, out=None) -> torch.Tensor:
    """act(x @ weight^T + bias) on the matrix cores: x [..., K] (rows may be
    strided, unit column stride), weight [N, K] contiguous, both float16 or
    both bfloat16; bias [N] float32 or None; f32 sums; out [..., N] in
    out_dtype (float32 or x's dtype, default x's)."""
    _dev(x, "linear")
    _dev(weight, "linear")
    dt = _dtype(x, "linear")
    if weight.dtype != x.dtype or weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("linear: weight must be a contiguous [N, K] tensor of x's dtype")
    n, k = weight.shape
    if x.shape[-1] != k or x.stride(-1) != 1:
        raise ValueError("linear: x's last dim must be K with unit stride")
    x2 = x.reshape(-1, k) if x.dim() != 2 else x
    rows, ldx = x2.shape[0], (x2.stride(0) if x2.shape[0] > 1 else k)
    if bias is not None:
        _dev(bias, "linear")
        if bias.dtype != torch.float32 or bias.numel() != n or not bias.is_contiguous():
            raise ValueError("linear: bias must be a contiguous float32 [N] tensor")
    od = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((*x.shape[:-1], n), dtype=od, device=x.device)
    elif out.dtype != od or out.shape != (*x.shape[:-1], n):
        raise ValueError("linear: out must be a [..., N] tensor of out_dtype")
    if out.is_contiguous():
        ldo = n
    elif out.dim() == 2 and out.stride(1) == 1 and out.stride(0) >= n:
        ldo = out.stride(0)   # rows of a wider buffer
    else:
        raise ValueError("linear: out must be contiguous, or [rows, N] with unit column stride")
    call("t2h_linear", x2.data_ptr(), ldx, weight.data_ptr(), bias.data_ptr() if bias is not None else None,
         out.data_ptr(), ldo, rows, k, n, dt, _dtype(out, "linear"), int(act), _stream())
    return out


def linear_gate_residual(x, weight, res, bias=None, gate=None, offsets=None, rows_per_batch: int = 0,
                         out=None) -> torch.Tensor:
    """res + fl(fl(x @ weight^T + bias) * gate[b]) on the matrix cores (gate
    None: res + fl(acc + bias)): x [rows, K] float16/bfloat16, weight [N, K]
    of x's dtype, res [rows, N] of x's dtype or float32 (the output type);
    gate rows [B, N] or [N] float32 with offsets / rows_per_batch as
    gate_residual. out=res updates the residual stream in place."""
    _dev(x, "linear_gate_residual")
    _dev(weight, "linear_gate_residual")
    _dev(res, "linear_gate_residual")
    dt = _dtype(x, "linear_gate_residual")
    if weight.dtype != x.dtype or weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("linear_gate_residual: weight must be a contiguous [N, K] tensor of x's dtype")
    n, k = weight.shape
    if x.dim() != 2 or x.shape[1] != k or x.stride(1) != 1:
        raise ValueError("linear_gate_residual: x must be [rows, K] with unit column stride")
    rows, ldx = x.shape[0], (x.stride(0) if x.shape[0] > 1 else k)
    if res.dtype not in (x.dtype, torch.float32) or res.shape != (rows, n) or not res.is_contiguous():
        raise ValueError("linear_gate_residual: res must be a contiguous [rows, N] tensor of x's dtype or float32")
    if bias is not None:
        _dev(bias, "linear_gate_residual")
        if bias.dtype != torch.float32 or bias.numel() != n or not bias.is_contiguous():
            raise ValueError("linear_gate_residual: bias must be a contiguous float32 [N] tensor")
    gp, gs, ng = _param_rows(gate, n, "linear_gate_residual")
    off, nb, rpb = _batch(offsets, rows_per_batch, ng, rows, "linear_gate_residual")
    if out is None:
        out = torch.empty_like(res)
    elif out.dtype != res.dtype or out.shape != res.shape or not out.is_contiguous():
        raise ValueError("linear_gate_residual: out must match res")
    call("t2h_linear_gate_residual", x.data_ptr(), ldx, weight.data_ptr(), bias.data_ptr() if bias is not None else None,
         res.data_ptr(), out.data_ptr(), n, rows, k, n, dt, _dtype(res, "linear_gate_residual"), gp, gs, off, nb, rpb,
         _stream())
    return out


def gate_residual(x, h, gate=None, bias=None, offsets=None, rows_per_batch: int = 0, out=None) -> torch.Tensor:
    """x + fl(fl(h + bias) * gate[b]); x None -> the gated term alone."""
    rows, c = _rows_view(h, "gate_residual")
    dt = _dtype(h, "gate_residual")
    if x is not None and (x.shape != h.shape or x.dtype != h.dtype or not x.is_contiguous()):
        raise ValueError("gate_residual: x must match h")
    gp, gs, ng = _param_rows(gate, c, "gate_residual")
    bp, _, _ = _param_rows(bias, c, "gate_residual")
    off, nb, rpb = _batch(offsets, rows_per_batch, ng, rows, "gate_residual")
    out = torch.empty_like(h) if out is None else out
    call("t2h_gate_residual", x.data_ptr() if x is not None else None, h.data_ptr(), out.data_ptr(), bp, gp, gs,
         rows, c, dt, off, nb, rpb, _stream())
    return out


def timestep_embedding(t, dim: int = 256, max_period: float = 10000.0, dtype=torch.float32) -> torch.Tensor:
    _dev(t, "timestep_embedding")
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError("timestep_embedding: t must be contiguous float32")
    n = t.numel()
    out = torch.empty((n, dim), dtype=dtype, device=t.device)
    call("t2h_timestep_embedding", t.data_ptr(), out.data_ptr(), n, dim, _dtype(out, "timestep_embedding"),
         float(max_period), _stream())
    return out


def coords_to_offsets_async(coords, nbatch: int):
    """(offsets int64 [B+1], first_bad int64 [1]) enqueued, no sync."""
    _dev(coords, "coords_to_offsets")
    if coords.dtype != torch.int32 or coords.dim() != 2 or not coords.is_contiguous():
        raise ValueError("coords_to_offsets: coords must be contiguous int32 [N, C]")
    off = torch.empty(nbatch + 1, dtype=torch.int64, device=coords.device)
    bad = torch.empty(1, dtype=torch.int64, device=coords.device)
    call("t2h_coords_to_offsets", coords.data_ptr(), coords.shape[0], coords.shape[1], int(nbatch), off.data_ptr(),
         bad.data_ptr(), _stream())
    return off, bad


INT64_MAX = (1 << 63) - 1


def coords_to_offsets(coords, nbatch: int) -> torch.Tensor:
    """Offsets with the reference's errors (synchronises to read the check)."""
    off, bad = coords_to_offsets_async(coords, nbatch)
    fb = int(bad.item())
    if fb != INT64_MAX:
        if fb & 1:
            raise ValueError("SparseTensor: batch index out of range")
        raise ValueError("SparseTensor: batches must be ordered/contiguous")
    return off


def modulation_add(mod, modulation) -> torch.Tensor:
    _dev(mod, "modulation_add")
    if mod.dtype != torch.float32 or not mod.is_contiguous() or mod.dim() != 2:
        raise ValueError("modulation_add: mod must be contiguous float32 [N, W]")
    if modulation.numel() != mod.shape[1]:
        raise ValueError("modulation_add: width mismatch")
    out = torch.empty_like(mod)
    call("t2h_modulation_add", mod.data_ptr(), modulation.data_ptr(), out.data_ptr(), mod.shape[0], mod.shape[1],
         _stream())
    return out


# ---- flow-matching Euler sampler step -------------------------------------------
def flow_euler_workspace(rows: int, row_size: int, n_seg_offsets: int = 0) -> int:
    return int(_lib.load().t2h_flow_euler_workspace(int(rows), int(row_size), int(n_seg_offsets)))


def flow_euler_step(x_t, v_pos, t: float, t_prev: float, sigma_min: float, v_neg=None,
                    guidance_strength: float = 1.0, guidance_rescale: float = 0.0, seg_offsets=None,
                    pred_x0: bool = True, workspace=None, x_prev=None):
    """One Euler step of the flow sampler on x_t [rows, ...]: returns
    (x_prev, pred_x0 or None). seg_offsets: host token offsets (varlen state)."""
    _dev(x_t, "flow_euler_step")
    if not x_t.is_contiguous() or x_t.dim() < 1:
        raise ValueError("flow_euler_step: x_t must be contiguous")
    dt = _dtype(x_t, "flow_euler_step")
    for v in (v_pos, v_neg):
        if v is not None and (v.shape != x_t.shape or v.dtype != x_t.dtype or not v.is_contiguous()):
            raise ValueError("Tensor binop: size mismatch")
    rows = x_t.shape[0]
    rs = x_t.numel() // rows if rows else 1
    so = None
    nso = 0
    if seg_offsets is not None:
        so = np.ascontiguousarray(np.asarray(seg_offsets, dtype=np.int64))
        nso = int(so.size)
    x_prev = torch.empty_like(x_t) if x_prev is None else x_prev
    x0 = torch.empty_like(x_t) if pred_x0 else None
    ws = workspace
    rescale = v_neg is not None and guidance_strength not in (0.0, 1.0) and guidance_rescale > 0.0
    if rescale and ws is None:
        ws = torch.empty(flow_euler_workspace(rows, rs, nso), dtype=torch.uint8, device=x_t.device)
    p = lambda t: t.data_ptr() if t is not None else None
    call("t2h_flow_euler_step", x_t.data_ptr(), v_pos.data_ptr(), p(v_neg), x_prev.data_ptr(), p(x0), rows, rs, dt,
         float(t), float(t_prev), float(sigma_min), float(guidance_strength), float(guidance_rescale),
         so.ctypes.data if so is not None else None, nso, p(ws), ws.numel() if ws is not None else 0, _stream())
    return x_prev, x0


# ---- resident-block glue over one const buffer ----------------------------------
def _block_consts(consts, c: int, offs, what: str) -> int:
    _dev(consts, what)
    if consts.dtype != torch.float32 or not consts.is_contiguous():
        raise ValueError(f"{what}: consts must be contiguous float32")
    for off in offs:
        if off < 0 or off + 2 * c > consts.numel():
            raise ValueError(f"{what}: const pair at {off} outside a buffer of {consts.numel()} floats")
    return consts.data_ptr()


def _same_rows(x, h, what: str):
    rows, c = _rows_view(x, what)
    if h.shape != x.shape or h.dtype != x.dtype or not h.is_contiguous():
        raise ValueError(f"{what}: tensors must match x")
    return rows, c


def ln_mod_rows(x, dst, consts, off: int, mode: int) -> torch.Tensor:
    """Metal ln_mod_rows: dst = LN(x) with the const pair at `off` (mode 1
    modulate, mode 2 affine), eps 1e-6."""
    rows, c = _same_rows(x, dst, "ln_mod_rows")
    cp = _block_consts(consts, c, [off], "ln_mod_rows")
    call("t2h_ln_mod_rows", x.data_ptr(), dst.data_ptr(), cp, rows, c, int(off), int(mode), _dtype(x, "ln_mod_rows"),
         _stream())
    return dst


def gate_add_bias_rows(x, h, consts, off: int, use_gate: int) -> torch.Tensor:
    """Metal gate_add_bias_rows, in place: x += (h + bias) [* gate]."""
    rows, c = _same_rows(x, h, "gate_add_bias_rows")
    cp = _block_consts(consts, c, [off], "gate_add_bias_rows")
    call("t2h_gate_add_bias_rows", x.data_ptr(), h.data_ptr(), cp, rows, c, int(off), int(use_gate),
         _dtype(x, "gate_add_bias_rows"), _stream())
    return x


def block_join_ln(x, h, dst, consts, join_off: int, use_gate: int, norm_off: int, mode: int) -> torch.Tensor:
    """gate_add_bias_rows(join_off) then ln_mod_rows(norm_off) in one pass;
    x updated in place, dst = the normed rows."""
    rows, c = _same_rows(x, h, "block_join_ln")
    _same_rows(x, dst, "block_join_ln")
    cp = _block_consts(consts, c, [join_off, norm_off], "block_join_ln")
    call("t2h_block_join_ln", x.data_ptr(), h.data_ptr(), dst.data_ptr(), cp, rows, c, int(join_off), int(use_gate),
         int(norm_off), int(mode), _dtype(x, "block_join_ln"), _stream())
    return dst


def device_init(device: int = 0) -> None:
    call("t2h_device_init", int(device))


def version() -> int:
    return int(_lib.load().t2h_version())
