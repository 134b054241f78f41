"""numpy binding of the C oracle (oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker. The product path (libt2h.so and the
t2h package) never imports it.

Every wrapper takes/returns float32 numpy arrays (int32 for coords, int64 for
offsets) and raises ValueError where the reference raises `Error`.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ACT_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH = 0, 1, 2, 3   # modules/nn.mojo:582-585
OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3                # sparse/tensor.mojo:4-7

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_rng_next_u64.restype = ctypes.c_uint64
        L.orc_rng_next_f64.restype = ctypes.c_double
        L.orc_rng_normal.restype = ctypes.c_double
        L.orc_rmsnorm_scale.restype = ctypes.c_float
        L.orc_rope_freqs.restype = ctypes.c_int64
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.restype = ctypes.c_float
        for name in ("orc_layernorm", "orc_modulate", "orc_cal_offsets", "orc_binop_rows",
                     "orc_mod_shift_scale", "orc_multihead_rmsnorm",
                     "orc_rope_phases_from_positions", "orc_rope_phases_from_coords",
                     "orc_apply_rotary", "orc_rope_rotate", "orc_activation"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    if a.dtype == np.float32:
        return a.ctypes.data_as(_f32p)
    if a.dtype == np.int32:
        return a.ctypes.data_as(_i32p)
    if a.dtype == np.int64:
        return a.ctypes.data_as(_i64p)
    raise TypeError(a.dtype)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- seeded inputs (rng.mojo) --------------------------------------------
class Rng(ctypes.Structure):
    """xorshift64* seeded through splitmix64 (trellis2_mojo/rng.mojo:17-46)."""
    _fields_ = [("state", ctypes.c_uint64)]

    def __init__(self, seed: int):
        super().__init__()
        lib().orc_rng_init(ctypes.byref(self), ctypes.c_uint64(seed))

    def next_u64(self) -> int:
        return lib().orc_rng_next_u64(ctypes.byref(self))

    def next_f64(self) -> float:
        return lib().orc_rng_next_f64(ctypes.byref(self))

    def normal(self) -> float:
        return lib().orc_rng_normal(ctypes.byref(self))

    def randn(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        lib().orc_randn(ctypes.byref(self), _p(out), _i64(out.size),
                        ctypes.c_double(mean), ctypes.c_double(std))
        return out

    def uniform(self, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        lib().orc_uniform(ctypes.byref(self), _p(out), _i64(out.size),
                          ctypes.c_double(lo), ctypes.c_double(hi))
        return out


def randn(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    return Rng(seed).randn(shape, mean, std)


# ---- ops -------------------------------------------------------------------
def layernorm(x, eps: float = 1e-5, affine: bool = False, w=None, b=None) -> np.ndarray:
    x = _f32(x)
    c = x.shape[-1]
    out = np.empty_like(x)
    if affine:
        w, b = _f32(w), _f32(b)
        if w.size != c or b.size != c:
            raise ValueError("LayerNorm32: affine params mismatch")
    else:
        w = b = np.zeros(1, np.float32)
    rc = lib().orc_layernorm(_p(x), _p(out), _i64(x.size // c), _i64(c),
                             ctypes.c_double(eps), int(affine), _p(w), _p(b))
    if rc:
        raise ValueError("LayerNorm32: last dim mismatch")
    return out


def modulate(x, shift, scale) -> np.ndarray:
    """x [N, L, C], shift/scale [N, C] (modules/nn.mojo:660-689)."""
    x, shift, scale = _f32(x), _f32(shift), _f32(scale)
    n, l, c = x.shape
    if shift.size != n * c or scale.size != n * c:
        raise ValueError("modulate: shift/scale shape mismatch")
    out = np.empty_like(x)
    lib().orc_modulate(_p(x), _p(shift), _p(scale), _p(out), _i64(n), _i64(l), _i64(c))
    return out


def cal_offsets(coords, batch_size: int) -> np.ndarray:
    coords = np.ascontiguousarray(coords, dtype=np.int32)
    off = np.zeros(batch_size + 1, np.int64)
    rc = lib().orc_cal_offsets(_p(coords), _i64(coords.shape[0]), _i64(coords.shape[1]),
                               _i64(batch_size), _p(off))
    if rc == -1:
        raise ValueError("SparseTensor: batches must be ordered/contiguous")
    if rc == -2:
        raise ValueError("SparseTensor: batch index out of range")
    return off


def batch_broadcast_map(offsets) -> np.ndarray:
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    out = np.empty(int(offsets[-1]), np.int64)
    lib().orc_batch_broadcast_map(_p(offsets), _i64(offsets.size - 1), _p(out))
    return out


def binop_rows(x, other, row_map, op: int) -> np.ndarray:
    x, other = _f32(x), _f32(other)
    row_map = np.ascontiguousarray(row_map, dtype=np.int64)
    rows = x.shape[0]
    c = x.size // rows if rows else 0
    oc = other.size // other.shape[0]
    out = np.empty_like(x)
    if lib().orc_binop_rows(_p(x), _p(other), _p(row_map), _p(out), _i64(rows), _i64(c), _i64(oc), op):
        raise ValueError("Tensor._binop_rows: incompatible row size")
    return out


def binop_scalar(x, v: float, op: int, reverse: bool = False) -> np.ndarray:
    """Tensor._binop_scalar (sparse/tensor.mojo:200-203): x OP v, or v OP x
    when reverse."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_binop_scalar(_p(x), ctypes.c_float(v), _p(out), _i64(x.size), op, int(reverse))
    return out


def binop_flat(x, y, op: int) -> np.ndarray:
    x, y = _f32(x), _f32(y)
    if x.size != y.size:
        raise ValueError("Tensor binop: size mismatch")
    out = np.empty_like(x)
    lib().orc_binop_flat(_p(x), _p(y), _p(out), _i64(x.size), op)
    return out


def mod_shift_scale(h, shift, scale, offsets) -> np.ndarray:
    h, shift, scale = _f32(h), _f32(shift), _f32(scale)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    rows, c = h.shape
    out = np.empty_like(h)
    lib().orc_mod_shift_scale(_p(h), _p(shift), _p(scale), _p(offsets), _i64(offsets.size - 1),
                              _p(out), _i64(rows), _i64(c))
    return out


def modulation_add(mod, modulation) -> np.ndarray:
    mod, modulation = _f32(mod), _f32(modulation)
    out = np.empty_like(mod)
    lib().orc_modulation_add(_p(mod), _p(modulation), _p(out), _i64(mod.shape[0]), _i64(mod.shape[1]))
    return out


def multihead_rmsnorm(x, gamma, nthreads: int = 1) -> np.ndarray:
    x, gamma = _f32(x), _f32(gamma)
    h, d = x.shape[-2], x.shape[-1]
    rows = x.size // (h * d)
    out = np.empty_like(x)
    lib().orc_multihead_rmsnorm(_p(x), _p(gamma), _p(out), _i64(rows), _i64(h), _i64(d), int(nthreads))
    return out


def rmsnorm_scale(d: int) -> float:
    return lib().orc_rmsnorm_scale(_i64(d))


def rope_freqs(head_dim: int, dim: int = 3, freq_lo: float = 1.0, freq_hi: float = 10000.0) -> np.ndarray:
    if head_dim % 2:
        raise ValueError("RotaryPositionEmbedder: head_dim must be even")
    fd = head_dim // 2 // dim
    out = np.zeros(max(fd, 1), np.float32)
    lib().orc_rope_freqs(_i64(head_dim), _i64(dim), ctypes.c_double(freq_lo), ctypes.c_double(freq_hi), _p(out))
    return out[:fd]


def rope_phases_from_positions(pos, head_dim: int, freqs) -> np.ndarray:
    pos, freqs = _f32(pos), _f32(freqs)
    l, dim = pos.shape
    out = np.empty((l, head_dim // 2, 2), np.float32)
    lib().orc_rope_phases_from_positions(_p(pos), _i64(l), _i64(dim), _i64(head_dim),
                                         _p(freqs if freqs.size else np.zeros(1, np.float32)),
                                         _i64(freqs.size), _p(out))
    return out


def rope_phases_from_coords(coords, head_dim: int, freqs, dim: int = 3) -> np.ndarray:
    coords = np.ascontiguousarray(coords, dtype=np.int32)
    freqs = _f32(freqs)
    n, ncols = coords.shape
    out = np.empty((n, head_dim // 2, 2), np.float32)
    rc = lib().orc_rope_phases_from_coords(_p(coords), _i64(n), _i64(ncols), _i64(dim), _i64(head_dim),
                                           _p(freqs if freqs.size else np.zeros(1, np.float32)),
                                           _i64(freqs.size), _p(out))
    if rc:
        raise ValueError("rope: coords must have dim+1 columns")
    return out


def grid_positions(r: int) -> np.ndarray:
    out = np.empty((r * r * r, 3), np.float32)
    lib().orc_grid_positions(_i64(r), _p(out))
    return out


def apply_rotary(x, phases) -> np.ndarray:
    x, phases = _f32(x), _f32(phases)
    n, l, h, d = x.shape
    if phases.shape[0] != l or phases.shape[1] != d // 2:
        raise ValueError("apply_rotary_embedding: phases shape mismatch")
    out = np.empty_like(x)
    lib().orc_apply_rotary(_p(x), _p(phases), _p(out), _i64(n), _i64(l), _i64(h), _i64(d))
    return out


def rope_rotate(feats, phases, nthreads: int = 1) -> np.ndarray:
    feats, phases = _f32(feats), _f32(phases)
    n = feats.shape[0]
    d = feats.shape[-1]
    h = feats.size // (n * d) if n else 0
    out = np.empty_like(feats)
    lib().orc_rope_rotate(_p(feats), _p(phases), _p(out), _i64(n), _i64(h), _i64(d), int(nthreads))
    return out


def activation(x, kind: int, nthreads: int = 1) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    if lib().orc_activation(_p(x), _p(out), _i64(x.size), int(kind), int(nthreads)):
        raise ValueError("unknown activation")
    return out


def add_bias(x, bias) -> np.ndarray:
    x, bias = _f32(x), _f32(bias)
    c = bias.size
    out = np.empty_like(x)
    lib().orc_add_bias(_p(x), _p(bias), _p(out), _i64(x.size // c), _i64(c))
    return out


def gate(x, g) -> np.ndarray:
    """x [N, L, C] * g [N, C] (modules/transformer/modulated.mojo:22-33)."""
    x, g = _f32(x), _f32(g)
    n, l, c = x.shape
    out = np.empty_like(x)
    lib().orc_gate(_p(x), _p(g), _p(out), _i64(n), _i64(l), _i64(c))
    return out


def timestep_embedding(t, dim: int = 256, max_period: float = 10000.0) -> np.ndarray:
    t = _f32(t).reshape(-1)
    out = np.empty((t.size, dim), np.float32)
    lib().orc_timestep_embedding(_p(t), _i64(t.size), _i64(dim), ctypes.c_double(max_period), _p(out))
    return out


def round_f16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_round_f16(_p(x), _p(out), _i64(x.size))
    return out


def round_bf16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_round_bf16(_p(x), _p(out), _i64(x.size))
    return out


# ---- compositions used by the parity tests --------------------------------
def ln_modulate(x, shift, scale, offsets=None, eps: float = 1e-6) -> np.ndarray:
    """norm (non-affine) then batch-gathered modulate: the block's
    `modulate(norm1(x), shift, scale)` / `_mod_shift_scale(norm1(h), ...)`."""
    x = _f32(x)
    rows, c = x.shape
    n = layernorm(x, eps=eps)
    shift = _f32(shift).reshape(-1, c)
    scale = _f32(scale).reshape(-1, c)
    if offsets is None:
        offsets = np.array([0, rows], np.int64)
    return mod_shift_scale(n, shift, scale, offsets)


def qk_rms_rope(q, k, gamma_q, gamma_k, phases, bias_q=None, bias_k=None,
                use_rms: bool = True, use_rope: bool = True, nthreads: int = 1):
    """bias -> MultiHeadRMSNorm -> RoPE on q and k [rows, H, D] with per-row
    phases [rows, D/2, 2] (sparse/attention/modules.mojo:206-212,
    gpu/attention.mojo:507-563 order)."""
    q, k = _f32(q), _f32(k)
    if bias_q is not None:
        q = (q + _f32(bias_q).reshape(q.shape[1:])).astype(np.float32)
    if bias_k is not None:
        k = (k + _f32(bias_k).reshape(k.shape[1:])).astype(np.float32)
    if use_rms:
        q = multihead_rmsnorm(q, gamma_q, nthreads)
        k = multihead_rmsnorm(k, gamma_k, nthreads)
    if use_rope:
        q = rope_rotate(q, phases, nthreads)
        k = rope_rotate(k, phases, nthreads)
    return q, k


def gelu_tanh_bias(h, bias=None, nthreads: int = 1) -> np.ndarray:
    h = _f32(h)
    v = add_bias(h, bias) if bias is not None else h
    return activation(v, ACT_GELU_TANH, nthreads)


def gate_residual(x, h, gate_rows, offsets=None, bias=None) -> np.ndarray:
    """x + fl(fl(h [+ bias]) * gate[b(r)]) — the block's `y + _gate(h, g)` /
    `x + h.elemwise_batch(gate, MUL)`, with gpu/block.mojo:86-110's
    out-linear bias fold when bias is given."""
    x, h = _f32(x), _f32(h)
    rows, c = x.shape
    if bias is not None:
        h = add_bias(h, bias)
    if gate_rows is not None:
        g = _f32(gate_rows).reshape(-1, c)
        if offsets is None:
            offsets = np.array([0, rows], np.int64)
        h = binop_rows(h, g, batch_broadcast_map(offsets), OP_MUL)
    return binop_flat(x, h, OP_ADD)


def cross_block(x, m, norm2_w, norm2_b, self_attn, cross_attn, mlp, offsets=None, eps: float = 1e-6,
                store=None) -> np.ndarray:
    """Glue of the CPU cross block on feats [rows, C]: the order of
    ModulatedSparseTransformerCrossBlock.forward (sparse/transformer/modulated.mojo:219-226)
    and of the dense block (modules/transformer/modulated.mojo:186-200, _tail 192-200).
    m: the six adaLN chunks [B, C]; the chains are numpy callables returning complete
    outputs. `store` rounds a tensor to the storage type where the device path stores one."""
    rnd = store or (lambda a: a)
    x = _f32(x)
    rows = x.shape[0]
    if offsets is None:
        offsets = np.array([0, rows], np.int64)
    h = rnd(ln_modulate(x, m[0], m[1], offsets, eps))
    h = rnd(_f32(self_attn(h)))
    y = rnd(gate_residual(x, h, m[2], offsets))
    h2 = rnd(layernorm(y, eps, affine=True, w=norm2_w, b=norm2_b))
    h2 = rnd(_f32(cross_attn(h2)))
    y = rnd(gate_residual(y, h2, None))
    h3 = rnd(ln_modulate(y, m[3], m[4], offsets, eps))
    h3 = rnd(_f32(mlp(h3)))
    return rnd(gate_residual(y, h3, m[5], offsets))


def cross_block_resident(x, bk, self_chain, cross_chain, mlp_chain, eps: float = 1e-6, store=None) -> np.ndarray:
    """Glue of gpu_cross_block_enqueue (gpu/block.mojo:304-397) with the const
    buffer bk [12C] (layout 255-289): the out-linear biases are folded into the
    joins, the chains return their outputs without them."""
    rnd = store or (lambda a: a)
    x = _f32(x)
    c = x.shape[1]
    bk = _f32(bk).reshape(-1)
    v = lambda k: bk[k * c:(k + 1) * c]
    hs = rnd(ln_modulate(x, v(0), v(1), None, eps))                 # ln_mod_rows off 0, mode 1
    x = rnd(gate_residual(x, rnd(_f32(self_chain(hs))), v(3), bias=v(2)))   # off 2C, gate
    hs = rnd(layernorm(x, eps, affine=True, w=v(4), b=v(5)))        # off 4C, mode 2
    x = rnd(gate_residual(x, rnd(_f32(cross_chain(hs))), None, bias=v(6)))  # off 6C, ungated
    hs = rnd(ln_modulate(x, v(8), v(9), None, eps))                 # off 8C, mode 1
    return rnd(gate_residual(x, rnd(_f32(mlp_chain(hs))), v(11), bias=v(10)))  # off 10C, gate


def linear(a, w, bias=None, act=None, nthreads: int = 8) -> np.ndarray:
    """act(a @ w^T + bias): gemm_tiled / gemm_tiled_f16sh (gpu/linear.mojo:
    108-160, 326-388; k summed in order, one f32 rounding per step), then the
    bias add and activation of gelu_tanh_bias (662-684) / activation
    (modules/nn.mojo:588-647). a [..., k], w [n, k]."""
    a, w = _f32(a), _f32(w)
    k = w.shape[1]
    a2 = a.reshape(-1, k)
    out = np.empty((a2.shape[0], w.shape[0]), np.float32)
    lib().orc_linear(_p(a2), _p(w), _p(out), _i64(a2.shape[0]), _i64(w.shape[0]), _i64(k), int(nthreads))
    if bias is not None:
        out = add_bias(out, bias)
    if act is not None and act >= 0:
        out = activation(out, act, nthreads)
    return out.reshape(*a.shape[:-1], w.shape[0])


def pack_q(q, l: int, h: int, d: int, mp: int, stride: int) -> np.ndarray:
    """pack_q_z (gpu/attention.mojo:566-594): q rows `stride` apart -> qh
    [h, mp, d] scaled by 1/sqrt(f32(d)), pad rows zero."""
    q = _f32(q).reshape(-1)
    out = np.empty((h, mp, d), np.float32)
    lib().orc_pack_q(_p(q), _p(out), _i64(l), _i64(h), _i64(d), _i64(mp), _i64(stride))
    return out


def pack_kv(qkv, l: int, h: int, d: int, lp: int):
    """pack_kv_z (gpu/attention.mojo:634-662): qkv [l, 3, h, d] -> kt [h, d, lp]
    (transposed) and vh [h, lp, d], pads zero."""
    qkv = _f32(qkv).reshape(-1)
    kt = np.empty((h, d, lp), np.float32)
    vh = np.empty((h, lp, d), np.float32)
    lib().orc_pack_kv(_p(qkv), _p(kt), _p(vh), _i64(l), _i64(h), _i64(d), _i64(lp))
    return kt, vh


def bias_rms_rope_qkv(qkv, h: int, d: int, bias, gamma_q, gamma_k, phases, use_rms: bool = True,
                      use_rope: bool = True) -> np.ndarray:
    """bias_rms_rope_qkv (gpu/attention.mojo:507-563) on qkv [rows, 3, h, d]:
    + bias [3hd] on q, k and v, then RMS-normalise and rotate q and k."""
    qkv = _f32(qkv).reshape(-1, 3, h, d)
    if bias is not None:
        qkv = (qkv + _f32(bias).reshape(3, h, d)).astype(np.float32)
    q, k = qk_rms_rope(qkv[:, 0], qkv[:, 1], gamma_q, gamma_k, phases, use_rms=use_rms, use_rope=use_rope)
    return np.stack([q, k, qkv[:, 2]], axis=1).astype(np.float32)


def attn_pack(qkv, h: int, d: int, mp: int, lp: int, bias=None, gamma_q=None, gamma_k=None, phases=None):
    """The self-attention chain's epilogue: bias_rms_rope_qkv, pack_q_z and
    pack_kv_z in the order of gpu/attention.mojo:987-1013, all in f32.
    Returns (qh, kt, vh)."""
    rows = _f32(qkv).reshape(-1, 3 * h * d).shape[0]
    e = bias_rms_rope_qkv(qkv, h, d, bias, gamma_q, gamma_k, phases, use_rms=gamma_q is not None,
                          use_rope=phases is not None)
    e = e.reshape(rows, 3 * h * d)
    qh = pack_q(e, rows, h, d, mp, 3 * h * d)
    kt, vh = pack_kv(e, rows, h, d, lp)
    return qh, kt, vh


# ---- FlowEulerSampler (samplers/flow_euler.mojo) --------------------------------
GUIDANCE_NONE, GUIDANCE_CFG, GUIDANCE_CFG_INTERVAL = 0, 1, 2   # flow_euler.mojo:27-29


def flow_v_to_xstart(x, v, t: float, sigma_min: float) -> np.ndarray:
    x, v = _f32(x), _f32(v)
    out = np.empty_like(x)
    lib().orc_flow_v_to_xstart(_p(x), _p(v), _p(out), _i64(x.size), ctypes.c_double(t), ctypes.c_double(sigma_min))
    return out


def flow_cfg(pos, neg, g: float) -> np.ndarray:
    pos, neg = _f32(pos), _f32(neg)
    out = np.empty_like(pos)
    lib().orc_flow_cfg(_p(pos), _p(neg), _p(out), _i64(pos.size), ctypes.c_double(g))
    return out


def flow_rescale(x_t, pred, pred_pos, t: float, sigma_min: float, guidance_rescale: float,
                 seg_offsets=None) -> np.ndarray:
    """_rescale_pred on x_t [rows, ...]: one segment per row (dense), or the
    token segments seg_offsets (varlen)."""
    x_t, pred, pred_pos = _f32(x_t), _f32(pred), _f32(pred_pos)
    rows = x_t.shape[0]
    rs = x_t.size // rows if rows else 0
    so = np.ascontiguousarray(seg_offsets if seg_offsets is not None else np.zeros(0), dtype=np.int64)
    out = np.empty_like(x_t)
    lib().orc_flow_rescale(_p(x_t), _p(pred), _p(pred_pos), _p(out), _i64(rows), _i64(rs), ctypes.c_double(t),
                           ctypes.c_double(sigma_min), ctypes.c_double(guidance_rescale), _p(so) if so.size else None,
                           _i64(so.size))
    return out


def flow_step(x, v, t: float, t_prev: float) -> np.ndarray:
    x, v = _f32(x), _f32(v)
    out = np.empty_like(x)
    lib().orc_flow_step(_p(x), _p(v), _p(out), _i64(x.size), ctypes.c_double(t), ctypes.c_double(t_prev))
    return out


def flow_t_seq(steps: int, rescale_t: float):
    """t_seq of _sample_impl (flow_euler.mojo:195-198), float64."""
    out = []
    for i in range(steps + 1):
        t = 1.0 - float(i) / float(steps)
        out.append(rescale_t * t / (1.0 + (rescale_t - 1.0) * t))
    return out


def flow_inference(model, x_t, t: float, mode: int, g: float, lo: float, hi: float, gr: float, sigma_min: float,
                   seg_offsets=None) -> np.ndarray:
    """_inference (flow_euler.mojo:151-181); model(x_t, t1000, use_neg_cond)."""
    use_cfg = mode == GUIDANCE_CFG
    if mode == GUIDANCE_CFG_INTERVAL:
        use_cfg = lo <= t <= hi
    if not use_cfg or g == 1.0:
        return _f32(model(x_t, 1000.0 * t, False))
    if g == 0.0:
        return _f32(model(x_t, 1000.0 * t, True))
    pos = _f32(model(x_t, 1000.0 * t, False))
    neg = _f32(model(x_t, 1000.0 * t, True))
    pred = flow_cfg(pos, neg, g)
    if gr > 0.0:
        return flow_rescale(x_t, pred, pos, t, sigma_min, gr, seg_offsets)
    return pred


def flow_sample(model, noise, steps: int, rescale_t: float, sigma_min: float, mode: int = GUIDANCE_NONE,
                g: float = 1.0, lo: float = 0.0, hi: float = 1.0, gr: float = 0.0, seg_offsets=None):
    """_sample_impl (flow_euler.mojo:183-214). Returns (samples, pred_x_t list, pred_x_0 list)."""
    sample = _f32(noise).copy()
    ts = flow_t_seq(steps, rescale_t)
    xs, x0s = [], []
    for i in range(steps):
        t, tp = ts[i], ts[i + 1]
        v = flow_inference(model, sample, t, mode, g, lo, hi, gr, sigma_min, seg_offsets)
        x0s.append(flow_v_to_xstart(sample, v, t, sigma_min))
        sample = flow_step(sample, v, t, tp)
        xs.append(sample.copy())
    return sample, xs, x0s
