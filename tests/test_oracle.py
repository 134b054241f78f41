"""Pins for the C oracle (CPU only).

Each check is independent of the oracle's own code: the reference's golden
values (tests/test_runtime.mojo:35-47, tests/parity/test_sparse_basic.mojo),
float64 closed forms, brute force on tiny inputs, numpy's IEEE float32
elementwise arithmetic (for the ops that are exact sequences of f32 roundings),
and identities (RoPE composition / norm preservation, GELU odd part). The
`mutant` tests show that the checks catch plausible mistakes (a dropped term,
a wrong sign, an off-by-one variance): the same check applied to a mutated
restatement fails.
"""
import math

import numpy as np
import pytest
import torch

import oracle as orc


# ---- RNG: tests/test_runtime.mojo:35-47 ----------------------------------------
def test_rng_golden():
    r = orc.Rng(1337)
    assert [r.next_u64() for _ in range(3)] == [76748464051394776, 17093336004959153412, 4605377540300676664]


def test_randn_deterministic():
    a, b = orc.Rng(42), orc.Rng(42)
    ta, tb = a.randn((2, 3, 4)), b.randn((2, 3, 4))
    assert np.array_equal(ta, tb) and a.state == b.state
    # Box-Muller closed form from the raw stream (rng.mojo:41-46)
    r = orc.Rng(7)
    u = [(r.next_u64() >> 11) * (1.0 / 2 ** 53) for _ in range(2)]
    want = math.sqrt(-2.0 * math.log(u[0])) * math.cos(6.283185307179586 * u[1])
    assert orc.Rng(7).normal() == want
    big = orc.randn(1, (200000,))
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


# ---- SparseTensor layout / gather: tests/parity/test_sparse_basic.mojo ----------
COORDS = np.array([[0, 0, 0, 0], [0, 1, 0, 1], [1, 0, 1, 0], [1, 1, 1, 1], [1, 1, 0, 0]], np.int32)
FEATS = np.arange(1, 11, dtype=np.float32).reshape(5, 2)


def test_sparse_basic_layout():
    off = orc.cal_offsets(COORDS, 2)
    assert off.tolist() == [0, 2, 5]                                  # seqlen 2, 3 (:149-158)
    assert orc.batch_broadcast_map(off).tolist() == [0, 0, 1, 1, 1]   # bm[0]=0, bm[2]=1, bm[4]=1 (:55-59)


def test_sparse_basic_elemwise_batch():
    rm = orc.batch_broadcast_map(orc.cal_offsets(COORDS, 2))
    b = np.array([[10, 20], [100, 200]], np.float32)
    y = orc.binop_rows(FEATS, b, rm, orc.OP_ADD).reshape(-1)
    assert y[0] == 11.0 and y[9] == 210.0                              # (:263-265)
    assert orc.binop_rows(FEATS, b, rm, orc.OP_MUL).reshape(-1)[1] == 40.0   # (:266-267)
    s = orc.binop_rows(FEATS, np.array([[10], [100]], np.float32), rm, orc.OP_ADD).reshape(-1)
    assert s[0] == 11.0 and s[4] == 105.0                              # (:81-84)
    assert orc.binop_rows(FEATS, b, rm, orc.OP_ADD).reshape(-1)[1] == 22.0   # (:86-89)


def test_sparse_contiguity_enforced():
    bad = np.zeros((2, 4), np.int32)
    bad[0, 0] = 1
    with pytest.raises(ValueError, match="ordered/contiguous"):
        orc.cal_offsets(bad, 2)                                        # (:161-171)
    bad = np.zeros((2, 4), np.int32)
    bad[1, 0] = 2
    with pytest.raises(ValueError, match="out of range"):
        orc.cal_offsets(bad, 2)


def test_offsets_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(50):
        nb = int(rng.integers(1, 6))
        counts = rng.integers(0, 5, nb)
        coords = np.zeros((counts.sum(), 4), np.int32)
        coords[:, 0] = np.repeat(np.arange(nb), counts)
        assert orc.cal_offsets(coords, nb).tolist() == [0] + np.cumsum(counts).tolist()
        assert orc.batch_broadcast_map(orc.cal_offsets(coords, nb)).tolist() == coords[:, 0].tolist()


# ---- exact f32 sequences: numpy float32 ufuncs round each step -------------------
def test_modulate_exact_f32():
    x = orc.randn(1, (3, 40, 64))
    sh, sc = orc.randn(2, (3, 64)), orc.randn(3, (3, 64))
    want = x * (np.float32(1) + sc[:, None, :]) + sh[:, None, :]
    assert np.array_equal(orc.modulate(x, sh, sc), want.astype(np.float32))
    off = np.array([0, 40, 80, 120], np.int64)
    assert np.array_equal(orc.mod_shift_scale(x.reshape(-1, 64), sh, sc, off), want.reshape(-1, 64))


def test_gate_and_residual_exact_f32():
    x, h = orc.randn(4, (2, 30, 32)), orc.randn(5, (2, 30, 32))
    g, b = orc.randn(6, (2, 32)), orc.randn(7, (32,))
    assert np.array_equal(orc.gate(h, g), h * g[:, None, :])
    off = np.array([0, 30, 60], np.int64)
    want = x.reshape(-1, 32) + ((h.reshape(-1, 32) + b) * np.repeat(g, 30, axis=0))
    assert np.array_equal(orc.gate_residual(x.reshape(-1, 32), h.reshape(-1, 32), g, offsets=off, bias=b), want)


_NP_OPS = {orc.OP_ADD: np.add, orc.OP_SUB: np.subtract, orc.OP_MUL: np.multiply, orc.OP_DIV: np.divide}


def test_binop_rows_every_op_exact_f32():
    """Tensor._binop_rows (sparse/tensor.mojo:205-219) for all four ops, with
    [B, C] rows and per-batch scalars [B, 1], over offsets with an empty
    batch: self OP other[row_map[r]] is one IEEE f32 op per element, so numpy
    float32 gives the same bits. The swapped operand order (other OP self) of
    SUB and DIV, and a row map shifted by one batch, both fail the check."""
    x = orc.randn(2000, (37, 24))
    other = orc.randn(2001, (3, 24), mean=1.5)     # away from 0 for DIV
    offsets = np.array([0, 10, 10, 37], np.int64)   # batch 1 is empty
    rm = orc.batch_broadcast_map(offsets)
    assert rm.tolist() == [0] * 10 + [2] * 27
    for op, f in _NP_OPS.items():
        assert np.array_equal(orc.binop_rows(x, other, rm, op), f(x, other[rm])), op
        s = other[:, :1].copy()
        assert np.array_equal(orc.binop_rows(x, s, rm, op), f(x, s[rm])), op
    for op in (orc.OP_SUB, orc.OP_DIV):
        got = orc.binop_rows(x, other, rm, op)
        assert not np.array_equal(got, _NP_OPS[op](other[rm], x))            # swapped operands
        assert not np.array_equal(got, _NP_OPS[op](x, other[np.maximum(rm - 1, 0)]))   # shifted map
    with pytest.raises(ValueError, match="incompatible row size"):
        orc.binop_rows(x, other[:, :5], rm, orc.OP_ADD)


def test_binop_flat_and_scalar_every_op_exact_f32():
    """_binop_flat (sparse/tensor.mojo:193-198) and _binop_scalar with its
    reverse form (200-203, _opscalar_span 469-524): x OP v, or v OP x for
    reverse SUB/DIV; reverse ADD/MUL equal the forward form (commutative).
    The forward result of SUB/DIV differs from the reverse one, so an
    operand swap in either form fails."""
    x = orc.randn(2002, (5, 131))       # 655 elements: SIMD body and scalar tail
    y = orc.randn(2003, (5, 131), mean=-2.0)
    v = np.float32(0.37)
    for op, f in _NP_OPS.items():
        assert np.array_equal(orc.binop_flat(x, y, op), f(x, y)), op
        assert np.array_equal(orc.binop_scalar(x, float(v), op), f(x, v)), op
        rev = orc.binop_scalar(x, float(v), op, reverse=True)
        assert np.array_equal(rev, f(v, x) if op in (orc.OP_SUB, orc.OP_DIV) else f(x, v)), op
    for op in (orc.OP_SUB, orc.OP_DIV):
        assert not np.array_equal(orc.binop_flat(x, y, op), _NP_OPS[op](y, x))
        assert not np.array_equal(orc.binop_scalar(x, float(v), op), _NP_OPS[op](v, x))
    with pytest.raises(ValueError, match="size mismatch"):
        orc.binop_flat(x, y[:, :3], orc.OP_ADD)


def test_modulation_add_exact_f32():
    """Modulation.chunks, share_mod branch (sparse/transformer/modulated.mojo:
    41-48): m[r, j] = mod[r, j] + modulation[j], one f32 add, broadcast over
    rows. Adding only the first C-wide chunk of modulation to all six chunks,
    or pairing row r of mod with a row-offset slice, fails the check."""
    c = 48
    mod = orc.randn(2004, (3, 6 * c))
    modulation = orc.randn(2005, (6 * c,), std=0.5)
    got = orc.modulation_add(mod, modulation)
    assert np.array_equal(got, mod + modulation[None, :])
    assert not np.array_equal(got, mod + np.tile(modulation[:c], 6)[None, :])
    assert not np.array_equal(got, mod + np.roll(modulation, c)[None, :])


# ---- LayerNorm: float64 closed form ---------------------------------------------
def _ln64(x, eps, w=None, b=None):
    x = x.astype(np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)    # biased variance
    y = (x - m) / np.sqrt(v + eps)
    return y * w + b if w is not None else y


def _rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b) / np.maximum(np.abs(b), 1.0)))


def test_layernorm_float64():
    x = orc.randn(11, (64, 1536), mean=0.7, std=2.5)
    assert _rel(orc.layernorm(x, 1e-6), _ln64(x, 1e-6)) < 2e-6
    w, b = orc.randn(12, (1536,), mean=1.0, std=0.1), orc.randn(13, (1536,), std=0.1)
    assert _rel(orc.layernorm(x, 1e-5, True, w, b), _ln64(x, 1e-5, w, b)) < 2e-6
    assert _rel(orc.layernorm(x[:, :13], 1e-6), _ln64(x[:, :13], 1e-6)) < 2e-6   # scalar tail
    assert np.all(orc.layernorm(np.full((2, 24), 5.0, np.float32), 1e-6) == 0.0)
    t = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (1536,), eps=1e-6).numpy()
    assert _rel(orc.layernorm(x, 1e-6), t) < 2e-6


def test_layernorm_mutant_unbiased_variance_is_caught():
    x = orc.randn(14, (16, 64))
    xd = x.astype(np.float64)
    m = xd.mean(-1, keepdims=True)
    mutant = (xd - m) / np.sqrt(((xd - m) ** 2).sum(-1, keepdims=True) / 63 + 1e-6)
    assert _rel(mutant, _ln64(x, 1e-6)) > 1e-3
    assert _rel(orc.layernorm(x, 1e-6), _ln64(x, 1e-6)) < 2e-6


# ---- MultiHeadRMSNorm -------------------------------------------------------------
def test_rmsnorm_float64():
    x = orc.randn(21, (100, 12, 128), std=3.0)
    g = orc.randn(22, (12, 128), mean=1.0, std=0.02)
    xd = x.astype(np.float64)
    want = xd / np.maximum(np.linalg.norm(xd, axis=-1, keepdims=True), 1e-12) * g * math.sqrt(128)
    assert _rel(orc.multihead_rmsnorm(x, g), want) < 2e-6
    assert orc.rmsnorm_scale(128) == np.float32(math.sqrt(128))
    # gamma = 1: every head has norm sqrt(D)
    y = orc.multihead_rmsnorm(x, np.ones((12, 128), np.float32)).astype(np.float64)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), math.sqrt(128), rtol=1e-6)
    assert np.all(orc.multihead_rmsnorm(np.zeros((2, 12, 128), np.float32), g) == 0.0)   # 1e-12 clamp
    # parallel chunks give identical bits (sparse/attention/modules.mojo:96-101)
    assert np.array_equal(orc.multihead_rmsnorm(x, g, nthreads=4), orc.multihead_rmsnorm(x, g, nthreads=1))


# ---- RoPE -------------------------------------------------------------------------
def test_rope_freqs_closed_form():
    f = orc.rope_freqs(128)
    assert f.size == 21                                   # 128 // 2 // 3 (rope.mojo:32)
    want = 1.0 / 10000.0 ** (np.arange(21) / 21.0)
    np.testing.assert_allclose(f, want, rtol=3e-7)
    assert f[0] == 1.0
    assert orc.rope_freqs(64).size == 10


def test_rope_slot_mapping_brute_force():
    """slot p < 63: axis p // 21, freq p % 21; slot 63 = identity pad (D2)."""
    d = 128
    f = orc.rope_freqs(d)
    pos = np.array([[3.0, 7.0, 11.0], [0.0, 0.0, 0.0], [127.0, 64.0, 1.0]], np.float32)
    ph = orc.rope_phases_from_positions(pos, d, f)
    for r in range(3):
        for p in range(64):
            if p < 63:
                ang = np.float32(pos[r, p // 21] * f[p % 21])           # f32 product
                assert abs(ph[r, p, 0] - math.cos(float(ang))) < 2e-7
                assert abs(ph[r, p, 1] - math.sin(float(ang))) < 2e-7
            else:
                assert ph[r, p, 0] == 1.0 and ph[r, p, 1] == 0.0
    assert np.all(ph[1, :, 0] == 1.0) and np.all(ph[1, :, 1] == 0.0)   # position 0 = identity
    co = np.concatenate([np.zeros((3, 1), np.int32), pos.astype(np.int32)], 1)
    assert np.array_equal(orc.rope_phases_from_coords(co, d, f), ph)    # int coords == float positions


def test_grid_positions():
    g = orc.grid_positions(4)
    for l in range(64):
        assert g[l].tolist() == [l // 16, (l // 4) % 4, l % 4]           # meshgrid 'ij'


def _rotate64(x, ph):
    z = x.astype(np.float64).reshape(*x.shape[:-1], -1, 2)
    c = (z[..., 0] + 1j * z[..., 1]) * (ph[..., 0] + 1j * ph[..., 1])
    return np.stack([c.real, c.imag], -1).reshape(x.shape)


def test_rope_rotate_complex_and_composition():
    d, n, h = 128, 40, 12
    x = orc.randn(31, (n, h, d))
    co = np.zeros((n, 4), np.int32)
    co[:, 1:] = np.random.default_rng(1).integers(0, 128, (n, 3))
    f = orc.rope_freqs(d)
    ph = orc.rope_phases_from_coords(co, d, f)
    out = orc.rope_rotate(x, ph)
    assert _rel(out, _rotate64(x, ph.astype(np.float64)[:, None])) < 2e-6
    z, o = x.reshape(n, h, 64, 2).astype(np.float64), out.reshape(n, h, 64, 2).astype(np.float64)
    np.testing.assert_allclose(np.hypot(o[..., 0], o[..., 1]), np.hypot(z[..., 0], z[..., 1]), rtol=2e-6, atol=1e-7)
    # composition R(a) R(b) = R(a + b) for integer positions a, b
    co2 = np.zeros((n, 4), np.int32)
    co2[:, 1:] = np.random.default_rng(2).integers(0, 64, (n, 3))
    co3 = co.copy()
    co3[:, 1:] = co[:, 1:] + co2[:, 1:]
    two = orc.rope_rotate(orc.rope_rotate(x, ph), orc.rope_phases_from_coords(co2, d, f))
    one = orc.rope_rotate(x, orc.rope_phases_from_coords(co3, d, f))
    assert _rel(two, one) < 2e-5
    # a sign mistake in the rotation breaks composition
    mut = x.reshape(n, h, 64, 2).copy()
    re, im = mut[..., 0].copy(), mut[..., 1].copy()
    c, s = ph[:, None, :, 0], ph[:, None, :, 1]
    mut[..., 0], mut[..., 1] = re * c + im * s, re * s + im * c
    assert _rel(mut.reshape(x.shape), _rotate64(x, ph.astype(np.float64)[:, None])) > 1e-2


def test_apply_rotary_equals_rotate():
    """Dense apply_rotary (phases per l) and sparse _rotate (phases per row)
    use the same per-pair formula: identical bits."""
    l, h, d = 64, 4, 128
    x = orc.randn(41, (1, l, h, d))
    ph = orc.rope_phases_from_positions(orc.grid_positions(4), d, orc.rope_freqs(d))
    assert np.array_equal(orc.apply_rotary(x, ph)[0], orc.rope_rotate(x[0], ph))


# ---- activations ---------------------------------------------------------------
def test_gelu_tanh_float64_and_identities():
    x = orc.randn(51, (4096,), std=4.0)
    t = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    g = orc.activation(x, orc.ACT_GELU_TANH)
    assert _rel(g, t) < 3e-6
    assert orc.activation(np.zeros(1, np.float32), orc.ACT_GELU_TANH)[0] == 0.0
    gm = orc.activation(-x, orc.ACT_GELU_TANH)
    np.testing.assert_allclose(g.astype(np.float64) - gm, x, rtol=1e-5, atol=1e-6)   # odd part is x/2 * 2
    # mutant: dropping the cubic term is caught by the float64 check
    xd = x.astype(np.float64)
    mutant = 0.5 * xd * (1 + np.tanh(0.7978845608028654 * xd))
    assert _rel(mutant, t) > 1e-3
    # parallel chunks are bit-identical (nn.mojo:641-646)
    big = orc.randn(52, (1 << 18,))
    assert np.array_equal(orc.activation(big, 3, 4), orc.activation(big, 3, 1))


def test_other_activations_float64():
    x = orc.randn(53, (4096,), std=4.0)
    xt = torch.from_numpy(x).double()
    assert _rel(orc.activation(x, orc.ACT_RELU), torch.relu(xt).numpy()) == 0.0
    assert _rel(orc.activation(x, orc.ACT_SILU), torch.nn.functional.silu(xt).numpy()) < 3e-6
    assert _rel(orc.activation(x, orc.ACT_GELU), torch.nn.functional.gelu(xt).numpy()) < 3e-6
    with pytest.raises(ValueError, match="unknown activation"):
        orc.activation(x, 9)


# ---- timestep embedding -----------------------------------------------------------
@pytest.mark.parametrize("dim", [256, 255])
def test_timestep_float64(dim):
    t = np.array([0.0, 0.5, 1.0, 999.0], np.float32)
    e = orc.timestep_embedding(t, dim)
    half = dim // 2
    fr = np.exp(-math.log(10000.0) * np.arange(half) / half)
    ang = t[:, None].astype(np.float64) * fr
    want = np.concatenate([np.cos(ang), np.sin(ang)], 1)
    # the f32 angle carries ~|angle| * 6e-8 of rounding: compare within that
    assert np.max(np.abs(e[:, :2 * half] - want)) < 2e-4
    assert np.max(np.abs(e[:3, :2 * half] - want[:3])) < 2e-6
    assert np.all(e[0, :half] == 1.0) and np.all(e[0, half:2 * half] == 0.0)
    if dim % 2:
        assert np.all(e[:, -1] == 0.0)


# ---- storage rounding -------------------------------------------------------------
def test_f16_bf16_rounding_matches_torch():
    x = np.concatenate([orc.randn(61, (100000,), std=1000.0), orc.randn(62, (100000,), std=1e-5),
                        np.array([65504, 65520, 65519.99, 1e-8, -0.0, np.inf], np.float32)]).astype(np.float32)
    assert np.array_equal(orc.round_f16(x), torch.from_numpy(x).half().float().numpy())
    assert np.array_equal(orc.round_bf16(x), torch.from_numpy(x).bfloat16().float().numpy())


# ---- DiT cross-block glue: the two reference forms of one block ----------------
def _block_case(seed, rows=64, c=48):
    x = orc.randn(seed, (rows, c), std=2.0)
    m = [orc.randn(seed + 1 + i, (1, c), std=0.3) for i in range(6)]
    w2 = orc.randn(seed + 7, (c,), mean=1.0, std=0.2)
    b2 = orc.randn(seed + 8, (c,), std=0.2)
    biases = [orc.randn(seed + 9 + i, (c,), std=0.1) for i in range(3)]
    return x, m, w2, b2, biases


def _chains():
    self_chain = lambda h: (np.roll(h, 1, axis=0) * np.float32(0.5)).astype(np.float32)
    cross_chain = lambda h: (h[:, ::-1] * np.float32(-0.25)).astype(np.float32)
    mlp_chain = lambda h: orc.activation(h, orc.ACT_GELU_TANH)
    return self_chain, cross_chain, mlp_chain


def _bk(m, w2, b2, biases):
    c = w2.size
    z = np.zeros(c, np.float32)
    return np.concatenate([m[0].ravel(), m[1].ravel(), biases[0], m[2].ravel(), w2, b2, biases[1], z,
                           m[3].ravel(), m[4].ravel(), biases[2], m[5].ravel()]).astype(np.float32)


def test_block_resident_equals_cpu_order():
    """gpu/block.mojo folds each out-linear bias into its residual join
    (x + fl(h + bias) * gate); the CPU block adds it inside the chain
    (x + fl(fl(h + bias) * gate)). Both are the same f32 sequence, so the
    two restatements agree bit for bit, which pins the const-buffer pair
    order (a swapped shift/scale or gate/bias pair fails)."""
    x, m, w2, b2, biases = _block_case(900)
    sc, cc, mc = _chains()
    ab = lambda f, b: (lambda h: orc.add_bias(f(h), b))
    cpu = orc.cross_block(x, m, w2, b2, ab(sc, biases[0]), ab(cc, biases[1]), ab(mc, biases[2]))
    res = orc.cross_block_resident(x, _bk(m, w2, b2, biases), sc, cc, mc)
    assert np.array_equal(cpu, res)
    swapped = list(m)
    swapped[0], swapped[1] = m[1], m[0]
    assert not np.array_equal(orc.cross_block_resident(x, _bk(swapped, w2, b2, biases), sc, cc, mc), cpu)


def test_block_closed_forms():
    """Zero gates and a zero cross chain leave x unchanged; with gate1 = 1,
    identity chains and zero shift/scale the self join is x + LN(x), checked
    against float64."""
    x, m, w2, b2, biases = _block_case(950)
    c = x.shape[1]
    zero = lambda h: np.zeros_like(h)
    mz = [mm.copy() for mm in m]
    mz[2][:] = 0
    mz[5][:] = 0
    out = orc.cross_block(x, mz, w2, b2, lambda h: h, zero, lambda h: h)
    assert np.array_equal(out, x)
    m1 = [np.zeros((1, c), np.float32) for _ in range(6)]
    m1[2][:] = 1
    out = orc.cross_block(x, m1, w2, b2, lambda h: h, zero, zero)
    xd = x.astype(np.float64)
    ln = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6)
    assert np.max(np.abs(out - (xd + ln)) / np.maximum(np.abs(xd + ln), 1)) < 2e-6


def test_pack_block_consts_layout():
    """Host logic of t2h.block (torch CPU tensors): the const buffer follows
    gpu/block.mojo:255-289, a missing out bias is zeros."""
    from t2h import block

    x, m, w2, b2, biases = _block_case(990, c=16)
    bk = block.pack_block_consts([torch.from_numpy(mm) for mm in m], torch.from_numpy(w2), torch.from_numpy(b2),
                                 *[torch.from_numpy(b) for b in biases])
    assert np.array_equal(bk.numpy(), _bk(m, w2, b2, biases))
    bk0 = block.pack_block_consts([torch.from_numpy(mm) for mm in m], torch.from_numpy(w2), torch.from_numpy(b2))
    z = [np.zeros(16, np.float32)] * 3
    assert np.array_equal(bk0.numpy(), _bk(m, w2, b2, z))
    with pytest.raises(ValueError, match="expected 6 mod chunks"):
        block.pack_block_consts([torch.from_numpy(mm) for mm in m[:5]], torch.from_numpy(w2), torch.from_numpy(b2))


# ---- head-major attention packs: gpu/attention.mojo:566-594, 634-662 -----------
def test_packs_are_numpy_transposes():
    """pack_q_z / pack_kv_z restated, checked against numpy's own reshapes:
    qh[z, t] = q[t, z] * f32(1/sqrt(d)) (one f32 product), kt[z, e, t] =
    k[t, z, e], vh[z, t] = v[t, z], pads zero. A transposed kt (the
    [h, lp, d] layout) or a missing scale fails."""
    l, h, d, lp = 37, 3, 16, 64
    qkv = orc.randn(77, (l, 3, h, d))
    qh = orc.pack_q(qkv.reshape(l, -1), l, h, d, lp, 3 * h * d)
    kt, vh = orc.pack_kv(qkv, l, h, d, lp)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    want_q = np.zeros((h, lp, d), np.float32)
    want_q[:, :l] = (qkv[:, 0] * scale).transpose(1, 0, 2)
    want_k = np.zeros((h, d, lp), np.float32)
    want_k[:, :, :l] = qkv[:, 1].transpose(1, 2, 0)
    want_v = np.zeros((h, lp, d), np.float32)
    want_v[:, :l] = qkv[:, 2].transpose(1, 0, 2)
    assert np.array_equal(qh, want_q) and np.array_equal(kt, want_k) and np.array_equal(vh, want_v)
    assert not np.array_equal(kt, want_v.transpose(0, 2, 1))
    # cross-chain stride (q alone, rows h*d apart)
    q = orc.randn(78, (l, h, d))
    assert np.array_equal(orc.pack_q(q.reshape(l, -1), l, h, d, l, h * d)[:, :l], (q * scale).transpose(1, 0, 2))


# ---- FlowEulerSampler: samplers/flow_euler.mojo ----------------------------------
def test_flow_elementwise_exact_f32():
    """_v_to_xstart, the CFG combine and the Euler update are sequences of
    single f32 roundings: numpy's IEEE float32 ufuncs give the same bits.
    Dropping the (1 - sigma_min) factor of c (a plausible slip) changes them."""
    x, v, w = orc.randn(1600, (5000,)), orc.randn(1601, (5000,)), orc.randn(1602, (5000,))
    t, tp, sm, g = 0.7371, 0.6012, 1e-5, 3.0
    a = np.float32(1.0 - sm)
    c = np.float32(sm + (1.0 - sm) * t)
    assert np.array_equal(orc.flow_v_to_xstart(x, v, t, sm), x * a - v * c)
    c_mut = np.float32(sm + t)
    assert c_mut != c and not np.array_equal(orc.flow_v_to_xstart(x, v, t, sm), x * a - v * c_mut)
    assert np.array_equal(orc.flow_cfg(v, w, g), v * np.float32(g) + w * np.float32(1.0 - g))
    assert np.array_equal(orc.flow_step(x, v, t, tp), x - v * np.float32(t - tp))


def _rescale_case(seed, rows, rs):
    x = orc.randn(seed, (rows, rs))
    pos = orc.randn(seed + 1, (rows, rs))
    neg = orc.randn(seed + 2, (rows, rs), std=0.5)
    return x, pos, neg


@pytest.mark.parametrize("varlen", [False, True])
def test_flow_rescale_float64_properties(varlen):
    """With guidance_rescale 1 the rescaled x_0 of every segment has the
    positive branch's std (checked in float64 on x_0 = a*x - cc*out); with 0
    the output is the CFG prediction itself. Segments: one per row (dense)
    or token offsets (varlen); a dense reading of a varlen state fails the
    per-segment check."""
    rows, rs, t, sm = 6, 40, 0.63, 1e-5
    x, pos, neg = _rescale_case(1700, rows, rs)
    pred = orc.flow_cfg(pos, neg, 3.0)
    segs = np.array([0, 2, 6], np.int64) if varlen else None
    bounds = [(0, 2), (2, 6)] if varlen else [(r, r + 1) for r in range(rows)]
    a = 1.0 - sm
    cc = float(np.float32(sm + (1.0 - sm) * t))
    out = orc.flow_rescale(x, pred, pos, t, sm, 1.0, segs)
    x0 = a * x.astype(np.float64) - cc * out.astype(np.float64)
    x0p = a * x.astype(np.float64) - cc * pos.astype(np.float64)
    for lo, hi in bounds:
        assert abs(x0[lo:hi].std() / x0p[lo:hi].std() - 1) < 2e-5
    if varlen:   # the dense (per-row) reading does not satisfy the segment property
        dense = orc.flow_rescale(x, pred, pos, t, sm, 1.0, None)
        x0d = a * x.astype(np.float64) - cc * dense.astype(np.float64)
        assert abs(x0d[2:6].std() / x0p[2:6].std() - 1) > 1e-3
    out0 = orc.flow_rescale(x, pred, pos, t, sm, 0.0, segs)
    assert np.max(np.abs(out0 - pred)) < 2e-5 / cc


def test_flow_rescale_uncovered_and_empty_segments():
    """Rows outside the token segments keep a zero prediction; an empty
    segment is skipped (flow_euler.mojo:100-112)."""
    x, pos, neg = _rescale_case(1800, 8, 16)
    pred = orc.flow_cfg(pos, neg, 2.0)
    out = orc.flow_rescale(x, pred, pos, 0.5, 1e-5, 0.7, np.array([2, 2, 5], np.int64))
    assert not out[:2].any() and not out[5:].any() and out[2:5].all()


def test_flow_schedule_and_sampler_float64():
    """t_seq = rescale_t*t/(1+(rescale_t-1)*t) over linspace(1, 0) (1.0 and 0.0
    at the ends; rescale_t 1 is the plain linspace). With v = -x (no
    guidance) the sampler is explicit Euler for dx/dt = -x backwards in t:
    x_{i+1} = x_i * (1 + (t_i - t_{i+1})), checked in float64."""
    ts = orc.flow_t_seq(12, 3.0)
    assert ts[0] == 1.0 and ts[-1] == 0.0 and all(a > b for a, b in zip(ts, ts[1:]))
    assert orc.flow_t_seq(4, 1.0) == [1.0, 0.75, 0.5, 0.25, 0.0]
    x = orc.randn(1900, (3, 7))
    model = lambda xt, t1000, neg: (-xt).astype(np.float32)
    out, xs, x0s = orc.flow_sample(model, x, 12, 3.0, 1e-5)
    want = x.astype(np.float64)
    for a, b in zip(ts, ts[1:]):
        want = want * (1.0 + (a - b))
    assert np.max(np.abs(out - want) / np.abs(want)) < 1e-5 and len(xs) == 12 and len(x0s) == 12


class _StubModel:
    """A velocity model that returns a distinct constant for each branch
    (2 for the positive condition, -3 for the negative one) and records its
    calls as (t1000, use_neg)."""

    def __init__(self):
        self.calls = []

    def __call__(self, x_t, t1000, use_neg):
        self.calls.append((t1000, use_neg))
        return np.full_like(x_t, -3.0 if use_neg else 2.0)


def _infer(mode, g, t, lo=0.3, hi=0.6, gr=0.0):
    m = _StubModel()
    x = orc.randn(2100, (4, 16))
    out = orc.flow_inference(m, x, t, mode, g, lo, hi, gr, 1e-5, None)
    return out, m.calls, x


def test_flow_inference_branches():
    """_inference (samplers/flow_euler.mojo:151-181) with a stub model:
    - no guidance, g == 1 and g == 0 each make one call and return that
      branch unchanged, also with guidance_rescale > 0 (rescale is skipped);
    - CFG returns fl(g*pos) + fl((1-g)*neg) from pos then neg;
    - CFG_INTERVAL applies CFG on the closed interval [lo, hi] (t exactly
      on lo and on hi included) and the positive branch outside it, while
      plain CFG ignores the interval;
    - guidance_rescale > 0 routes the CFG prediction through _rescale_pred;
    - the model sees t * 1000 in float64."""
    pos = np.float32(2.0)
    neg = np.float32(-3.0)
    out, calls, _ = _infer(orc.GUIDANCE_NONE, 3.0, 0.45)
    assert calls == [(1000.0 * 0.45, False)] and np.all(out == pos)
    out, calls, _ = _infer(orc.GUIDANCE_CFG, 1.0, 0.45, gr=0.7)
    assert calls == [(1000.0 * 0.45, False)] and np.all(out == pos)
    out, calls, _ = _infer(orc.GUIDANCE_CFG, 0.0, 0.45, gr=0.7)
    assert calls == [(1000.0 * 0.45, True)] and np.all(out == neg)
    g = 3.0
    cfg = pos * np.float32(g) + neg * np.float32(1.0 - g)
    assert cfg == np.float32(12.0)
    out, calls, _ = _infer(orc.GUIDANCE_CFG, g, 0.9)              # outside [lo, hi]: plain CFG ignores it
    assert [c[1] for c in calls] == [False, True] and np.all(out == cfg)
    for t in (0.3, 0.45, 0.6):                                     # inclusive ends
        out, calls, _ = _infer(orc.GUIDANCE_CFG_INTERVAL, g, t)
        assert [c[1] for c in calls] == [False, True] and np.all(out == cfg), t
    for t in (0.29999, 0.60001, 1.0):
        out, calls, _ = _infer(orc.GUIDANCE_CFG_INTERVAL, g, t)
        assert calls == [(1000.0 * t, False)] and np.all(out == pos), t
    out, calls, x = _infer(orc.GUIDANCE_CFG_INTERVAL, g, 0.6, gr=0.7)
    assert len(calls) == 2
    assert not np.array_equal(out, np.full_like(x, cfg))
    assert np.array_equal(out, orc.flow_rescale(x, np.full_like(x, cfg), np.full_like(x, pos), 0.6, 1e-5, 0.7))


# ---- weight GEMM: gpu/linear.mojo:108-160, 326-388 ---------------------------
def test_linear_integer_operands_exact():
    """Small-integer operands: every product and partial sum is an integer
    below 2^24, so the f32 GEMM is exact in any order and equals numpy's
    integer matmul. A transposed weight (w [n, k] read as [k, n]) or a dropped
    k term fails."""
    rng = np.random.default_rng(5)
    m, n, k = 37, 24, 40
    a = rng.integers(-8, 9, (m, k)).astype(np.float32)
    w = rng.integers(-8, 9, (n, k)).astype(np.float32)
    want = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    got = orc.linear(a, w, nthreads=3)
    assert np.array_equal(got, want)
    assert not np.array_equal(got, (a[:, :-1].astype(np.int64) @ w[:, :-1].astype(np.int64).T).astype(np.float32))
    sq = rng.integers(-8, 9, (k, k)).astype(np.float32)
    assert not np.array_equal(orc.linear(a, sq), (a @ sq).astype(np.float32))


def test_linear_sums_k_in_order():
    """Products 2^24, 1, -2^24 summed in k order: fl(fl(2^24 + 1) - 2^24) = 0,
    while the reverse order gives fl(fl(-2^24 + 1) + 2^24) = 1 (2^24 - 1 is
    representable). Pins the reference's serial per-thread accumulation."""
    a = np.array([[1.0, 1.0, 1.0]], np.float32)
    w = np.array([[2.0 ** 24, 1.0, -(2.0 ** 24)], [-(2.0 ** 24), 1.0, 2.0 ** 24]], np.float32)
    got = orc.linear(a, w)
    assert got[0, 0] == 0.0 and got[0, 1] == 1.0


def test_linear_float64_bound_bias_and_activation():
    """f16-valued operands at the DiT's scale: each output is within the
    serial-sum bound k * 2^-24 * sum|a w| of the float64 product (the
    products are exact). Bias and GELU-tanh compose as add_bias then
    activation (act(fl(acc + b)))."""
    m, n, k = 64, 48, 512
    a = orc.round_f16(orc.randn(880, (m, k)))
    w = orc.round_f16(orc.randn(881, (n, k), std=0.02))
    b = orc.randn(882, (n,), std=0.02)
    got = orc.linear(a, w)
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    bound = k * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got - exact) <= bound)
    assert np.max(np.abs(got - exact)) > 0.0      # f32 sums do round
    full = orc.linear(a, w, bias=b, act=orc.ACT_GELU_TANH)
    assert np.array_equal(full, orc.activation(orc.add_bias(got, b), orc.ACT_GELU_TANH))


# ---- compositions the GPU tests check against -------------------------------
def test_compositions_float64_and_order():
    """The oracle's compositions follow the reference's op order, checked in
    float64 against closed forms of the same order; each plausible reordering
    (RoPE before RMS with a non-uniform gamma, the bias after RMS, GELU of x
    then + bias, modulate before LN) fails the same check.
    - qk_rms_rope: bias -> MultiHeadRMSNorm -> RoPE (sparse/attention/
      modules.mojo:206-212; gpu/attention.mojo:507-563);
    - ln_modulate: LN then x*(1+scale)+shift (modules/nn.mojo:660-689);
    - gelu_tanh_bias: GELU-tanh(x + bias) (gpu/linear.mojo:662-684);
    - attn_pack: the epilogue, then pack_q_z / pack_kv_z (987-1013)."""
    n, h, d = 24, 4, 64
    q = orc.randn(2200, (n, h, d), std=2.0)
    k = orc.randn(2201, (n, h, d), std=2.0)
    g = orc.randn(2202, (h, d), mean=1.0, std=0.3)       # non-uniform: RMS and RoPE do not commute
    bq = orc.randn(2203, (h, d), std=0.5)
    co = np.zeros((n, 4), np.int32)
    co[:, 1:] = np.random.default_rng(3).integers(0, 40, (n, 3))
    ph = orc.rope_phases_from_coords(co, d, orc.rope_freqs(d))
    ph64 = ph.astype(np.float64)[:, None]

    def rms64(x, gam):
        x = x.astype(np.float64)
        return x / np.maximum(np.linalg.norm(x, axis=-1, keepdims=True), 1e-12) * gam * math.sqrt(d)

    want = _rotate64(rms64(q + bq, g).astype(np.float32), ph64)
    got_q, _ = orc.qk_rms_rope(q, k, g, g, ph, bias_q=bq)
    assert _rel(got_q, want) < 5e-6
    assert _rel(rms64(_rotate64(q + bq, ph64), g), want) > 1e-3            # RoPE before RMS
    assert _rel(_rotate64(rms64(q, g) + bq, ph64), want) > 1e-3            # bias after RMS

    x = orc.randn(2204, (16, 96), mean=0.3, std=1.7)
    sh, sc = orc.randn(2205, (96,), std=0.3), orc.randn(2206, (96,), std=0.3)
    ln = _ln64(x, 1e-6)
    want = ln * (1.0 + sc.astype(np.float64)) + sh
    assert _rel(orc.ln_modulate(x, sh, sc, eps=1e-6), want) < 2e-6
    assert _rel(_ln64((x * (1.0 + sc) + sh).astype(np.float32), 1e-6), want) > 1e-3   # modulate first

    u = orc.randn(2207, (8, 300), std=2.0)
    b = orc.randn(2208, (300,), std=0.5)
    gelu64 = lambda v: 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    want = gelu64(u.astype(np.float64) + b)
    assert _rel(orc.gelu_tanh_bias(u, b), want) < 2e-6
    assert _rel(gelu64(u.astype(np.float64)) + b, want) > 1e-3                       # bias after GELU

    qkv = orc.randn(2209, (n, 3, h, d))
    bias = orc.randn(2210, (3, h, d), std=0.5)
    qh, kt, vh = orc.attn_pack(qkv, h, d, 32, 32, bias.reshape(-1), g, g, ph)
    eq, ek = orc.qk_rms_rope(qkv[:, 0], qkv[:, 1], g, g, ph, bias_q=bias[0], bias_k=bias[1])
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    assert np.array_equal(qh[:, :n], (eq * scale).astype(np.float32).transpose(1, 0, 2))
    assert np.array_equal(kt[:, :, :n], ek.transpose(1, 2, 0))
    assert np.array_equal(vh[:, :n], (qkv[:, 2] + bias[2]).astype(np.float32).transpose(1, 0, 2))
    assert not qh[:, n:].any() and not kt[:, :, n:].any() and not vh[:, n:].any()
