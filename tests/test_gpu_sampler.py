"""GPU parity: the flow-matching Euler sampler step (t2h_flow_euler_step) and
the sampler loop built on it (t2h.sampler.FlowEulerSampler), through the C
ABI, against the C oracle's restatement of samplers/flow_euler.mojo.

Bars: the CFG combine, the Euler update and pred_x0 are single f32 roundings
and are compared bit for bit. The CFG rescale's std is summed in f64 on the
device and serially in f32 by the reference, so the rescaled prediction is
compared to tolerance; the step divides by cc = f32(sigma_min + (1 -
sigma_min) t), so the bar is 1e-5 / cc (f32 storage; t >= 0.5 keeps it within
2e-5). Metric: tests/_parity.py."""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, host, max_err, storage_round, to_dev
from t2h import ops, sampler, workloads
from t2h._lib import T2HError

pytestmark = pytest.mark.gpu
SM = 1e-5


def _case(seed, shape, dtype=torch.float32):
    x = storage_round(orc.randn(seed, shape), dtype)
    pos = storage_round(orc.randn(seed + 1, shape), dtype)
    neg = storage_round(orc.randn(seed + 2, shape, std=0.5), dtype)
    return x, pos, neg


def _bits(got, want, dtype):
    w = torch.from_numpy(np.ascontiguousarray(storage_round(want, dtype))).to(dtype)
    return torch.equal(got.cpu(), w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_step_no_guidance_and_cfg_bit_exact(dev, dtype):
    """ss-flow latent shape [2, 8, 16, 16, 16]: Euler step alone and with the
    CFG combine (g = 3): x_prev and pred_x0 bit-exact."""
    shape = (2, 8, 16, 16, 16)
    x, pos, neg = _case(3000, shape, dtype)
    t, tp = 0.8123, 0.7311
    xp, x0 = ops.flow_euler_step(to_dev(x, dev, dtype), to_dev(pos, dev, dtype), t, tp, SM)
    assert _bits(xp, orc.flow_step(x, pos, t, tp), dtype)
    assert _bits(x0, orc.flow_v_to_xstart(x, pos, t, SM), dtype)
    xp, x0 = ops.flow_euler_step(to_dev(x, dev, dtype), to_dev(pos, dev, dtype), t, tp, SM,
                                 v_neg=to_dev(neg, dev, dtype), guidance_strength=3.0)
    pred = orc.flow_cfg(pos, neg, 3.0)
    assert _bits(xp, orc.flow_step(x, pred, t, tp), dtype)
    assert _bits(x0, orc.flow_v_to_xstart(x, pred, t, SM), dtype)


def test_step_guidance_strength_edges(dev):
    """g = 1 uses the positive prediction alone, g = 0 the negative alone,
    and neither is rescaled (flow_euler.mojo:167-170)."""
    x, pos, neg = _case(3100, (4, 300))
    for g, v in ((1.0, pos), (0.0, neg)):
        xp, _ = ops.flow_euler_step(to_dev(x, dev), to_dev(pos, dev), 0.9, 0.8, SM, v_neg=to_dev(neg, dev),
                                    guidance_strength=g, guidance_rescale=0.7)
        assert _bits(xp, orc.flow_step(x, v, 0.9, 0.8), torch.float32)


@pytest.mark.parametrize("t", [0.9, 0.55])
def test_step_rescale_dense(dev, t):
    """Dense state [2, 8, 16, 16, 16], guidance_rescale 0.7 (the ss stage of
    pipeline.json): one std per row, unbiased."""
    shape = (2, 8, 16, 16, 16)
    x, pos, neg = _case(3200, shape)
    tp = t - 0.07
    pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, 7.5), pos, t, SM, 0.7)
    xp, x0 = ops.flow_euler_step(to_dev(x, dev), to_dev(pos, dev), t, tp, SM, v_neg=to_dev(neg, dev),
                                 guidance_strength=7.5, guidance_rescale=0.7)
    cc = float(np.float32(SM + (1 - SM) * t))
    assert max_err(x0, orc.flow_v_to_xstart(x, pred, t, SM)) <= 1e-5
    assert max_err(xp, orc.flow_step(x, pred, t, tp)) <= 1e-5 / cc


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_step_rescale_varlen_config4(dev, dtype):
    """Varlen state: config-4 token rows (T = 39,804, two batches) x 32
    latent channels, per-segment biased std (the shape stage, rescale 0.5).
    bf16 storage runs the 16-bit vector statistics path with bf16 unpacking
    (bar 8e-3 / cc: bf16 keeps 8 significant bits)."""
    _, offsets = workloads.config4()
    shape = (int(offsets[-1]), 32)
    x, pos, neg = _case(3300, shape, dtype)
    t, tp = 0.74, 0.66
    pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, 5.0), pos, t, SM, 0.5, offsets)
    xp, x0 = ops.flow_euler_step(to_dev(x, dev, dtype), to_dev(pos, dev, dtype), t, tp, SM,
                                 v_neg=to_dev(neg, dev, dtype), guidance_strength=5.0, guidance_rescale=0.5,
                                 seg_offsets=offsets)
    tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 8e-3}[dtype]
    cc = float(np.float32(SM + (1 - SM) * t))
    assert max_err(xp, storage_round(orc.flow_step(x, pred, t, tp), dtype)) <= tol / cc
    assert max_err(x0, storage_round(orc.flow_v_to_xstart(x, pred, t, SM), dtype)) <= tol / cc


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shift", [0, 1])
def test_step_rescale_varlen_unaligned(dev, dtype, shift):
    """Varlen rescale on the scalar path: shape (300, 3) with segments
    [0, 121, 300], whose element bounds (363, 900) are not whole 16-byte
    vectors, and the same state one element into its buffers (no 16-byte
    alignment at all): the per-segment statistics blocks and the
    elementwise pass then run their scalar loops."""
    shape = (300, 3)
    segs = np.array([0, 121, 300], np.int64)
    x, pos, neg = _case(3800, shape, dtype)
    t, tp = 0.77, 0.69
    pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, 4.0), pos, t, SM, 0.6, segs)
    bufs = []
    for a in (x, pos, neg):
        b = torch.zeros(a.size + shift, dtype=dtype, device=dev)
        b[shift:] = to_dev(a.reshape(-1), dev, dtype)
        bufs.append(b[shift:].reshape(shape))
    xp, x0 = ops.flow_euler_step(bufs[0], bufs[1], t, tp, SM, v_neg=bufs[2], guidance_strength=4.0,
                                 guidance_rescale=0.6, seg_offsets=segs)
    tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 8e-3}[dtype]
    cc = float(np.float32(SM + (1 - SM) * t))
    assert max_err(xp, storage_round(orc.flow_step(x, pred, t, tp), dtype)) <= tol / cc
    assert max_err(x0, storage_round(orc.flow_v_to_xstart(x, pred, t, SM), dtype)) <= tol / cc


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_step_rescale_config5_latent(dev, dtype):
    """The config-5 token rows (T = 201,436) x 32 latent channels as one
    varlen segment (6.4M elements: the statistics pass caps a segment at 256
    blocks, so each block takes a share of ~25K elements in two load
    groups), and the same
    state split into three segments of unequal sizes; two calls give the
    same bits (fixed-order sums).

    Bars. The reference sums the std serially in f32; over a 6.4M-element
    segment that sum is itself off from the exact value: on this case the
    oracle's x_prev differs by 2.4e-5 from the same step with a float64
    ratio. The device sums in f64, so against the oracle the f32 bar here is
    3e-5 / cc (f16: 2e-3 / cc). The defining property is checked tightly in
    float64 on the device output: with guidance_rescale 1, each segment's
    x_0 = a*x - cc*x_prev-derived prediction has the positive branch's std
    (relative 2e-6 for f32 storage)."""
    coords, offsets = workloads.config5()
    T = int(offsets[-1])
    shape = (T, 32)
    x, pos, neg = _case(3700, shape, dtype)
    t, tp = 0.81, 0.72
    cc = float(np.float32(SM + (1 - SM) * t))
    tol = 3e-5 if dtype == torch.float32 else 2e-3
    dx, dp, dn = (to_dev(a, dev, dtype) for a in (x, pos, neg))
    for segs in (np.array([0, T], np.int64), np.array([0, 1000, 150001, T], np.int64)):
        pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, 3.0), pos, t, SM, 0.5, segs)
        outs = [ops.flow_euler_step(dx, dp, t, tp, SM, v_neg=dn, guidance_strength=3.0, guidance_rescale=0.5,
                                    seg_offsets=segs) for _ in range(2)]
        xp, x0 = outs[0]
        assert torch.equal(xp, outs[1][0]) and torch.equal(x0, outs[1][1])
        assert max_err(xp, storage_round(orc.flow_step(x, pred, t, tp), dtype)) <= tol / cc
        assert max_err(x0, storage_round(orc.flow_v_to_xstart(x, pred, t, SM), dtype)) <= tol / cc
    if dtype == torch.float32:
        segs = np.array([0, 1000, 150001, T], np.int64)
        _, x0 = ops.flow_euler_step(dx, dp, t, tp, SM, v_neg=dn, guidance_strength=3.0, guidance_rescale=1.0,
                                    seg_offsets=segs)
        x0d = host(x0).astype(np.float64)
        x0p = np.float32(1 - SM) * x - np.float32(cc) * pos
        for lo, hi in zip(segs[:-1], segs[1:]):
            assert abs(x0d[lo:hi].std() / x0p[lo:hi].astype(np.float64).std() - 1) < 2e-6


# the workspace of the one-launch rescale: the barrier words (a 64-bit error
# word in the first 64 bytes, 8 release slots of 128 bytes each starting with
# a 64-bit epoch and a 64-bit release word (the epoch's low half and the
# ratio), then per block, for up to 2048 blocks, a 64-bit arrival
# flag, leave mark and claim word), then one f64 quad per block
FUSE_BYTES = 64 + 8 * 128 + 3 * 2048 * 8 + 2048 * 32


def _step(x, p, n, t, tp, g, gr, segs, ws):
    return ops.flow_euler_step(x, p, t, tp, SM, v_neg=n, guidance_strength=g, guidance_rescale=gr,
                               seg_offsets=segs, workspace=ws)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,segs", [
    ((201436, 32), [0, 201436]),      # the config-5 latent: one segment, 4 vectors per thread (f32)
    ((4097, 32), [0, 4097]),          # a last block with 8 of its vectors
    ((4097, 32), [5, 3000]),          # one segment with uncovered rows on both sides
    ((3, 8), [0, 3]),                 # 24 elements: one partial block
    ((1, 8 * 16 ** 3), None),         # a dense state of one row: unbiased std
])
def test_step_rescale_one_launch(dev, dtype, shape, segs):
    """A single segment on whole 16-byte vectors takes the one-launch form
    (inputs held in registers across a grid barrier). Against the oracle to
    the sampler bars, and against the two-launch form (a workspace without
    room for the barrier) to 2 ulp of the storage type: both sum the std in
    f64, in different orders."""
    rows = shape[0]
    assert ops.flow_euler_workspace(rows, shape[1], 0 if segs is None else len(segs)) == FUSE_BYTES
    x, pos, neg = _case(3900 + rows, shape, dtype)
    t, tp, g, gr = 0.8, 0.72, 3.0, 0.6
    so = None if segs is None else np.array(segs, np.int64)
    pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, g), pos, t, SM, gr, so)
    dx, dp, dn = (to_dev(a, dev, dtype) for a in (x, pos, neg))
    one = _step(dx, dp, dn, t, tp, g, gr, segs, torch.empty(FUSE_BYTES, dtype=torch.uint8, device=dev))
    two = _step(dx, dp, dn, t, tp, g, gr, segs, torch.empty(FUSE_BYTES - 16, dtype=torch.uint8, device=dev))
    cc = float(np.float32(SM + (1 - SM) * t))
    tol = {torch.float32: 3e-5, torch.float16: 2e-3, torch.bfloat16: 8e-3}[dtype]
    assert max_err(one[0], storage_round(orc.flow_step(x, pred, t, tp), dtype)) <= tol / cc
    assert max_err(one[1], storage_round(orc.flow_v_to_xstart(x, pred, t, SM), dtype)) <= tol / cc
    ulp = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[dtype]
    for a, b in zip(one, two):
        d = (a.float() - b.float()).abs() / b.float().abs().clamp(min=1.0)
        assert d.max().item() <= 2 * ulp / cc, (shape, segs, d.max().item())
    if segs is not None and segs[0] > 0:   # uncovered rows: x_prev = x exactly
        assert torch.equal(one[0][:segs[0]], dx[:segs[0]]) and torch.equal(one[0][segs[1]:], dx[segs[1]:])


def test_step_rescale_one_launch_repeats_on_a_dirty_workspace(dev):
    """The barrier words need no set-up by the caller: on a workspace filled
    with 0xFF bytes, three calls in a row give the same bits; each advances
    every release slot's epoch by one and leaves the error word unequal to
    it (a block that stopped waiting writes the new epoch there)."""
    T = 201436
    x, pos, neg = (to_dev(a, dev) for a in _case(4100, (T, 32)))
    ws = torch.full((FUSE_BYTES,), 255, dtype=torch.uint8, device=dev)
    outs = []
    for call in range(3):
        outs.append(_step(x, pos, neg, 0.8, 0.72, 3.0, 0.6, [0, T], ws))
        words = ws[:64 + 8 * 128].view(torch.int64).cpu()
        epochs = [int(words[8 + 16 * k]) for k in range(8)]
        assert epochs == [call] * 8, epochs        # 0xFF..FF + 1 wraps to 0
        assert int(words[0]) != epochs[0], "error word"
    for o in outs[1:]:
        assert torch.equal(o[0], outs[0][0]) and torch.equal(o[1], outs[0][1])


@pytest.mark.parametrize("polls", ["0", "1"])
def test_step_rescale_one_launch_blocks_that_leave(dev, polls, monkeypatch):
    """A data block that waits too long for the ratio (its grid not resident
    at once) leaves its vectors to the reducing block. Forced from the host
    with T2H_FUSE_WAIT_POLLS = 0 or 1 (every block, or nearly every, leaves):
    the same bits as the normal launch, also with x_prev aliasing x_t (a
    left vector is stored once, by one of the two), and the error word
    stays unequal to the new epoch."""
    T = 201436
    x, pos, neg = (to_dev(a, dev) for a in _case(4300, (T, 32)))
    ws = torch.empty(FUSE_BYTES, dtype=torch.uint8, device=dev)
    want = _step(x, pos, neg, 0.8, 0.72, 3.0, 0.6, [0, T], ws)
    monkeypatch.setenv("T2H_FUSE_WAIT_POLLS", polls)
    for _ in range(2):
        got = _step(x, pos, neg, 0.8, 0.72, 3.0, 0.6, [0, T], ws)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        words = ws[:64 + 8 * 128].view(torch.int64).cpu()
        assert int(words[0]) != int(words[8]), "error word"
    xi = x.clone()
    _, x0 = ops.flow_euler_step(xi, pos, 0.8, 0.72, SM, v_neg=neg, guidance_strength=3.0, guidance_rescale=0.6,
                                seg_offsets=[0, T], workspace=ws, x_prev=xi)
    assert torch.equal(xi, want[0]) and torch.equal(x0, want[1])


def test_step_rescale_one_launch_in_a_hip_graph(dev):
    """The one-launch step (its barrier reset and its grid) recorded into a
    HIP graph: three replays with fresh inputs, eager steps on the same
    workspace in between, each replay equal to an eager step bit for bit."""
    T = 201436
    x, pos, neg = (to_dev(a, dev) for a in _case(4200, (T, 32)))
    ws = torch.empty(FUSE_BYTES, dtype=torch.uint8, device=dev)
    xp, x0 = torch.empty_like(x), torch.empty_like(x)

    def step():
        return ops.flow_euler_step(x, pos, 0.8, 0.72, SM, v_neg=neg, guidance_strength=3.0, guidance_rescale=0.6,
                                   seg_offsets=[0, T], workspace=ws, x_prev=xp)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _, gx0 = step()
    g = torch.Generator(device=dev).manual_seed(4201)
    for rep in range(3):
        for a in (x, pos, neg):
            a.copy_(torch.randn(a.shape, generator=g, device=dev))
        graph.replay()
        got = (xp.clone(), gx0.clone())
        want = _step(x, pos, neg, 0.8, 0.72, 3.0, 0.6, [0, T], ws)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), f"replay {rep}"


def test_step_odd_rows_and_unaligned_state(dev):
    """Rows of 12,289 elements (one statistics block per row, one per
    16,384 elements started; six 2,048-element elementwise blocks and a
    1-element tail block per row; rows starting at odd element offsets, so
    the scalar path runs), and
    the same state viewed one element into its buffer (no 16-byte
    alignment): the oracle's bits without rescale and its tolerance with it."""
    shape = (3, 12289)
    x, pos, neg = _case(3400, shape)
    t, tp = 0.83, 0.77
    pred = orc.flow_cfg(pos, neg, 4.0)
    want = orc.flow_rescale(x, pred, pos, t, SM, 0.6)
    cc = float(np.float32(SM + (1 - SM) * t))
    for off in (0, 1):
        bufs = []
        for a in (x, pos, neg):
            b = torch.zeros(a.size + off, dtype=torch.float32, device=dev)
            b[off:] = to_dev(a.reshape(-1), dev)
            bufs.append(b[off:].reshape(shape))
        xp, x0 = ops.flow_euler_step(bufs[0], bufs[1], t, tp, SM, v_neg=bufs[2], guidance_strength=4.0)
        assert _bits(xp, orc.flow_step(x, pred, t, tp), torch.float32)
        assert _bits(x0, orc.flow_v_to_xstart(x, pred, t, SM), torch.float32)
        xp, x0 = ops.flow_euler_step(bufs[0], bufs[1], t, tp, SM, v_neg=bufs[2], guidance_strength=4.0,
                                     guidance_rescale=0.6)
        assert max_err(x0, orc.flow_v_to_xstart(x, want, t, SM)) <= 1e-5
        assert max_err(xp, orc.flow_step(x, want, t, tp)) <= 1e-5 / cc


def test_step_rescale_uncovered_rows_and_workspace_reuse(dev):
    """Rows outside the token segments keep a zero prediction (x_prev = x,
    pred_x0 = x * a, bit-exact); one workspace serves consecutive calls."""
    x, pos, neg = _case(3400, (50, 24))
    segs = np.array([5, 5, 30, 41], np.int64)
    ws = torch.empty(ops.flow_euler_workspace(50, 24, 4), dtype=torch.uint8, device=dev)
    for t in (0.95, 0.6):
        pred = orc.flow_rescale(x, orc.flow_cfg(pos, neg, 3.0), pos, t, SM, 0.7, segs)
        xp, x0 = ops.flow_euler_step(to_dev(x, dev), to_dev(pos, dev), t, t - 0.1, SM, v_neg=to_dev(neg, dev),
                                     guidance_strength=3.0, guidance_rescale=0.7, seg_offsets=segs, workspace=ws)
        want = orc.flow_step(x, pred, t, t - 0.1)
        assert np.array_equal(host(xp)[:5], x[:5]) and np.array_equal(host(xp)[41:], x[41:])
        assert np.array_equal(host(x0)[:5], x[:5] * np.float32(1 - SM))
        assert max_err(xp, want) <= 2e-5


def test_sampler_loop_bit_exact_without_rescale(dev):
    """FlowEulerSampler.sample_cfg_interval with a model whose predictions
    are exact in f32 on both sides (v = x/2, negative branch -x/4): the whole
    12-step trajectory matches the oracle's sampler bit for bit, including the
    guidance interval switching CFG on and off."""
    noise = orc.randn(3500, (2, 8, 4, 4, 4))
    dmodel = lambda xt, t1000, neg: xt * (-0.25 if neg else 0.5)
    omodel = lambda xt, t1000, neg: (xt * np.float32(-0.25 if neg else 0.5)).astype(np.float32)
    s = sampler.FlowEulerSampler(SM)
    res = s.sample_cfg_interval(dmodel, to_dev(noise, dev), steps=12, rescale_t=3.0, guidance_strength=3.0,
                                interval_lo=0.6, interval_hi=0.9)
    want, xs, x0s = orc.flow_sample(omodel, noise, 12, 3.0, SM, orc.GUIDANCE_CFG_INTERVAL, 3.0, 0.6, 0.9)
    assert np.array_equal(host(res.samples), want)
    assert all(np.array_equal(host(a), b) for a, b in zip(res.pred_x_t, xs))
    assert all(np.array_equal(host(a), b) for a, b in zip(res.pred_x_0, x0s))


def test_sampler_loop_with_rescale(dev):
    """The same loop with guidance_rescale 0.7 on a varlen state: per-step
    errors of the rescale (f64 vs serial f32 std) stay at the 1e-5 level
    across 6 steps."""
    noise = orc.randn(3600, (300, 16))
    segs = [0, 120, 300]
    dmodel = lambda xt, t1000, neg: xt * (-0.25 if neg else 0.5)
    omodel = lambda xt, t1000, neg: (xt * np.float32(-0.25 if neg else 0.5)).astype(np.float32)
    res = sampler.FlowEulerSampler(SM).sample_cfg(dmodel, to_dev(noise, dev), steps=6, rescale_t=3.0,
                                                  guidance_strength=3.0, guidance_rescale=0.7, seg_offsets=segs)
    want, _, _ = orc.flow_sample(omodel, noise, 6, 3.0, SM, orc.GUIDANCE_CFG, 3.0, 0.0, 1.0, 0.7,
                                 np.array(segs, np.int64))
    assert max_err(res.samples, want) <= 1e-4


def test_step_errors(dev):
    x = torch.zeros((4, 8), device=dev)
    with pytest.raises(ValueError, match="workspace"):
        ops.flow_euler_step(x, x, 0.5, 0.4, SM, v_neg=x, guidance_strength=3.0, guidance_rescale=0.5,
                            workspace=torch.empty(8, dtype=torch.uint8, device=dev))
    with pytest.raises(ValueError, match="ordered"):
        ops.flow_euler_step(x, x, 0.5, 0.4, SM, v_neg=x, guidance_strength=3.0, guidance_rescale=0.5,
                            seg_offsets=[0, 3, 2])
    x1 = x.reshape(-1, 1)   # 32 rows
    with pytest.raises(T2HError, match="more than 64 segments"):
        ops.flow_euler_step(x1, x1, 0.5, 0.4, SM, v_neg=x1, guidance_strength=3.0, guidance_rescale=0.5,
                            seg_offsets=list(range(32)) + [32] * 34)
    with pytest.raises(ValueError, match="size mismatch"):
        ops.flow_euler_step(x, x[:2], 0.5, 0.4, SM)
