"""GPU: t2h_flow_euler_step_noalloc (the sampler step for callers that cannot
allocate device memory) through the C ABI, against t2h_flow_euler_step with
a caller workspace on the same inputs. Both run the same kernels and sum the
statistics in the same fixed order, so the results must agree bit for bit.
Two no-allocation calls in a row, the second on a smaller state, show that
the shared built-in scratch carries nothing from one call to the next."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
from _parity import max_err, to_dev
from t2h import _lib, ops, workloads

pytestmark = pytest.mark.gpu
SM = 1e-5


def _noalloc(x, vp, vn, t, tp, g, gr, segs):
    """One t2h_flow_euler_step_noalloc call; returns (x_prev, pred_x0)."""
    xp, x0 = torch.empty_like(x), torch.empty_like(x)
    so = None if segs is None else np.ascontiguousarray(np.asarray(segs, np.int64))
    rows = x.shape[0]
    rc = _lib.load().t2h_flow_euler_step_noalloc(
        x.data_ptr(), vp.data_ptr(), vn.data_ptr() if vn is not None else None, xp.data_ptr(), x0.data_ptr(), rows,
        x.numel() // rows, _lib.F32 if x.dtype == torch.float32 else _lib.F16, t, tp, SM, g, gr,
        so.ctypes.data if so is not None else None, 0 if so is None else so.size, ops._stream())
    _lib.check(rc)
    return xp, x0


def _state(seed, shape, dev):
    return [to_dev(orc.randn(seed + i, shape, std=0.5 if i == 2 else 1.0), dev) for i in range(3)]


def test_noalloc_equals_workspace_entry_point(dev):
    _, off5 = workloads.config5()
    _, off4 = workloads.config4()
    cases = [
        # (state, seg_offsets): config-5 latent as one segment, then the smaller
        # config-4 latent as two, then a dense state (one segment per row)
        (_state(4000, (int(off5[-1]), 32), dev), [0, int(off5[-1])]),
        (_state(4010, (int(off4[-1]), 32), dev), off4.tolist()),
        (_state(4020, (2, 8 * 16 ** 3), dev), None),
    ]
    for (x, vp, vn), segs in cases:
        for t, tp, g, gr in ((0.8, 0.7, 3.0, 0.5), (0.55, 0.45, 7.5, 0.7), (0.9, 0.8, 3.0, 0.0)):
            got = _noalloc(x, vp, vn, t, tp, g, gr, segs)
            want = ops.flow_euler_step(x, vp, t, tp, SM, v_neg=vn, guidance_strength=g, guidance_rescale=gr,
                                       seg_offsets=segs)
            assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), (x.shape, segs, t, gr)
    # and the oracle, on the last (smaller) varlen case, to the sampler tests' bar
    x, vp, vn = cases[1][0]
    segs = cases[1][1]
    xh, ph, nh = (a.cpu().numpy() for a in (x, vp, vn))
    pred = orc.flow_rescale(xh, orc.flow_cfg(ph, nh, 3.0), ph, 0.8, SM, 0.5, np.asarray(segs, np.int64))
    xp, _ = _noalloc(x, vp, vn, 0.8, 0.7, 3.0, 0.5, segs)
    cc = float(np.float32(SM + (1 - SM) * 0.8))
    assert max_err(xp, orc.flow_step(xh, pred, 0.8, 0.7)) <= 1e-5 / cc


def test_noalloc_rejects_states_beyond_its_scratch(dev):
    """A dense state of 16,385 rows needs 16,385 statistics blocks, one more
    than the built-in scratch holds: refused before any launch, with the
    reason, while the workspace entry point still runs it."""
    x = torch.zeros((16385, 8), device=dev)
    with pytest.raises(_lib.T2HError, match="built-in scratch holds 16384"):
        _noalloc(x, x, x, 0.8, 0.7, 3.0, 0.5, None)
    xp, _ = ops.flow_euler_step(x, x, 0.8, 0.7, SM, v_neg=x, guidance_strength=3.0, guidance_rescale=0.5)
    assert xp.shape == x.shape
    # the largest dense state it takes (16,384 rows) runs
    x, vp, vn = _state(4030, (16384, 8), dev)
    got = _noalloc(x, vp, vn, 0.8, 0.7, 3.0, 0.5, None)
    want = ops.flow_euler_step(x, vp, 0.8, 0.7, SM, v_neg=vn, guidance_strength=3.0, guidance_rescale=0.5)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.parametrize("which", ["config4_two_segments", "config5_one_segment"])
def test_noalloc_step_in_a_hip_graph(dev, which):
    """The entry point's purpose: a sampler step recorded into a HIP graph.
    t2h_device_init did the scratch lookup, so the call only enqueues its
    kernels. Three replays with fresh inputs, eager no-allocation calls in
    between (which reuse the same scratch), each equal to the workspace entry
    point's result bit for bit. Two segments take the statistics pass and
    the elementwise pass; the config-5 latent as one segment takes the
    one-launch form, whose grid barrier lives in the same scratch."""
    if which == "config4_two_segments":
        _, off = workloads.config4()
        segs = off.tolist()
    else:
        _, off = workloads.config5()
        segs = [0, int(off[-1])]
    x, vp, vn = _state(4040, (int(off[-1]), 32), dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _noalloc(x, vp, vn, 0.8, 0.7, 3.0, 0.5, segs)          # warm-up off the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _noalloc(x, vp, vn, 0.8, 0.7, 3.0, 0.5, segs)
    g = torch.Generator(device=dev).manual_seed(4041)
    for rep in range(3):
        for a in (x, vp, vn):
            a.copy_(torch.randn(a.shape, generator=g, device=dev))
        graph.replay()
        other = _noalloc(vn, x, vp, 0.6, 0.5, 2.0, 0.7, segs)   # an eager call on the same scratch
        want = ops.flow_euler_step(x, vp, 0.8, 0.7, SM, v_neg=vn, guidance_strength=3.0, guidance_rescale=0.5,
                                   seg_offsets=segs)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], want[0]) and torch.equal(outs[1], want[1]), f"replay {rep}"
        ref_other = ops.flow_euler_step(vn, x, 0.6, 0.5, SM, v_neg=vp, guidance_strength=2.0, guidance_rescale=0.7,
                                        seg_offsets=segs)
        assert torch.equal(other[0], ref_other[0]), f"eager call after replay {rep}"
