"""GPU: the device entry points are stateless, reentrant and stream-ordered
(include/t2h.h, "Conventions"): two host threads, each enqueueing the
config-5 chain's ops (LN + modulate, QK RMSNorm + RoPE, GELU + bias, gated
residual, the sampler step with its rescale) on a stream of its own with
inputs of its own, interleaved many times, give bit for bit the results of
the same calls made one thread at a time on the default stream. Both streams
are created at the default priority."""
import threading

import numpy as np
import pytest
import torch

import oracle as orc
from _parity import to_dev
from t2h import nn, ops

pytestmark = pytest.mark.gpu


def make_inputs(seed, dev):
    rows, c, h, d, f = 3000, 1536, 12, 128, 6144
    g = torch.Generator(device=dev).manual_seed(seed)
    rn = lambda shape, std=1.0, mean=0.0, dt=torch.float16: (
        torch.randn(shape, generator=g, device=dev) * std + mean).to(dt)
    coords = np.zeros((rows, 4), np.int32)
    coords[:, 1:] = orc.Rng(seed).uniform((rows, 3), 0.0, 128.0).astype(np.int32)
    return dict(
        x=rn((rows, c)), shift=rn((c,), 0.1, dt=torch.float32), scale=rn((c,), 0.1, dt=torch.float32),
        q=rn((rows, h, d)), k=rn((rows, h, d)), gq=rn((h, d), 0.02, 1.0, torch.float32),
        gk=rn((h, d), 0.02, 1.0, torch.float32), coords=to_dev(coords, dev), u=rn((rows, f)),
        bias=rn((f,), 0.02, dt=torch.float32), y=rn((rows, c)), gate=rn((c,), 0.1, dt=torch.float32),
        lat=rn((rows, 32), dt=torch.float32), vp=rn((rows, 32), dt=torch.float32),
        vn=rn((rows, 32), dt=torch.float32))


def run_ops(inp, freqs):
    ws = torch.empty(ops.flow_euler_workspace(inp["lat"].shape[0], 32), dtype=torch.uint8, device=inp["x"].device)
    out = [ops.ln_modulate(inp["x"], 1e-6, shift=inp["shift"], scale=inp["scale"])]
    out += list(ops.qk_rmsnorm_rope(q=inp["q"], k=inp["k"], gamma_q=inp["gq"], gamma_k=inp["gk"], freqs=freqs,
                                    coords=inp["coords"]))
    out.append(ops.activation(inp["u"], ops.ACT_GELU_TANH, bias=inp["bias"]))
    out.append(ops.gate_residual(inp["x"], inp["y"], gate=inp["gate"]))
    out += list(ops.flow_euler_step(inp["lat"], inp["vp"], 0.6, 0.5, 1e-5, v_neg=inp["vn"], guidance_strength=3.0,
                                    guidance_rescale=0.7, workspace=ws))
    return out


def test_two_threads_two_streams_bit_exact(dev):
    freqs = nn.rope_freqs(128)
    inputs = [make_inputs(s, dev) for s in (101, 102)]
    want = [run_ops(i, freqs) for i in inputs]   # one thread, default stream
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in inputs]   # default priority
    got = [None, None]
    errors = []
    start = threading.Barrier(2)

    def worker(j):
        try:
            start.wait()
            with torch.cuda.stream(streams[j]):
                res = None
                for _ in range(8):   # interleave many enqueues with the other thread
                    res = run_ops(inputs[j], freqs)
                streams[j].synchronize()
                got[j] = res
        except Exception as e:   # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for j in range(2):
        assert len(got[j]) == len(want[j])
        for a, b in zip(got[j], want[j]):
            assert torch.equal(a, b), f"thread {j}: an op differs from the single-stream result"


def test_one_launch_rescale_on_two_streams(dev):
    """The one-launch rescale sizes its grid to fill the GPU and meets at a
    grid barrier. Two host threads each enqueue it on a stream of their own
    (config-5-sized latents, one segment each), interleaved, so the two grids
    compete for the CUs; blocks that are not resident in time leave their
    vectors to their grid's reducing block. Bit for bit the results of the
    same steps one at a time on the default stream."""
    T = 201436
    g = torch.Generator(device=dev).manual_seed(103)
    states = [[torch.randn((T, 32), generator=g, device=dev) for _ in range(3)] for _ in range(2)]
    wss = [torch.empty(ops.flow_euler_workspace(T, 32, 2), dtype=torch.uint8, device=dev) for _ in range(2)]

    def step(j):
        x, vp, vn = states[j]
        return ops.flow_euler_step(x, vp, 0.7, 0.6, 1e-5, v_neg=vn, guidance_strength=3.0, guidance_rescale=0.5,
                                   seg_offsets=[0, T], workspace=wss[j])

    want = [step(j) for j in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]   # default priority
    got, errors = [None, None], []
    start = threading.Barrier(2)

    def worker(j):
        try:
            start.wait()
            with torch.cuda.stream(streams[j]):
                res = None
                for _ in range(16):
                    res = step(j)
                streams[j].synchronize()
                got[j] = res
        except Exception as e:   # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for j in range(2):
        assert torch.equal(got[j][0], want[j][0]) and torch.equal(got[j][1], want[j][1]), f"thread {j}"
