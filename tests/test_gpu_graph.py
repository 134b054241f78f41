"""HIP graph capture. Every device entry point of t2h only enqueues kernels
on the caller's stream: no allocation, memset or host synchronisation inside
it. So torch.cuda.graph can capture a block's per-token chain together with
the MFMA qkv GEMM + pack and the sampler step (with its rescale workspace).
Each replay, with fresh inputs copied in and eager launches between the
replays, must equal the eager results bit for bit."""
import pytest
import torch

from t2h import nn, ops, workloads

pytestmark = pytest.mark.gpu


def test_graph_replays_equal_eager(dev):
    coords_np, offsets_np = workloads.config4()
    T = coords_np.shape[0]
    C, H, D, F = 1536, 12, 128, 6144
    B = offsets_np.shape[0] - 1
    g = torch.Generator(device=dev).manual_seed(77)

    def rn(shape, std=1.0, mean=0.0, dt=torch.float16):
        return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dt)

    coords = torch.from_numpy(coords_np).to(dev)
    offsets = torch.from_numpy(offsets_np).to(dev)
    t = torch.rand((1,), generator=g, device=dev) * 1000.0
    x, y, u = rn((T, C)), rn((T, C)), rn((T, F))
    q, k = rn((T, H, D)), rn((T, H, D))
    lat = [rn((T, 32), dt=torch.float32) for _ in range(3)]
    shift, scale, gate = (rn((B, C), 0.1, dt=torch.float32) for _ in range(3))
    gq, gk = rn((H, D), 0.02, 1.0, torch.float32), rn((H, D), 0.02, 1.0, torch.float32)
    bias = rn((F,), 0.02, dt=torch.float32)
    wqkv = rn((3 * C, C), 0.02)
    freqs = nn.rope_freqs(D)
    mp = (T + 63) // 64 * 64
    phases = ops.rope_phases(T, D, freqs, coords=coords, device=dev)
    seg = [int(v) for v in offsets_np]
    ws = torch.empty(ops.flow_euler_workspace(T, 32, len(seg)), dtype=torch.uint8, device=dev)

    def chain():
        return [ops.timestep_embedding(t, 256),
                ops.ln_modulate(x, 1e-6, shift=shift, scale=scale, offsets=offsets),
                *ops.qk_rmsnorm_rope(q=q, k=k, gamma_q=gq, gamma_k=gk, freqs=freqs, coords=coords),
                ops.activation(u, ops.ACT_GELU_TANH, bias=bias),
                ops.gate_residual(x, y, gate=gate, offsets=offsets),
                *ops.qkv_linear_pack(x, wqkv, H, bias=bias[:3 * C], gamma_q=gq, gamma_k=gk, mp=mp, lp=mp,
                                     freqs=freqs, phases=phases),
                *ops.flow_euler_step(lat[0], lat[1], 0.8, 0.7, 1e-5, v_neg=lat[2], guidance_strength=3.0,
                                     guidance_rescale=0.5, seg_offsets=seg, workspace=ws)]

    side = torch.cuda.Stream()   # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()                  # warm-up off the capture stream, as torch requires
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = chain()
    fresh = [t, x, y, u, q, k, *lat]
    for rep in range(3):
        print(f"graph replay {rep}", flush=True)
        for a in fresh:
            a.copy_(torch.randn(a.shape, generator=g, device=dev).to(a.dtype) * (1000.0 if a is t else 1.0))
        t.abs_()
        graph.replay()
        want = chain()
        torch.cuda.synchronize()
        assert len(outs) == len(want)
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), f"replay {rep}, output {i}"
