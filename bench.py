#!/usr/bin/env python3
"""Benchmark of the fused per-token DiT layer ops on one MI355X.

Default workload: the per-block chain over T = 201,436
sparse tokens (a thickened sphere shell on a 128^3 grid), width 1536,
12 x 128 heads, hidden 6144, f16 storage:

    timestep embedding [1, 256]
    -> LayerNorm + adaLN modulate          x[T,1536] -> h[T,1536]
    -> QK RMSNorm + 3D RoPE from coords    q,k[T,12,128], in place
    -> GELU-tanh(+bias)                    u[T,6144], in place
    -> gated residual                      x + gate*y -> out[T,1536]

One step = one pass of this chain; inputs are resident in HBM before the
timed region. value = algorithmic HBM bytes of the chain / time (GB/s);
52,240 bytes per token (6,144 + 12,304 + 24,576 + 9,216).

Prints ONE JSON line on stdout; per-op and per-config detail goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "trellis2-mojo_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16/bf16 matrix peak
METRIC = "fused-layer HBM GB/s (% of MI355X peak) and tokens/s at width 1536, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-ms", type=float, default=400.0,
                   help="GPU time of untimed chain steps before the steady-state windows")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU baseline sample time")
    p.add_argument("--no-configs", action="store_true", help="skip BASELINE configs 1-4")
    p.add_argument("--configs-only", action="store_true",
                   help="time only BASELINE configs 1-4 and print their JSON (for profiler runs)")
    p.add_argument("--op", default=None, help="time only one op of the chain (for profiling)")
    p.add_argument("--sweep", action="store_true",
                   help="time the config-5 chain at several token counts and print their JSON")
    p.add_argument("--small-t", action="store_true",
                   help="time only the small-T block and the chain at the SLat token count and print their JSON")
    return p.parse_args()


class Chain:
    """Device buffers and launches of the config-5 chain."""

    C, H, D, F = 1536, 12, 128, 6144

    def __init__(self, dev, dtype, tokens=None):
        import numpy as np
        import torch

        from t2h import nn, ops, workloads

        self.torch, self.ops, self.np = torch, ops, np
        if tokens is None:
            coords, offsets = workloads.config5()
        else:   # one batch of `tokens` voxels at random positions on the 128^3 grid
            coords = np.zeros((tokens, 4), np.int32)
            coords[:, 1:] = np.random.default_rng(tokens).integers(0, 128, (tokens, 3), dtype=np.int32)
            offsets = np.array([0, tokens], np.int64)
        self.coords_np = coords
        self.T = T = coords.shape[0]
        C, H, D, F = self.C, self.H, self.D, self.F
        g = torch.Generator(device=dev).manual_seed(5)

        def rn(shape, std=1.0, mean=0.0, dt=dtype):
            return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std + mean).to(dt)

        self.coords = torch.from_numpy(coords).to(dev)
        self.offsets = torch.from_numpy(offsets).to(dev)
        self.t = torch.rand((1,), generator=g, device=dev) * 1000.0            # t * 1000 (flow_euler.mojo:168)
        self.x = rn((T, C))
        self.shift, self.scale, self.gate = rn((1, C), 0.1, dt=torch.float32), rn((1, C), 0.1, dt=torch.float32), \
            rn((1, C), 0.1, dt=torch.float32)
        self.h = torch.empty_like(self.x)
        self.q, self.k = rn((T, H, D)), rn((T, H, D))
        self.gq, self.gk = rn((H, D), 0.02, 1.0, torch.float32), rn((H, D), 0.02, 1.0, torch.float32)
        self.freqs = nn.rope_freqs(D)
        self.u = rn((T, F))
        self.bias = rn((F,), 0.02, dt=torch.float32)
        self.y = rn((T, C))
        # QK and GELU + bias run in place, as the reference's device kernels
        # do (bias_rms_rope_qkv on the qkv rows, gpu/attention.mojo:507-563;
        # gelu_tanh_bias on the fc1 rows, gpu/linear.mojo:662-690): the bytes
        # of an out-of-place launch over half the pages, 2 % and 1 % faster.
        # The gated residual writes a new tensor: in place on x (as
        # gpu/block.mojo:86-110 does) the next step's LN + modulate ran
        # 15-17 us slower, more than the residual gained.
        self.qo, self.ko = self.q, self.k
        self.gout = self.u
        self.res = torch.empty_like(self.x)
        self.temb = None
        e = 2 if dtype != torch.float32 else 4
        self.bytes = {  # algorithmic HBM bytes per launch
            "timestep": 1 * (4 + 256 * 4),
            "ln_modulate": 2 * T * C * e + 2 * C * 4,
            "qk_rmsnorm_rope": 4 * T * C * e + T * 16 + 2 * H * D * 4,
            "gelu_tanh_bias": 2 * T * F * e + F * 4,
            "gate_residual": 3 * T * C * e + C * 4,
            "copy": 2 * T * F * e,
        }
        # algorithmic bytes per token: LN+modulate, QK RMSNorm+RoPE, GELU+bias, gated residual
        self.chain_bytes = (6144 + 12304 + 24576 + 9216) * T

    def op(self, name):
        o = self.ops
        if name == "timestep":
            return lambda: o.timestep_embedding(self.t, 256)
        if name == "ln_modulate":
            return lambda: o.ln_modulate(self.x, 1e-6, shift=self.shift, scale=self.scale, offsets=self.offsets,
                                         out=self.h)
        if name == "qk_rmsnorm_rope":
            return lambda: o.qk_rmsnorm_rope(q=self.q, k=self.k, gamma_q=self.gq, gamma_k=self.gk, freqs=self.freqs,
                                             coords=self.coords, q_out=self.qo, k_out=self.ko)
        if name == "gelu_tanh_bias":
            return lambda: o.activation(self.u, o.ACT_GELU_TANH, bias=self.bias, out=self.gout)
        if name == "gate_residual":
            return lambda: o.gate_residual(self.x, self.y, gate=self.gate, offsets=self.offsets, out=self.res)
        if name == "copy":  # calibration: torch's vectorized elementwise kernel over the GELU tensor (u *= 1)
            return lambda: self.torch.mul(self.u, 1.0, out=self.gout)
        if name == "chain":
            return self.step
        if name in self.NEXT_OPS:
            return self.next_op(name)
        if name in self.GEMM_OPS:
            g = self.gemm_state()
            if name == "linear_qkv":
                return lambda: o.linear(self.x, g["wqkv"], out=g["out"][:, :3 * self.C])
            if name == "linear_fc1_gelu":
                return lambda: o.linear(self.x, g["w1"], bias=self.bias, act=o.ACT_GELU_TANH, out=g["out"])
            if name == "linear_fc2_gate_residual":
                return lambda: o.linear_gate_residual(self.u, g["w2"], self.x, bias=self.bias[:self.C],
                                                      gate=self.gate, offsets=self.offsets, out=self.res)
            return lambda: o.qkv_linear_pack(self.x, g["wqkv"], self.H, bias=self.bias[:3 * self.C], gamma_q=self.gq,
                                             gamma_k=self.gk, mp=g["mp"], lp=g["mp"], freqs=self.freqs,
                                             phases=g["phases"], k_transposed=True)
        raise KeyError(name)

    # the per-token work around the chain on the config-5 rows (f16): the
    # block glue over one const buffer (chains stubbed by a resident tensor,
    # so only the glue kernels run), the attention epilogue + head-major pack,
    # and the sampler step on the tokens' 32-channel f32 latent
    NEXT_OPS = ("block_glue_fused", "block_glue_unfused", "attn_pack_kt", "attn_pack_krows",
                "flow_euler_step_cfg", "flow_euler_step_cfg_rescale", "flow_euler_step_cfg_rescale_two_launch")

    def next_state(self):
        if getattr(self, "_next", None) is None:
            torch = self.torch
            from t2h import block, ops

            T, C, H = self.T, self.C, self.H
            dev = self.x.device
            m = [self.shift, self.scale, self.gate, self.shift, self.scale, self.gate]
            ones = torch.ones(C, dtype=torch.float32, device=dev)
            st = {"bk": block.pack_block_consts(m, ones, self.shift.reshape(-1), self.bias[:C], self.bias[C:2 * C],
                                                self.bias[2 * C:3 * C]),
                  "xs": self.x.clone(), "mp": (T + 63) // 64 * 64}
            st["q3"] = self.u[:, :3 * C].contiguous().reshape(T, 3, H, self.D)
            st["b3"] = self.bias[:3 * C].reshape(3, H * self.D)
            g = torch.Generator(device=dev).manual_seed(7)
            st["lat"] = [torch.randn((T, 32), generator=g, device=dev) for _ in range(3)]
            st["lat_out"] = [torch.empty((T, 32), device=dev) for _ in range(2)]
            st["ws"] = torch.empty(ops.flow_euler_workspace(T, 32, 2), dtype=torch.uint8, device=dev)
            st["ws2"] = torch.empty(256 * 32, dtype=torch.uint8, device=dev)   # 256 statistics partials
            self._next = st
        return self._next

    def next_bytes(self, name):
        T, C = self.T, self.C
        e = 2
        n = T * 32 * 4
        mp = (T + 63) // 64 * 64
        return {"block_glue_fused": 13 * T * C * e, "block_glue_unfused": 15 * T * C * e,   # row-passes of C
                "attn_pack_kt": T * 3 * C * e + 3 * mp * C * e + T * 16,
                "attn_pack_krows": T * 3 * C * e + 3 * mp * C * e + T * 16,
                # CFG: reads x, v_pos, v_neg, writes x_prev, pred_x0. The rescale in
                # one launch holds the three inputs in registers across its grid
                # barrier (the same five passes); in two launches its statistics
                # pass reads them once more
                "flow_euler_step_cfg": 5 * n, "flow_euler_step_cfg_rescale": 5 * n,
                "flow_euler_step_cfg_rescale_two_launch": 8 * n}[name]

    def next_op(self, name):
        from t2h import block, ops

        st = self.next_state()
        if name.startswith("block_glue"):
            stub = lambda h: self.y
            fused = name.endswith("_fused")
            return lambda: block.cross_block_enqueue(st["xs"], st["bk"], stub, stub, stub, fused=fused)
        if name.startswith("attn_pack"):
            q3, b3, mp = st["q3"], st["b3"], st["mp"]
            kt = name == "attn_pack_kt"
            return lambda: ops.attn_pack(q3[:, 0], q3[:, 1], q3[:, 2], mp=mp, lp=mp, bias_q=b3[0], bias_k=b3[1],
                                         bias_v=b3[2], gamma_q=self.gq, gamma_k=self.gk, freqs=self.freqs,
                                         coords=self.coords, k_transposed=kt)
        lat, lo = st["lat"], st["lat_out"]
        if name == "flow_euler_step_cfg":
            return lambda: ops.flow_euler_step(lat[0], lat[1], 0.8, 0.7, 1e-5, v_neg=lat[2], guidance_strength=3.0,
                                               x_prev=lo[0], pred_x0=True)
        # CFG 3.0 + rescale 0.5 over one token segment; a workspace without
        # room for the one-launch form's barrier gives the two-launch form
        ws = st["ws"] if name == "flow_euler_step_cfg_rescale" else st["ws2"]
        return lambda: ops.flow_euler_step(lat[0], lat[1], 0.8, 0.7, 1e-5, v_neg=lat[2], guidance_strength=3.0,
                                           guidance_rescale=0.5, seg_offsets=[0, self.T], workspace=ws,
                                           x_prev=lo[0])

    # the GEMM rows (f16 operands on the matrix cores): flops per launch
    GEMM_OPS = ("linear_qkv", "linear_fc1_gelu", "qkv_linear_pack", "linear_fc2_gate_residual")

    def gemm_flops(self, name):
        if name == "linear_fc2_gate_residual":
            return 2.0 * self.T * self.C * self.F
        n = self.F if name == "linear_fc1_gelu" else 3 * self.C
        return 2.0 * self.T * n * self.C

    def gemm_state(self):
        if getattr(self, "_gemm", None) is None:
            torch, o = self.torch, self.ops
            g = torch.Generator(device=self.x.device).manual_seed(9)
            rw = lambda n: (torch.randn((n, self.C), generator=g, device=self.x.device) * 0.02).to(self.x.dtype)
            self._gemm = {"wqkv": rw(3 * self.C), "w1": rw(self.F),
                          "w2": (torch.randn((self.C, self.F), generator=g, device=self.x.device) * 0.02).to(
                              self.x.dtype),
                          "out": torch.empty((self.T, self.F), dtype=self.x.dtype, device=self.x.device),
                          "mp": (self.T + 63) // 64 * 64,
                          "phases": o.rope_phases(self.T, self.D, self.freqs, coords=self.coords,
                                                  device=self.x.device)}
        return self._gemm

    ORDER = ["timestep", "ln_modulate", "qk_rmsnorm_rope", "gelu_tanh_bias", "gate_residual"]

    def step(self):
        for n in self.ORDER:
            self.op(n)()


def time_region(torch, fn, steps):
    """Events on torch's current stream (the stream every t2h op enqueues on)."""
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e)


def steady_state(torch, chain, settle_ms, steps, rounds=3):
    """The chain after settle_ms of untimed chain steps.
    - steady: windows of `steps` whole chain steps (median of `rounds`);
    - per_op (in-chain marginal time of each op): the same window with that
      op left out, subtracted from the interleaved whole-chain window, so no
      event sits inside a timed window (each event record between two kernels
      adds a ~5.6 us gap, which a kernel trace shows);
    - per_op_events: one window with an event between consecutive ops (each
      interval includes one such gap)."""
    t0 = time.perf_counter()
    settled = 0.0
    while settled < settle_ms:
        settled += time_region(torch, chain.step, 20)
        if time.perf_counter() - t0 > 10.0:
            break
    fns = {n: chain.op(n) for n in Chain.ORDER}

    def without(skip):
        rest = [fns[n] for n in Chain.ORDER if n != skip]

        def run():
            for f in rest:
                f()
        return run

    full, left = [], {n: [] for n in Chain.ORDER}
    for _ in range(rounds):
        full.append(time_region(torch, chain.step, steps) / steps)
        for n in Chain.ORDER:
            left[n].append(time_region(torch, without(n), steps) / steps)
    ms = statistics.median(full)
    per_op = {}
    for n in Chain.ORDER:
        m = ms - statistics.median(left[n])
        # an op whose marginal time is within the windows' noise (the ~4 us
        # timestep in a ~1.6 ms step) can come out at or below zero: its time
        # is kept as measured and it gets no rate
        ok = m > 1e-3
        per_op[n] = {"us": round(m * 1e3, 2), "bytes": chain.bytes[n],
                     "gbs": round(chain.bytes[n] / m / 1e6, 1) if ok else None,
                     "pct_of_peak": round(chain.bytes[n] / m / 1e6 / HBM_PEAK_GBS * 100, 2) if ok else None}
    order = [fns[n] for n in Chain.ORDER]
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(order) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    # ten untimed chain steps ahead of the window (~16 ms of GPU work): the
    # host enqueues the window's launches and events meanwhile, so no
    # interval waits for the host and the GPU never idles
    for _ in range(10):
        chain.step()
    for k in range(steps):
        e = ev[k]
        e[0].record()
        for i, fn in enumerate(order):
            fn()
            e[i + 1].record()
    torch.cuda.synchronize()
    per_ev = {}
    for i, n in enumerate(Chain.ORDER):
        ts = [ev[k][i].elapsed_time(ev[k][i + 1]) for k in range(steps)]
        m = statistics.mean(ts)
        per_ev[n] = {"us": round(m * 1e3, 2), "median_us": round(statistics.median(ts) * 1e3, 2),
                     "gbs": round(chain.bytes[n] / m / 1e6, 1)}
    gbs = chain.chain_bytes / ms / 1e6
    return {"settle_ms": round(settled, 1), "steps": steps, "rounds": rounds, "us_per_step": round(ms * 1e3, 2),
            "gbs": round(gbs, 1), "pct_of_peak": round(gbs / HBM_PEAK_GBS * 100, 2),
            "tokens_per_s": round(chain.T / ms * 1e3),
            "per_op_sum_us": round(sum(v["us"] for v in per_op.values()), 2), "per_op": per_op,
            "per_op_events": per_ev,
            "per_op_events_sum_us": round(sum(v["us"] for v in per_ev.values()), 2)}

def time_op(torch, fn, reps, flush=None):
    """Median per-launch ms of one launch between two events. With `flush`,
    the device caches are flushed (>= 1 GiB streamed) before each launch;
    without, a short spin kernel runs first. Either way the GPU is still busy
    when the host enqueues the launch, so the host's call overhead stays
    outside the timed interval."""
    times = []
    for _ in range(reps):
        if flush is not None:
            flush()
        else:
            torch.cuda._sleep(200000)   # ~0.1 ms of GPU spin, no memory traffic
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return statistics.median(times)


def cpu_info():
    """nproc, the CPUs this process may run on, and the CPU model."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count() or 1, "usable_cpus": usable, "cpu_model": model}


def cpu_baseline(chain, target_s):
    """The C oracle (the reference's CPU path restated) over the config-5
    chain, f32 math on the f16-rounded inputs of the first n tokens (n grows
    until one pass takes about target_s), timed two ways on the host cores:
    - "reference threading": LN/modulate, the phase build and the gated
      residual serial, GELU/RMSNorm/RoPE-rotate in OpenMP chunks above 2^17
      elements, as the reference's parallelize calls;
    - "all cores": every op split by rows over the same threads (ctypes
      releases the GIL, so the C oracle runs in parallel).
    Threads = the CPUs this process may use, at most 16 (the box's CPU share
    for one GPU)."""
    import concurrent.futures as cf

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    info = cpu_info()
    threads = max(1, min(info["usable_cpus"], 16))
    D = chain.D
    pool = cf.ThreadPoolExecutor(threads)

    def inputs(n):
        d = {"x": chain.x[:n].float().cpu().numpy(), "q": chain.q[:n].float().cpu().numpy(),
             "k": chain.k[:n].float().cpu().numpy(), "u": chain.u[:n].float().cpu().numpy(),
             "y": chain.y[:n].float().cpu().numpy(), "co": chain.coords_np[:n]}
        d.update(sh=chain.shift.cpu().numpy(), sc=chain.scale.cpu().numpy(), gt=chain.gate.cpu().numpy(),
                 gq=chain.gq.cpu().numpy(), gk=chain.gk.cpu().numpy(), bias=chain.bias.cpu().numpy(),
                 tt=chain.t.cpu().numpy(), freqs=orc.rope_freqs(D))
        return d

    def run_reference(d, n):
        off = np.array([0, n], np.int64)
        t0 = time.perf_counter()
        orc.timestep_embedding(d["tt"], 256)
        orc.ln_modulate(d["x"], d["sh"], d["sc"], offsets=off, eps=1e-6)
        ph = orc.rope_phases_from_coords(d["co"], D, d["freqs"])
        orc.qk_rms_rope(d["q"], d["k"], d["gq"], d["gk"], ph, nthreads=threads)
        orc.gelu_tanh_bias(d["u"], d["bias"], nthreads=threads)
        orc.gate_residual(d["x"], d["y"], d["gt"], offsets=off)
        return time.perf_counter() - t0

    def run_all_cores(d, n):
        cuts = np.linspace(0, n, threads + 1).astype(np.int64)
        parts = list(zip(cuts[:-1], cuts[1:]))

        def piece(lo, hi):
            m = hi - lo
            off = np.array([0, m], np.int64)
            orc.ln_modulate(d["x"][lo:hi], d["sh"], d["sc"], offsets=off, eps=1e-6)
            ph = orc.rope_phases_from_coords(d["co"][lo:hi], D, d["freqs"])
            orc.qk_rms_rope(d["q"][lo:hi], d["k"][lo:hi], d["gq"], d["gk"], ph, nthreads=1)
            orc.gelu_tanh_bias(d["u"][lo:hi], d["bias"], nthreads=1)
            orc.gate_residual(d["x"][lo:hi], d["y"][lo:hi], d["gt"], offsets=off)

        t0 = time.perf_counter()
        orc.timestep_embedding(d["tt"], 256)
        list(pool.map(lambda p: piece(*p), parts))
        return time.perf_counter() - t0

    out = {}
    for name, fn in (("reference_threading", run_reference), ("all_cores", run_all_cores)):
        n = 2048
        dt = fn(inputs(n), n)
        n = int(min(chain.T, max(n, n * target_s / max(dt, 1e-3))))
        dt = fn(inputs(n), n)
        out[name] = {"tokens_per_s": n / dt, "seconds": dt, "tokens": n,
                     "gbs_equiv": chain.chain_bytes / chain.T * n / dt / 1e9}
    pool.shutdown()
    ref = out["reference_threading"]
    n = ref["tokens"]
    return {"value": ref["tokens_per_s"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"one pass of the config-5 chain over the first {n} of {chain.T} tokens (f32 C oracle on "
                      f"f16-rounded inputs, {ref['seconds']:.1f} s) with the reference's threading: OpenMP "
                      f"{threads} threads for GELU/RMSNorm/RoPE-rotate as its parallelize, the rest serial",
            "all_cores": {"value": out["all_cores"]["tokens_per_s"], "threads": threads,
                          "seconds": out["all_cores"]["seconds"], "tokens": out["all_cores"]["tokens"],
                          "note": "every op split by rows over the same threads"},
            **info, "gbs_equiv": ref["gbs_equiv"]}


def other_configs(torch, dev, cpu=True):
    """BASELINE configs 1-4, each op alone: GPU warm and cold (caches flushed
    by a 1 GiB fill before each launch), and the C oracle on the same inputs
    on the host (the reference's threading: LN/modulate/gate serial, GELU,
    RMSNorm and RoPE-rotate in OpenMP chunks; best of 2 passes)."""
    import numpy as np

    from t2h import nn, ops, workloads

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    threads = max(1, min(cpu_info()["usable_cpus"], 16))
    g = torch.Generator(device=dev).manual_seed(1)
    rn = lambda shape, std=1.0, mean=0.0, dt=torch.float32: (
        torch.randn(shape, generator=g, device=dev) * std + mean).to(dt)
    hst = lambda t: t.float().cpu().numpy()
    flush_buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    flush = lambda: flush_buf.zero_()
    res = {}

    def rec(name, fn, nbytes, tokens, cpu_fn, reps=30):
        for _ in range(3):
            fn()
        warm = time_op(torch, fn, reps)
        cold = time_op(torch, fn, reps, flush)
        r = {"bytes": nbytes, "tokens": tokens, "warm_us": round(warm * 1e3, 2), "cold_us": round(cold * 1e3, 2),
             "warm_gbs": round(nbytes / warm / 1e6, 1), "cold_gbs": round(nbytes / cold / 1e6, 1),
             "cold_pct_peak": round(nbytes / cold / 1e6 / HBM_PEAK_GBS * 100, 2),
             "warm_pct_peak": round(nbytes / warm / 1e6 / HBM_PEAK_GBS * 100, 2),
             "tokens_per_s_cold": round(tokens / cold * 1e3), "tokens_per_s_warm": round(tokens / warm * 1e3)}
        msg = ""
        if cpu and cpu_fn is not None:
            best = None
            for _ in range(2):
                t0 = time.perf_counter()
                cpu_fn()
                dt = time.perf_counter() - t0
                best = dt if best is None else min(best, dt)
            r["cpu_tokens_per_s"] = round(tokens / best)
            r["cpu_threads"] = threads
            msg = f" | cpu {tokens / best:10.0f} tok/s"
        res[name] = r
        log(f"  {name:<28s} warm {warm*1e3:8.1f} us {nbytes/warm/1e6:8.1f} GB/s | cold {cold*1e3:8.1f} us "
            f"{nbytes/cold/1e6:8.1f} GB/s ({nbytes/cold/1e6/HBM_PEAK_GBS*100:5.1f}%){msg}")

    def rec_stream(name, make, nbytes):
        """Back-to-back launches over rotating buffer sets whose footprint
        (>= 600 MB) exceeds the 256 MB infinity cache: every launch reads
        HBM, and a launch's dispatch overlaps its predecessor's tail, as in
        a block sequence. ~60 launches (the sets in turn) per event pair."""
        k = max(2, -(-600_000_000 // (2 * nbytes)))
        fns = [make() for _ in range(k)]
        for f in fns:
            f()
        rounds = max(1, 60 // k)   # ~60 launches per window, so the two events' cost is spread thin
        times = []
        for _ in range(9):
            torch.cuda.synchronize()
            # ~5 ms of GPU spin: the host enqueues all k * rounds launches meanwhile
            torch.cuda._sleep(10_000_000)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(rounds):
                for f in fns:
                    f()
            e.record()
            torch.cuda.synchronize()
            times.append(s.elapsed_time(e))
        ms = statistics.median(times) / (k * rounds)
        res[name].update({"stream_us": round(ms * 1e3, 2), "stream_gbs": round(nbytes / ms / 1e6, 1),
                          "stream_pct_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS * 100, 2), "stream_sets": k,
                          "stream_launches": k * rounds})
        log(f"  {name:<28s} back-to-back over {k} buffer sets: {ms*1e3:8.1f} us {nbytes/ms/1e6:8.1f} GB/s "
            f"({nbytes/ms/1e6/HBM_PEAK_GBS*100:5.1f}%)")
        del fns

    # The fixed cost of one launch under this protocol: a t2h kernel on one
    # 64-element row, bracketed by the same two events.
    tiny, tiny_o = rn((1, 64)), torch.empty(1, 64, device=dev)
    tiny_fn = lambda: ops.activation(tiny, 0, out=tiny_o)
    for _ in range(3):
        tiny_fn()
    fw, fc = time_op(torch, tiny_fn, 30), time_op(torch, tiny_fn, 30, flush)
    res["launch_floor"] = {"warm_us": round(fw * 1e3, 2), "cold_us": round(fc * 1e3, 2),
                           "what": "one t2h launch on a 64-element row, timed as the configs are"}
    log(f"  launch floor (64-element kernel): warm {fw*1e3:.1f} us, cold {fc*1e3:.1f} us")

    C = 1536
    x = rn((4096, C)); sh = rn((C,), 0.1); sc = rn((C,), 0.1); out = torch.empty_like(x)
    hx, hsh, hsc = hst(x), hst(sh), hst(sc)
    rec("c1_ln_modulate_f32", lambda: ops.ln_modulate(x, 1e-6, shift=sh, scale=sc, out=out),
        2 * 4096 * C * 4 + 2 * C * 4, 4096, lambda: orc.ln_modulate(hx, hsh, hsc, eps=1e-6))

    def make_c1():
        xi, oi = rn((4096, C)), torch.empty(4096, C, device=dev)
        return lambda: ops.ln_modulate(xi, 1e-6, shift=sh, scale=sc, out=oi)

    rec_stream("c1_ln_modulate_f32", make_c1, 2 * 4096 * C * 4 + 2 * C * 4)
    q, k = rn((4096, 12, 128)), rn((4096, 12, 128)); gq, gk = rn((12, 128), 0.02, 1.0), rn((12, 128), 0.02, 1.0)
    qo, ko = torch.empty_like(q), torch.empty_like(k); fr = nn.rope_freqs(128)
    hq, hk, hgq, hgk = hst(q), hst(k), hst(gq), hst(gk)
    ofr = orc.rope_freqs(128)

    def cpu_c2():   # phases built per forward from the grid (modules/rope.mojo:39-61), then RMS + rotate
        ph = orc.rope_phases_from_positions(orc.grid_positions(16), 128, ofr)
        orc.qk_rms_rope(hq, hk, hgq, hgk, ph, nthreads=threads)

    rec("c2_qk_rms_rope_f32", lambda: ops.qk_rmsnorm_rope(q=q, k=k, gamma_q=gq, gamma_k=gk, freqs=fr, grid_res=16,
                                                           q_out=qo, k_out=ko), 4 * 4096 * C * 4 + 2 * C * 4, 4096,
        cpu_c2)

    def make_c2():
        qi, ki = rn((4096, 12, 128)), rn((4096, 12, 128))
        qoi, koi = torch.empty_like(qi), torch.empty_like(ki)
        return lambda: ops.qk_rmsnorm_rope(q=qi, k=ki, gamma_q=gq, gamma_k=gk, freqs=fr, grid_res=16, q_out=qoi,
                                           k_out=koi)

    rec_stream("c2_qk_rms_rope_f32", make_c2, 4 * 4096 * C * 4 + 2 * C * 4)
    del x, out, q, k, qo, ko
    h = rn((32768, 6144), dt=torch.float16); b = rn((6144,), 0.02); ho = torch.empty_like(h)
    hh, hb = hst(h), hst(b)
    rec("c3a_gelu_bias_f16", lambda: ops.activation(h, 3, bias=b, out=ho), 2 * 32768 * 6144 * 2 + 6144 * 4, 32768,
        lambda: orc.gelu_tanh_bias(hh, hb, nthreads=threads), 20)
    del h, ho, hh
    xr, yr = rn((32768, C), dt=torch.float16), rn((32768, C), dt=torch.float16); gt = rn((C,), 0.1)
    ro = torch.empty_like(xr)
    hxr, hyr, hgt = hst(xr), hst(yr), hst(gt)
    rec("c3b_gated_residual_f16", lambda: ops.gate_residual(xr, yr, gate=gt, out=ro), 3 * 32768 * C * 2 + C * 4,
        32768, lambda: orc.gate_residual(hxr, hyr, hgt))
    del xr, yr, ro, hxr, hyr
    coords, offsets = workloads.config4()
    T = coords.shape[0]
    co, off = torch.from_numpy(coords).to(dev), torch.from_numpy(offsets).to(dev)
    f4 = rn((T, C)); s4, c4 = rn((2, C), 0.1), rn((2, C), 0.1); o4 = torch.empty_like(f4)
    hf4, hs4, hc4 = hst(f4), hst(s4), hst(c4)
    rec("c4_sparse_ln_mod_f32", lambda: ops.ln_modulate(f4, 1e-6, shift=s4, scale=c4, offsets=off, out=o4),
        2 * T * C * 4 + 2 * 2 * C * 4 + 16, T, lambda: orc.ln_modulate(hf4, hs4, hc4, offsets=offsets, eps=1e-6))
    q4, k4 = rn((T, 12, 128)), rn((T, 12, 128)); q4o, k4o = torch.empty_like(q4), torch.empty_like(k4)
    hq4, hk4 = hst(q4), hst(k4)

    def cpu_c4():   # phases from the int coords (sparse/attention/rope.mojo:48-66), then RMS + rotate
        ph = orc.rope_phases_from_coords(coords, 128, ofr)
        orc.qk_rms_rope(hq4, hk4, hgq, hgk, ph, nthreads=threads)

    rec("c4_sparse_qk_rope_f32", lambda: ops.qk_rmsnorm_rope(q=q4, k=k4, gamma_q=gq, gamma_k=gk, freqs=fr, coords=co,
                                                              q_out=q4o, k_out=k4o), 4 * T * C * 4 + T * 16, T,
        cpu_c4)
    return res


def small_t_block(torch, dev, reps):
    """The dense sparse-structure DiT's block at its real shape: 4096 tokens
    (16^3 grid), width 1536, 12 x 128 heads, hidden 6144, f32 (the
    reference's dtype; models/sparse_structure_flow.mojo:190-206 runs it 30
    blocks x 2 CFG branches x the sampler steps). One block's per-token work
    over the 12*C const buffer (gpu/block.mojo:217-397), the GEMM and SDPA
    outputs stubbed by resident tensors:
      LN1 + modulate -> qkv epilogue in place (bias, RMS q/k, RoPE from the
      grid) -> self join + norm2 (affine) -> cross join + LN3 + modulate ->
      GELU-tanh + bias in place on the MLP hidden -> gated MLP join.
    Timed as eager launches, as HIP-graph replays of 30 blocks (a forward's
    blocks in one graph; per-block time) and of one block."""
    from t2h import block, nn, ops

    T, C, H, D, F = 4096, 1536, 12, 128, 6144
    g = torch.Generator(device=dev).manual_seed(11)
    rn = lambda shape, std=1.0, mean=0.0: torch.randn(shape, generator=g, device=dev) * std + mean
    m = [rn((C,), 0.1) for _ in range(6)]
    bk = block.pack_block_consts(m, rn((C,), 0.1, 1.0), rn((C,), 0.1), rn((C,), 0.02), rn((C,), 0.02),
                                 rn((C,), 0.02))
    x0 = rn((T, C))
    x, hs, hs2 = x0.clone(), torch.empty(T, C, device=dev), torch.empty(T, C, device=dev)
    qkv, h_self, h_cross, hid, h_mlp = rn((T, 3 * C)), rn((T, C)), rn((T, C)), rn((T, F)), rn((T, C))
    qkv_bias, fbias = rn((3 * C,), 0.02), rn((F,), 0.02)
    gq, gk = rn((H, D), 0.02, 1.0), rn((H, D), 0.02, 1.0)
    freqs = nn.rope_freqs(D)

    def step():
        ops.ln_mod_rows(x, hs, bk, 0, 1)
        ops.qkv_bias_rmsnorm_rope(qkv, H, D, bias=qkv_bias, gamma_q=gq, gamma_k=gk, freqs=freqs, grid_res=16)
        ops.block_join_ln(x, h_self, hs2, bk, 2 * C, 1, 4 * C, 2)
        ops.block_join_ln(x, h_cross, hs, bk, 6 * C, 0, 8 * C, 1)
        ops.activation(hid, ops.ACT_GELU_TANH, bias=fbias, out=hid)   # in place (gpu/linear.mojo:662-690)
        ops.gate_add_bias_rows(x, h_mlp, bk, 10 * C, 1)

    e = 4
    nbytes = (2 + 6 + 4 + 4 + 3) * T * C * e + 2 * T * F * e + 12 * C * 4
    step()

    def gpu_time(fn, n):
        """GPU time of n calls: a GPU spin in front lets the host enqueue
        every launch before the first one runs, so host overhead between
        launches stays outside the interval."""
        torch.cuda.synchronize()
        torch.cuda._sleep(n * 200_000)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(n):
            fn()
        s1.record()
        torch.cuda.synchronize()
        return s0.elapsed_time(s1) / n

    def capture(nblocks):
        """One HIP graph of nblocks consecutive blocks (the reference enqueues
        every block of a forward before one barrier, sparse_structure_flow.mojo:
        191-206): each hipGraphLaunch costs a gap of ~8 us before the next one
        starts (kernel trace), which a whole forward in one graph pays once."""
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                for _ in range(nblocks):
                    step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph.replay()
        return graph

    g1 = capture(1)
    replay1 = gpu_time(g1.replay, reps)
    del g1
    # eager and the 30-block graph in interleaved windows of 30 blocks
    # (medians of 7: single windows vary by ~3 % between runs)
    nb = 30
    gf = capture(nb)
    ev, gr = [], []
    for _ in range(7):
        ev.append(gpu_time(step, nb))
        gr.append(gpu_time(gf.replay, 1) / nb)
    del gf
    eager, replay = statistics.median(ev), statistics.median(gr)
    res = {"tokens": T, "launches": 6, "bytes": nbytes,
           "eager_us": round(eager * 1e3, 2), "graph_us": round(replay * 1e3, 2), "graph_blocks": nb,
           "graph_1_block_us": round(replay1 * 1e3, 2),
           "eager_gbs": round(nbytes / eager / 1e6, 1), "graph_gbs": round(nbytes / replay / 1e6, 1),
           "eager_pct_peak": round(nbytes / eager / 1e6 / HBM_PEAK_GBS * 100, 2),
           "graph_pct_peak": round(nbytes / replay / 1e6 / HBM_PEAK_GBS * 100, 2)}
    log(f"  ss-flow block glue + qk f32 [4096]: eager {eager*1e3:.1f} us ({nbytes/eager/1e6:.0f} GB/s), "
        f"graph of {nb} blocks {replay*1e3:.1f} us/block ({nbytes/replay/1e6:.0f} GB/s), graph of one block "
        f"{replay1*1e3:.1f} us")
    return res


def next_rows(torch, dev, chain, reps):
    """The per-token work around the chain, on the config-5 rows (f16): the
    block glue over one const buffer (chains stubbed by a resident tensor, so
    only the glue kernels run) and the attention epilogue + head-major pack."""
    from t2h import block, ops

    T, C, H, D = chain.T, chain.C, chain.H, chain.D
    e = 2
    res = {}

    def rec(name, fn, nbytes):
        fn()
        ms = time_region(torch, fn, reps) / reps
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
                     "pct_of_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS * 100, 2)}
        log(f"  {name:<26s} {ms*1e3:8.1f} us  {nbytes/ms/1e6:8.1f} GB/s ({nbytes/ms/1e6/HBM_PEAK_GBS*100:5.1f}%)")

    for name in Chain.NEXT_OPS:
        rec(name, chain.op(name), chain.next_bytes(name))
    chain._next = None
    mp = (T + 63) // 64 * 64
    # N2's GEMM half on the matrix cores (f16 operands, f32 sums), config-5
    # tokens: the qkv linear alone, the MLP's first linear with GELU-tanh in
    # its store, and the qkv linear fused with the attention epilogue and the
    # head-major pack (RoPE from the phase table, built once per forward as
    # the reference does); hipBLASLt (torch.matmul) + the separate pack beside
    # them.
    def rec_f(name, fn, flops):
        fn()
        ms = time_region(torch, fn, reps) / reps
        tf = flops / ms / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "flops": flops, "tflops": round(tf, 1),
                     "pct_of_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS * 100, 2)}
        log(f"  {name:<26s} {ms*1e3:8.1f} us  {tf:8.1f} TFLOP/s ({tf/MFMA_F16_PEAK_TFLOPS*100:5.1f}% of f16 MFMA)")

    g = torch.Generator(device=dev).manual_seed(9)
    wqkv = (torch.randn((3 * C, C), generator=g, device=dev) * 0.02).to(torch.float16)
    w1 = (torch.randn((chain.F, C), generator=g, device=dev) * 0.02).to(torch.float16)
    xg = chain.x
    out = torch.empty((T, chain.F), dtype=torch.float16, device=dev)
    fq = 2.0 * T * 3 * C * C
    rec_f("linear_qkv", lambda: ops.linear(xg, wqkv, out=out[:, :3 * C]), fq)
    rec_f("linear_fc1_gelu", lambda: ops.linear(xg, w1, bias=chain.bias, act=ops.ACT_GELU_TANH, out=out),
          2.0 * T * chain.F * C)
    ph = ops.rope_phases(T, D, chain.freqs, coords=chain.coords, device=dev)
    bq = chain.bias[:3 * C]
    for kt in (True, False):
        rec_f(f"qkv_linear_pack_k{'t' if kt else 'rows'}",
              lambda kt=kt: ops.qkv_linear_pack(xg, wqkv, H, bias=bq, gamma_q=chain.gq, gamma_k=chain.gk, mp=mp,
                                                lp=mp, freqs=chain.freqs, phases=ph, k_transposed=kt), fq)
    qkv = out[:, :3 * C].contiguous()
    q3 = qkv.reshape(T, 3, H, D)
    b3 = bq.reshape(3, H * D)

    def hipblaslt_then_pack():
        torch.matmul(xg, wqkv.t(), out=qkv)
        ops.attn_pack(q3[:, 0], q3[:, 1], q3[:, 2], mp=mp, lp=mp, bias_q=b3[0], bias_k=b3[1], bias_v=b3[2],
                      gamma_q=chain.gq, gamma_k=chain.gk, freqs=chain.freqs, phases=ph, k_transposed=True)

    rec_f("hipblaslt_qkv", lambda: torch.matmul(xg, wqkv.t(), out=qkv), fq)
    rec_f("hipblaslt_qkv_then_pack_kt", hipblaslt_then_pack, fq)
    del wqkv, w1, out, ph, qkv, q3
    # the MLP's second linear with the gated residual join in its store
    # (x += (h + bias) * gate[b]), against hipBLASLt + the separate join
    w2 = (torch.randn((C, chain.F), generator=g, device=dev) * 0.02).to(torch.float16)
    hmid = torch.empty((T, C), dtype=torch.float16, device=dev)
    f2 = 2.0 * T * C * chain.F
    rec_f("linear_fc2_gate_residual",
          lambda: ops.linear_gate_residual(chain.u, w2, chain.x, bias=chain.bias[:C], gate=chain.gate,
                                           offsets=chain.offsets, out=chain.res), f2)

    def hipblaslt_fc2_then_join():
        torch.matmul(chain.u, w2.t(), out=hmid)
        ops.gate_residual(chain.x, hmid, gate=chain.gate, bias=chain.bias[:C], offsets=chain.offsets, out=chain.res)

    rec_f("hipblaslt_fc2_then_gate_residual", hipblaslt_fc2_then_join, f2)
    del w2, hmid
    return res


def small_chain(torch, dev, tokens, steps):
    """The config-5 chain (same ops, widths, f16) over one sparse batch of
    `tokens` random voxels of the 128^3 grid: 2,369 is the structured-latent
    DiT's token count in the reference's 512 pipeline. Launched eagerly back to
    back (a GPU spin ahead lets the host enqueue every launch first) and as
    one HIP graph of `steps` chain steps."""
    ch = Chain(dev, torch.float16, tokens)
    for _ in range(3):
        ch.step()
    torch.cuda.synchronize()
    torch.cuda._sleep(steps * 100_000)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(steps):
        ch.step()
    s1.record()
    torch.cuda.synchronize()
    eager = s0.elapsed_time(s1) / steps
    graph = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ch.step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=st):
            for _ in range(steps):
                ch.step()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph.replay()
    replay = time_region(torch, graph.replay, 3) / 3 / steps
    del graph
    res = {"tokens": tokens, "bytes": ch.chain_bytes}
    for k, ms in (("eager", eager), ("graph", replay)):
        gbs = ch.chain_bytes / ms / 1e6
        res[k] = {"us_per_step": round(ms * 1e3, 2), "gbs": round(gbs, 1), "pct_of_peak": round(gbs / HBM_PEAK_GBS * 100, 2),
                  "tokens_per_s": round(tokens / ms * 1e3)}
        log(f"  T={tokens} {k}: {ms*1e3:.1f} us/step, {gbs:.1f} GB/s ({gbs/HBM_PEAK_GBS*100:.1f}%), "
            f"{tokens/ms/1e3:.1f} M tokens/s")
    del ch
    torch.cuda.empty_cache()
    return res


def chain_sweep(torch, dev, steps):
    """The config-5 chain (same ops, widths and f16 storage) at token counts
    from the dense sparse-structure grid (4,096) to 2.6x config 5, one batch
    of random voxels each: how the chain's HBM efficiency grows with T.
    GPU time of n back-to-back steps enqueued behind a GPU spin. Prints one
    JSON line."""
    res = {}
    for tokens in (4096, 16384, 65536, 201436, 524288):
        ch = Chain(dev, torch.float16, tokens)
        for _ in range(3):
            ch.step()
        n = max(20, min(steps, int(2e5 // tokens) * 10))
        # a GPU spin ahead of the window lets the host enqueue every launch
        # first: at small T one Python call of an op takes longer than its
        # kernel, and the window would time the host
        torch.cuda.synchronize()
        torch.cuda._sleep(n * 150_000)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(n):
            ch.step()
        s1.record()
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / n
        gbs = ch.chain_bytes / ms / 1e6
        res[str(tokens)] = {"us_per_step": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                            "pct_peak": round(gbs / HBM_PEAK_GBS * 100, 2), "tokens_per_s": round(tokens / ms * 1e3)}
        log(f"  T={tokens:>7d}  {ms*1e3:9.1f} us/step  {gbs:8.1f} GB/s ({gbs/HBM_PEAK_GBS*100:5.1f}%)  "
            f"{tokens/ms/1e3:8.1f} M tokens/s")
        del ch
        torch.cuda.empty_cache()
    print(json.dumps({"chain_sweep": res, "bytes_per_token": 52240}), flush=True)


# The sources each chain op's kernel is built from (its launcher included).
TRAFFIC_SOURCES = {
    "ln_modulate": ["t2h_norm.hip"],
    "qk_rmsnorm_rope": ["t2h_qk.hip", "t2h_rope.h"],
    "gelu_tanh_bias": ["t2h_eltwise.hip"],
    "gate_residual": ["t2h_eltwise.hip"],
}
TRAFFIC_COMMON = ["t2h_device.h", "t2h_internal.h"]


def traffic_sources_sha(op):
    """sha256 over the csrc files `op`'s kernel is built from, in a fixed order."""
    import hashlib

    h = hashlib.sha256()
    for f in TRAFFIC_SOURCES[op] + TRAFFIC_COMMON:
        with open(os.path.join(ROOT, "trellis2-mojo_amd", "csrc", f), "rb") as fh:
            h.update(f.encode() + b"\0" + fh.read())
    return h.hexdigest()


def measured_traffic(op, path=None):
    """(HBM bytes per launch of `op` from profiles/traffic_c5.json, stale).
    The file records the sources' sha256 at measurement time; when the
    kernel's sources differ now, the figure belongs to another build and
    is not reported (None, True)."""
    path = path or os.path.join(ROOT, "profiles", "traffic_c5.json")
    try:
        rec = json.load(open(path))
    except (OSError, ValueError):
        return None, False
    if op not in rec:
        return None, False
    if rec.get("_sources_sha256", {}).get(op) != traffic_sources_sha(op):
        return None, True
    return rec[op], False


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (the per-token ops are row-"
              f"independent: each GPU would take a contiguous range of rows, with no exchange). "
              f"Got --gpus {args.gpus}.", file=sys.stderr)
        sys.exit(2)
    import torch

    from t2h import ops

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    ops.device_init(0)
    if args.sweep:
        chain_sweep(torch, dev, args.steps)
        return
    if args.small_t:
        small = small_t_block(torch, dev, max(20, args.steps))
        slat = small_chain(torch, dev, 2369, max(200, args.steps))
        print(json.dumps({"small_t_block": small, "slat_chain": slat}), flush=True)
        return
    if args.configs_only:
        log("BASELINE configs 1-4 (median of 30, warm / cold = caches flushed by a 1 GiB fill):")
        print(json.dumps({"configs": other_configs(torch, dev, cpu=not args.no_cpu)}), flush=True)
        return
    dtype = torch.float16
    chain = Chain(dev, dtype)
    log(f"config5: T={chain.T} tokens, chain bytes {chain.chain_bytes/1e9:.3f} GB/step")

    if args.op:  # one op (or "chain") only, for profiler runs
        fn = chain.op(args.op)
        for _ in range(args.warmup):
            fn()
        ms = time_region(torch, fn, args.steps)
        if args.op in chain.GEMM_OPS:
            tf = chain.gemm_flops(args.op) / (ms / args.steps) / 1e9
            log(f"{args.op}: {ms/args.steps*1e3:.1f} us/launch, {tf:.1f} TFLOP/s")
            return
        nb = chain.chain_bytes if args.op == "chain" else (
            chain.next_bytes(args.op) if args.op in chain.NEXT_OPS else chain.bytes[args.op])
        log(f"{args.op}: {ms/args.steps*1e3:.1f} us/launch, {nb/(ms/args.steps)/1e6:.1f} GB/s")
        return

    # The first timed event pair of a process sets up the runtime's timestamp
    # machinery (~50 ms, the GPU idle, in a kernel trace of a fresh process);
    # done here, before the warm-up, that idle does not fall between the
    # warm-up and the timed steps.
    time_region(torch, lambda: None, 1)
    for _ in range(args.warmup):
        chain.step()
    torch.cuda.synchronize()
    ms = time_region(torch, chain.step, args.steps)
    ms_step = ms / args.steps
    gbs = chain.chain_bytes / ms_step / 1e6
    tok_s = chain.T / ms_step * 1e3
    log(f"chain: {ms_step*1e3:.1f} us/step, {gbs:.1f} GB/s ({gbs/HBM_PEAK_GBS*100:.1f}% of peak), "
        f"{tok_s/1e6:.1f} M tokens/s")

    # The same chain once the GPU has left its idle clocks: the first tens of
    # milliseconds of load after a process starts run a few percent slower
    # (kernel traces of a fresh process show every kernel of the first steps
    # longer), so the window above can carry that ramp. The chain runs
    # untimed for settle_ms of GPU time, then one window is timed whole
    # (steady) and one with an event pair around every op (in-chain per-op
    # durations; the events add a little to that window only).
    # five interleaved rounds: the leave-one-out differences are ~0.3 % of a window each
    steady = steady_state(torch, chain, args.settle_ms, max(args.steps, 30), rounds=5)
    per_op = steady["per_op"]
    log(f"steady state after {steady['settle_ms']:.0f} ms of chain steps: {steady['us_per_step']:.1f} us/step, "
        f"{steady['gbs']:.1f} GB/s ({steady['pct_of_peak']:.1f}%); in-chain per-op sum "
        f"{steady['per_op_sum_us']:.1f} us (event pairs: {steady['per_op_events_sum_us']:.1f} us)")
    for n, v in per_op.items():
        rate = f"{v['gbs']:8.1f} GB/s ({v['pct_of_peak']:5.1f}%)" if v["gbs"] is not None else "   (within the windows' noise)"
        log(f"  in chain {n:<18s} {v['us']:8.1f} us  {rate}  event pair {steady['per_op_events'][n]['us']:8.1f} us")
    # each op repeated on its own (same stream, same buffers), for comparison
    alone = {}
    for n in Chain.ORDER:
        fn = chain.op(n)
        fn()
        reps = max(10, args.steps)
        t_ms = time_region(torch, fn, reps) / reps
        alone[n] = {"us": round(t_ms * 1e3, 2), "gbs": round(chain.bytes[n] / t_ms / 1e6, 1)}
    dom = "gelu_tanh_bias"
    dom_ev = steady["per_op_events"][dom]
    ach = chain.bytes[dom] / dom_ev["us"] * 1e-3
    traffic, stale = measured_traffic(dom)
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom,
                "bytes_per_launch": chain.bytes[dom], "launch_us": dom_ev["us"],
                "timing": "mean in-chain launch between the HIP events around it on the launch stream, in the "
                          "steady-state window (the interval includes one event-record gap)"}
    if stale:
        roofline["traffic_stale"] = True
        log(f"roofline.traffic: profiles/traffic_c5.json was measured on other {dom} sources; reported as null")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(chain, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.0f} tokens/s on {cpu['cores']} threads ({cpu['sample']}); all cores "
            f"{cpu['all_cores']['value']:.0f} tokens/s; nproc {cpu['nproc']}, usable {cpu['usable_cpus']}, "
            f"{cpu['cpu_model']}")
    log("next rows on the config-5 rows (f16):")
    extra = next_rows(torch, dev, chain, max(10, args.steps))
    log("small-T block (dense sparse-structure DiT, 4096 tokens):")
    small = small_t_block(torch, dev, max(20, args.steps))
    log("the chain at the SLat token count (one sparse batch of 2,369 tokens):")
    slat = small_chain(torch, dev, 2369, max(200, args.steps))
    other = None
    if not args.no_configs:
        log("BASELINE configs 1-4 (median of 30, warm / cold = caches flushed by a 1 GiB fill):")
        other = other_configs(torch, dev)

    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "tokens_per_s": round(tok_s, 0), "pct_of_peak": round(gbs / HBM_PEAK_GBS * 100, 2),
        "config": {"workload": "BASELINE config 5: per-block chain timestep-embed -> LN+adaLN modulate -> "
                               "QK RMSNorm+3D RoPE (int coords) -> GELU-tanh+bias -> gated residual, "
                               "f16 storage / f32 math",
                   "tokens": chain.T, "width": 1536, "heads": 12, "head_dim": 128, "hidden": 6144,
                   "grid": "128^3 thickened sphere shell", "bytes_per_token": 52240},
        "steady_state": {k: v for k, v in steady.items() if k not in ("per_op", "per_op_events")},
        "per_op": per_op,
        "per_op_events": steady["per_op_events"],
        "per_op_alone": alone,
        "next_rows": extra,
        "roofline": roofline,
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample",
                                                                      "all_cores", "nproc", "usable_cpus",
                                                                      "cpu_model")},
        "configs": other,
        "small_t_block": small,
        "slat_chain": slat,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
