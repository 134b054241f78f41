"""Flow-matching Euler sampler on the MI355X path.

Mirror of FlowEulerSampler (trellis2_mojo/samplers/flow_euler.mojo:62-264):
sample / sample_cfg / sample_cfg_interval, with the velocity model passed as
a callable model(x_t, t1000, use_neg_cond) -> device tensor (the DiT is GEMM
and attention work outside this library). The per-step tensor math (CFG
combine, CFG rescale, Euler update, x_0 prediction) is one
t2h_flow_euler_step call; the step schedule and the guidance decisions stay
on the host, in float64, as in the reference.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import torch

from . import ops

GUIDANCE_NONE, GUIDANCE_CFG, GUIDANCE_CFG_INTERVAL = 0, 1, 2   # flow_euler.mojo:27-29

Model = Callable[[torch.Tensor, float, bool], torch.Tensor]


@dataclass
class SampleResult:
    """edict returned by FlowEulerSampler.sample (flow_euler.mojo:44-53)."""
    samples: torch.Tensor
    pred_x_t: List[torch.Tensor] = field(default_factory=list)
    pred_x_0: List[torch.Tensor] = field(default_factory=list)


def t_schedule(steps: int, rescale_t: float) -> List[float]:
    """np.linspace(1, 0, steps+1) rescaled: rescale_t*t / (1 + (rescale_t-1)*t)
    (flow_euler.mojo:195-198)."""
    out = []
    for i in range(steps + 1):
        t = 1.0 - float(i) / float(steps)
        out.append(rescale_t * t / (1.0 + (rescale_t - 1.0) * t))
    return out


class FlowEulerSampler:
    def __init__(self, sigma_min: float):
        self.sigma_min = float(sigma_min)
        self._ws: Optional[torch.Tensor] = None

    def _workspace(self, x: torch.Tensor, seg_offsets) -> torch.Tensor:
        rows = x.shape[0]
        need = ops.flow_euler_workspace(rows, x.numel() // max(rows, 1), len(seg_offsets) if seg_offsets else 0)
        if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
            self._ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        return self._ws

    def _step(self, model: Model, sample, t, t_prev, mode, g, lo, hi, gr, seg_offsets):
        """_inference (flow_euler.mojo:151-181) + the Euler update (206-210):
        the model calls, then one fused step call."""
        use_cfg = mode == GUIDANCE_CFG
        if mode == GUIDANCE_CFG_INTERVAL:
            use_cfg = lo <= t <= hi
        if not use_cfg or g == 1.0:
            pos, neg, g_eff = model(sample, 1000.0 * t, False), None, 1.0
        elif g == 0.0:
            pos, neg, g_eff = model(sample, 1000.0 * t, True), None, 1.0
        else:
            pos, neg, g_eff = model(sample, 1000.0 * t, False), model(sample, 1000.0 * t, True), g
        ws = self._workspace(sample, seg_offsets) if (neg is not None and gr > 0.0) else None
        return ops.flow_euler_step(sample, pos.contiguous(), t, t_prev, self.sigma_min,
                                   v_neg=None if neg is None else neg.contiguous(), guidance_strength=g_eff,
                                   guidance_rescale=gr, seg_offsets=seg_offsets or None, workspace=ws)

    def _sample_impl(self, model: Model, noise: torch.Tensor, steps: int, rescale_t: float, mode: int, g: float,
                     lo: float, hi: float, gr: float, seg_offsets: Optional[Sequence[int]]) -> SampleResult:
        sample = noise.clone()
        ts = t_schedule(steps, rescale_t)
        ret = SampleResult(noise.clone())
        for i in range(steps):
            sample, x0 = self._step(model, sample, ts[i], ts[i + 1], mode, g, lo, hi, gr,
                                    list(seg_offsets) if seg_offsets else None)
            ret.pred_x_t.append(sample)
            ret.pred_x_0.append(x0)
        ret.samples = sample
        return ret

    def sample(self, model: Model, noise: torch.Tensor, steps: int = 50, rescale_t: float = 1.0) -> SampleResult:
        """FlowEulerSampler.sample (no guidance)."""
        return self._sample_impl(model, noise, steps, rescale_t, GUIDANCE_NONE, 1.0, 0.0, 1.0, 0.0, None)

    def sample_cfg(self, model: Model, noise: torch.Tensor, steps: int = 50, rescale_t: float = 1.0,
                   guidance_strength: float = 3.0, guidance_rescale: float = 0.0,
                   seg_offsets: Optional[Sequence[int]] = None) -> SampleResult:
        """FlowEulerCfgSampler.sample."""
        return self._sample_impl(model, noise, steps, rescale_t, GUIDANCE_CFG, guidance_strength, 0.0, 1.0,
                                 guidance_rescale, seg_offsets)

    def sample_cfg_interval(self, model: Model, noise: torch.Tensor, steps: int = 50, rescale_t: float = 1.0,
                            guidance_strength: float = 3.0, interval_lo: float = 0.0, interval_hi: float = 1.0,
                            guidance_rescale: float = 0.0,
                            seg_offsets: Optional[Sequence[int]] = None) -> SampleResult:
        """FlowEulerGuidanceIntervalSampler.sample; seg_offsets marks a varlen
        state (per-segment biased std in the CFG rescale)."""
        return self._sample_impl(model, noise, steps, rescale_t, GUIDANCE_CFG_INTERVAL, guidance_strength,
                                 interval_lo, interval_hi, guidance_rescale, seg_offsets)
