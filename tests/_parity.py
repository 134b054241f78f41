"""Helpers shared by the parity tests.

Error metric for floating-point parity (written out in every assertion):
    err_i = |gpu_i - oracle_i| / max(|oracle_i|, 1)
i.e. relative error for |oracle| >= 1 and absolute error below 1 (where a
relative error is undefined near zero). Tolerances:
    f32 storage          1e-5
    f16 storage          2e-3   (oracle = f32 math on the f16-rounded inputs)
    bf16 storage         8e-3   (2 bf16 ulp; not a north-star dtype)
Integer / index / gather work and the ops whose f32 arithmetic has no
transcendental or reduction (modulate, gated residual, binop) are compared
bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle as orc

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 8e-3}


def max_err(got, want) -> float:
    if isinstance(got, torch.Tensor):
        got = got.detach().float().cpu().numpy()
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.size == 0:
        return 0.0
    assert np.all(np.isfinite(got)), "non-finite output"
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)))


def assert_close(got, want, dtype, what=""):
    tol = TOL[dtype]
    e = max_err(got, want)
    assert e <= tol, f"{what}: max err {e:.3e} > {tol:g}"
    return e


def storage_round(x: np.ndarray, dtype) -> np.ndarray:
    """What storing x in `dtype` and reading it back yields (f32 array)."""
    if dtype == torch.float32:
        return np.asarray(x, np.float32)
    if dtype == torch.float16:
        return orc.round_f16(x)
    return orc.round_bf16(x)


def to_dev(x: np.ndarray, dev, dtype=torch.float32) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(dev).to(dtype) if t.dtype.is_floating_point else t.to(dev)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bits_equal(got: torch.Tensor, want_f32: np.ndarray, dtype) -> bool:
    """Bit-exact comparison of a device tensor of `dtype` with the oracle's
    f32 result rounded once to `dtype`."""
    w = torch.from_numpy(np.ascontiguousarray(want_f32, np.float32)).to(dtype)
    g = got.detach().cpu()
    return bool(torch.equal(g.view(torch.int16) if dtype != torch.float32 else g.view(torch.int32),
                            w.view(torch.int16) if dtype != torch.float32 else w.view(torch.int32)))
