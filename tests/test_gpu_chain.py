"""GPU parity on the headline workload itself: the chain
that bench.py times, on its own inputs.

T = 201,436 tokens of the 128^3 thickened shell (t2h.workloads.config5),
width 1536, 12 x 128 heads, hidden 6144, f16 storage, device offsets from
the coords, t * 1000 into the timestep embedding (samplers/flow_euler.mojo:
168). One `bench.Chain.step()` runs timestep embed -> LN + gathered modulate
-> QK RMSNorm + RoPE from the int coords -> GELU-tanh + bias -> gathered
gated residual (sparse/transformer/modulated.mojo:60-65, 214-226;
sparse/attention/rope.mojo:48-66; modules/nn.mojo:314-369, 588-647;
models/sparse_structure_flow.mojo:60-76). QK and GELU run in place, as the
reference's device kernels do; the fixture keeps a copy of each input from
before the step.

Every op is checked against the C oracle on sampled rows: the first and
last 8-row tiles, a middle tile, 6 more whole 8-row tiles, the rows with
the largest coordinate on each axis (angles up to 127 rad) and the largest
coordinate sum, and 32 seeded random rows. Whole-tensor properties on top:
the gated residual is bit-exact over all rows against single-rounding f32
steps, and RoPE keeps each pair's norm (RMS-only output vs RMS + RoPE
output). Metric and tolerances: tests/_parity.py (f16 storage: 2e-3, bf16:
8e-3). The chain runs in f16 (the benchmark's storage) and again in bf16.
"""
import numpy as np
import pytest
import torch

import oracle as orc
from _parity import assert_close, bits_equal, host, max_err, storage_round

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=[torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def chain(dev, request):
    import bench

    ch = bench.Chain(dev, request.param)
    ch.dt = request.param
    assert ch.qo.data_ptr() == ch.q.data_ptr() and ch.gout.data_ptr() == ch.u.data_ptr()
    ch.x_in, ch.q_in, ch.k_in, ch.u_in = (t.clone() for t in (ch.x, ch.q, ch.k, ch.u))
    ch.temb = ch.op("timestep")()
    ch.step()
    torch.cuda.synchronize()
    yield ch
    del ch
    torch.cuda.empty_cache()


def _sample_rows(coords):
    t = coords.shape[0]
    tiles = [0, t // 16, t // 8, (t // 2) // 8, (5 * t // 8) // 8, (7 * t // 8) // 8, (t - 1) // 8 - 1,
             (t - 1) // 8]
    rows = set()
    for k in tiles:
        rows.update(range(8 * k, min(8 * k + 8, t)))
    rows.update(range(t - 8, t))
    for ax in (1, 2, 3):
        rows.add(int(np.argmax(coords[:, ax])))
    rows.add(int(np.argmax(coords[:, 1:].sum(1))))
    rows.update(np.random.default_rng(5).integers(0, t, 32).tolist())
    return np.array(sorted(rows), np.int64)


def test_config5_shape_and_offsets(chain):
    coords = chain.coords_np
    assert chain.T == coords.shape[0] == 201436
    assert host(chain.offsets).astype(np.int64).tolist() == [0, chain.T]
    assert coords[:, 1:].max() <= 127 and coords[:, 1:].min() >= 0
    assert len(_sample_rows(coords)) >= 64


def test_config5_timestep(chain):
    t = host(chain.t)
    assert 0.0 <= t[0] <= 1000.0
    assert_close(chain.temb, orc.timestep_embedding(t, 256), torch.float32, "config-5 timestep embedding")


def test_config5_ln_modulate_sampled_rows(chain):
    idx = _sample_rows(chain.coords_np)
    x = host(chain.x_in[idx])
    want = orc.ln_modulate(x, host(chain.shift), host(chain.scale), eps=1e-6)
    assert_close(chain.h[idx], want, chain.dt, "config-5 LN + gathered modulate")


def test_config5_qk_rms_rope_sampled_rows(chain):
    idx = _sample_rows(chain.coords_np)
    ph = orc.rope_phases_from_coords(chain.coords_np[idx], chain.D, orc.rope_freqs(chain.D))
    wq, wk = orc.qk_rms_rope(host(chain.q_in[idx]), host(chain.k_in[idx]), host(chain.gq), host(chain.gk), ph)
    assert_close(chain.qo[idx], wq, chain.dt, "config-5 q RMS + RoPE")
    assert_close(chain.ko[idx], wk, chain.dt, "config-5 k RMS + RoPE")


def test_config5_rope_keeps_pair_norms(chain):
    """Over all T x 12 x 64 pairs: |RoPE(RMS(q))| per pair equals |RMS(q)|
    (a rotation), within the f16 storage tolerance."""
    from t2h import ops

    T, H, D = chain.T, chain.H, chain.D
    for src, gamma, out in ((chain.q_in, chain.gq, chain.qo), (chain.k_in, chain.gk, chain.ko)):
        rms = torch.empty_like(src)
        ops.qk_rmsnorm_rope(q=src, gamma_q=gamma, use_rope=False, q_out=rms)
        n_rope = out.float().reshape(T, H, D // 2, 2).square().sum(-1).sqrt()
        n_rms = rms.float().reshape(T, H, D // 2, 2).square().sum(-1).sqrt()
        err = ((n_rope - n_rms).abs() / n_rms.clamp(min=1.0)).max().item()
        tol = 2e-3 if chain.dt == torch.float16 else 8e-3
        assert err <= tol, f"pair norm changed by RoPE: {err:.3e}"
        del rms, n_rope, n_rms


def test_config5_gelu_sampled_rows(chain):
    idx = _sample_rows(chain.coords_np)
    want = orc.gelu_tanh_bias(host(chain.u_in[idx]), host(chain.bias))
    assert_close(chain.gout[idx], want, chain.dt, "config-5 GELU-tanh + bias")


def test_config5_gated_residual(chain):
    """Sampled rows vs the oracle, and every row bit-exact against
    x + fl(y * gate) in f32 (two separate single-rounding torch ops, the
    oracle's sequence) rounded once to the storage type."""
    idx = _sample_rows(chain.coords_np)
    want = orc.gate_residual(host(chain.x_in[idx]), host(chain.y[idx]), host(chain.gate),
                             offsets=np.array([0, len(idx)], np.int64))
    assert bits_equal(chain.res[idx], storage_round(want, chain.dt), chain.dt)
    T = chain.T
    for lo in range(0, T, 65536):
        hi = min(T, lo + 65536)
        prod = torch.mul(chain.y[lo:hi].float(), chain.gate)
        full = torch.add(chain.x_in[lo:hi].float(), prod).to(chain.dt)
        assert torch.equal(chain.res[lo:hi].view(torch.int16), full.view(torch.int16)), f"rows {lo}:{hi}"


def test_config5_max_err_report(chain):
    """The largest per-op error on the sampled rows stays inside the
    storage type's tolerance (printed for the record)."""
    idx = _sample_rows(chain.coords_np)
    x = host(chain.x_in[idx])
    e_ln = max_err(chain.h[idx], orc.ln_modulate(x, host(chain.shift), host(chain.scale), eps=1e-6))
    e_ge = max_err(chain.gout[idx], orc.gelu_tanh_bias(host(chain.u_in[idx]), host(chain.bias)))
    tol = 2e-3 if chain.dt == torch.float16 else 8e-3
    print(f"config-5 {chain.dt} max err: LN+mod {e_ln:.2e}, GELU {e_ge:.2e} (tol {tol:.0e})", flush=True)
    assert max(e_ln, e_ge) <= tol
