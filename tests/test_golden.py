"""The C oracle reproduces the committed golden fixtures (tests/golden/
oracle_golden.npz, written by tests/golden/make_golden.py). Integer and
exact-rounding outputs must match bit for bit; outputs that go through libm
transcendentals (cos/sin/exp/tanh/erf/pow) within 2 ulp-scale tolerance."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

GOLDEN = os.path.join(HERE, "golden", "oracle_golden.npz")
EXACT = {"rng_u64_seed1337", "randn_seed42", "ln_x", "ln_w", "ln_b", "mod_x", "mod_shift", "mod_scale", "mod_out",
         "sp_coords", "sp_offsets", "sp_h", "sp_shift", "sp_scale", "sp_mod_out", "rms_x", "rms_gamma", "act_x",
         "act_relu", "gelu_bias_h", "gelu_bias_b", "gr_x", "gr_y", "gr_gate", "gr_out", "gr_bias", "gr_out_bias",
         "ts_t", "ln_eps1e-6", "ln_affine_eps1e-5", "rms_out"}


@pytest.fixture(scope="module")
def fresh():
    return make_golden.build()


def test_golden_keys(fresh):
    with np.load(GOLDEN, allow_pickle=False) as g:
        assert set(g.files) == set(fresh)


@pytest.mark.parametrize("key", sorted(np.load(GOLDEN, allow_pickle=False).files))
def test_golden_value(fresh, key):
    with np.load(GOLDEN, allow_pickle=False) as g:
        want = g[key]
    got = fresh[key]
    assert got.dtype == want.dtype and got.shape == want.shape
    if key in EXACT:
        assert np.array_equal(got, want), key
    else:
        np.testing.assert_allclose(got, want, rtol=3e-7, atol=3e-7, err_msg=key)
