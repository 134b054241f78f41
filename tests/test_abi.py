"""C ABI checks that need no GPU: the library loads, exports every entry point
include/t2h.h declares, and rejects invalid arguments before touching the
device (no compute call is made here)."""
import ctypes
import os
import re

import numpy as np
import pytest

from t2h import _build, _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "t2h.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(t2h_\w+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in t2h.h but not exported"
    assert sorted(_lib.EXPORTED) == syms, "ctypes signature table out of sync with t2h.h"


def test_version(lib):
    assert lib.t2h_version() == 10000


def test_validation_without_device(lib):
    p = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    assert lib.t2h_ln_modulate(p, p, 4, 1536, 7, 1e-6, 0, None, None, 0, None, 1, 0, None) == _lib.T2H_EINVAL
    assert b"bad dtype" in lib.t2h_last_error()
    assert lib.t2h_ln_modulate(p, p, 4, 1536, 0, 1e-6, 1, None, None, 0, None, 1, 0, None) == _lib.T2H_EINVAL
    assert b"needs p0 and p1" in lib.t2h_last_error()
    assert lib.t2h_activation(p, p, None, 4, 8, 0, 9, None) == _lib.T2H_EINVAL
    assert lib.t2h_last_error() == b"unknown activation"
    assert lib.t2h_binop_rows(p, p, p, 4, 8, 3, 0, 0, None, 1, 0, None) == _lib.T2H_EINVAL
    assert b"incompatible row size" in lib.t2h_last_error()
    freqs = np.ones(21, np.float32)
    rc = lib.t2h_qk_rmsnorm_rope(p, p, p, p, 4, 0, 0, 12, 127, 0, None, None, None, None, 1,
                                 freqs.ctypes.data, 21, 3, None, 0, None, 0, 16, None)
    assert rc == _lib.T2H_EINVAL and b"head_dim must be even" in lib.t2h_last_error()
    rc = lib.t2h_qk_rmsnorm_rope(p, p, p, p, 4, 0, 0, 12, 128, 0, None, None, None, None, 1,
                                 freqs.ctypes.data, 21, 3, None, 0, None, 0, 0, None)
    assert rc == _lib.T2H_EINVAL and b"needs phases, coords or grid_res" in lib.t2h_last_error()
    rc = lib.t2h_timestep_embedding(p, p, 4, 4096, 0, 10000.0, None)
    assert rc == _lib.T2H_EUNSUPPORTED
    # resident-block glue: the reference kernels' mode / use_gate / offset domains
    assert lib.t2h_ln_mod_rows(p, p, p, 4, 1536, 0, 0, 0, None) == _lib.T2H_EINVAL
    assert b"bad mode 0" in lib.t2h_last_error()
    assert lib.t2h_gate_add_bias_rows(p, p, p, 4, 1536, -1, 1, 0, None) == _lib.T2H_EINVAL
    assert b"negative const offset" in lib.t2h_last_error()
    assert lib.t2h_gate_add_bias_rows(p, p, p, 4, 1536, 0, 2, 0, None) == _lib.T2H_EINVAL
    assert b"use_gate must be 0 or 1" in lib.t2h_last_error()
    assert lib.t2h_block_join_ln(p, p, p, None, 4, 1536, 0, 1, 0, 1, 0, None) == _lib.T2H_EINVAL
    assert b"NULL consts" in lib.t2h_last_error()
    assert lib.t2h_block_join_ln(p, p, p, p, 4, 1536, 0, 1, 0, 3, 0, None) == _lib.T2H_EINVAL
    assert b"bad mode 3" in lib.t2h_last_error()
    # attention pack: shape, padding and layout domains
    rc = lib.t2h_attn_pack(p, p, p, 0, 8, 4, 96, 0, None, None, None, None, None, 0, None, 0, 3, None, 0, None, 0,
                           0, p, 8, p, p, 8, 1, None)
    assert rc == _lib.T2H_EUNSUPPORTED and b"head_dim must be 64 or 128" in lib.t2h_last_error()
    rc = lib.t2h_attn_pack(p, p, p, 0, 8, 4, 128, 0, None, None, None, None, None, 0, None, 0, 3, None, 0, None, 0,
                           0, p, 4, None, None, 0, 1, None)
    assert rc == _lib.T2H_EINVAL and b"mp < rows" in lib.t2h_last_error()
    rc = lib.t2h_attn_pack(p, p, p, 0, 8, 4, 128, 0, None, None, None, None, None, 0, None, 0, 3, None, 0, None, 0,
                           0, None, 0, p, None, 12, 1, None)
    assert rc == _lib.T2H_EINVAL and b"lp % 8 == 0" in lib.t2h_last_error()


def test_empty_is_a_noop(lib):
    # rows == 0 returns before any device work
    assert lib.t2h_ln_modulate(None, None, 0, 1536, 0, 1e-6, 0, None, None, 0, None, 1, 0, None) == 0
    assert lib.t2h_activation(None, None, None, 0, 6144, 1, 3, None) == 0
    assert lib.t2h_gate_residual(None, None, None, None, None, 0, 0, 1536, 1, None, 1, 0, None) == 0
    p = ctypes.c_void_p(16)
    assert lib.t2h_gate_add_bias_rows(None, None, p, 0, 1536, 0, 1, 0, None) == 0
    assert lib.t2h_block_join_ln(None, None, None, p, 0, 1536, 2 * 1536, 1, 4 * 1536, 2, 1, None) == 0
    assert lib.t2h_last_error() == b""


def test_oracle_not_linked(lib):
    """The product library does not depend on the oracle."""
    import subprocess

    out = subprocess.run(["readelf", "-d", _build.LIB_PATH], stdout=subprocess.PIPE, text=True).stdout
    assert "oracle" not in out


def test_last_error_is_per_thread(lib):
    """t2h_last_error() is thread-local: each thread reads the message of its
    own last call, whatever the others did in between, and a successful call
    clears only its own thread's message."""
    import threading

    p = ctypes.c_void_p(16)
    n = 8
    barrier = threading.Barrier(n)
    results = {}

    def worker(i):
        if i % 2:
            rc = lib.t2h_activation(p, p, None, 4, 8, 0, 9, None)
            want = b"unknown activation"
        else:
            rc = lib.t2h_ln_modulate(p, p, 4, 1536, 7, 1e-6, 0, None, None, 0, None, 1, 0, None)
            want = b"bad dtype"
        barrier.wait()   # every thread has failed its call before any reads its message
        own = lib.t2h_last_error()
        barrier.wait()
        if i == 0:
            assert lib.t2h_activation(None, None, None, 0, 8, 0, 3, None) == 0   # rows 0: success
        barrier.wait()
        results[i] = (rc, own, lib.t2h_last_error(), want)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(n)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(results) == n
    for i, (rc, own, after, want) in results.items():
        assert rc == _lib.T2H_EINVAL and want in own, (i, own)
        assert after == (b"" if i == 0 else own), (i, after)
