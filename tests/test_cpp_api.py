"""The C++ operator interface (include/t2h.hpp), exercised by the compiled
test program tests/cpp/test_t2h_cpp (built by __graft_entry__.build() with
tests/cpp/Makefile): the reference's tests/parity/test_sparse_basic.mojo
cases and the oracle parity of each op, through the header's classes.

The CPU test runs the header's host-side checks: the f16 / bf16 storage
conversion against the oracle, and the argument errors raised before any
device call. The GPU test runs the whole program, one process, and reports
each case it ran."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "_build", "test_t2h_cpp")


def _binary() -> str:
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built: run __graft_entry__.build() (make -C tests/cpp)")
    return BINARY


def _build_if_missing() -> None:
    """On the CPU, build the program (and the two libraries it links) when a
    fresh tree has none, as the other CPU tests do for libt2h and the oracle."""
    if os.path.exists(BINARY):
        return
    import oracle as orc
    from t2h import _build

    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    orc.build()
    subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True, stdout=subprocess.PIPE,
                   stderr=subprocess.STDOUT)


def _run(args, timeout):
    p = subprocess.run([_binary(), *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout)
    print(p.stdout, flush=True)
    return p


def test_cpp_header_host_conversions():
    _build_if_missing()
    p = _run(["--host"], 60)
    assert p.returncode == 0, p.stdout[-2000:]
    assert "ok host_f16_conversion" in p.stdout and "ok host_errors" in p.stdout


@pytest.mark.gpu
def test_cpp_operator_interface(dev):
    p = _run([], 100)
    assert p.returncode == 0, p.stdout[-4000:]
    assert "FAIL" not in p.stdout
    assert "19 of 19 passed" in p.stdout
