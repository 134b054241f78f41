"""t2h — MI355X (gfx950) fused per-token ops of TRELLIS.2's flow-matching DiT
blocks, behind the C ABI of libt2h.so (include/t2h.h).

    t2h.ops     tensor-level wrappers of every C-ABI entry point
    t2h.nn      mirror of the reference's dense op interface (LayerNorm32, ...)
    t2h.sparse  SparseTensor rows: batch-gathered modulate / gate, sparse RoPE

All compute runs in libt2h's HIP kernels; nothing here falls back to CPU or
PyTorch math.
"""
from . import _lib, nn, ops, sparse  # noqa: F401
from ._build import LIB_PATH, build  # noqa: F401
from ._lib import T2HError  # noqa: F401

__all__ = ["ops", "nn", "sparse", "build", "LIB_PATH", "T2HError"]
