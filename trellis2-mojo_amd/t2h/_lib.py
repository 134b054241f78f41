"""ctypes binding of libt2h.so (include/t2h.h).

The library is loaded once, after torch (so torch's HIP runtime — SONAME
libamdhip64.so.7 — is the one the library binds to and device pointers are
shared). There is no fallback: if the library is missing every op raises.
"""
from __future__ import annotations

import ctypes
import os

from ._build import LIB_PATH

c_i32, c_i64, c_f32, c_f64, c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p

# status codes / constants mirrored from include/t2h.h
T2H_OK = 0
T2H_EINVAL = -1
T2H_EUNSUPPORTED = -2
T2H_EHIP = -3
T2H_EBATCH_ORDER = -4
T2H_EBATCH_RANGE = -5
T2H_EDEVICE = -6
F32, F16, BF16 = 0, 1, 2
LN_PLAIN, LN_MODULATE, LN_AFFINE = 0, 1, 2

# (name, argtypes); every entry point returns int32 status
_SIGNATURES = {
    "t2h_device_init": [c_i32],
    "t2h_ln_modulate": [c_p, c_p, c_i64, c_i32, c_i32, c_f32, c_i32, c_p, c_p, c_i64, c_p, c_i32, c_i64, c_p],
    "t2h_modulate": [c_p, c_p, c_i64, c_i32, c_i32, c_p, c_p, c_i64, c_p, c_i32, c_i64, c_p],
    "t2h_binop_rows": [c_p, c_p, c_p, c_i64, c_i32, c_i32, c_i32, c_i32, c_p, c_i32, c_i64, c_p],
    "t2h_qk_rmsnorm_rope": [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_p,
                            c_i32, c_p, c_i32, c_i32, c_p, c_i64, c_p, c_i32, c_i32, c_p],
    "t2h_qkv_bias_rmsnorm_rope": [c_p, c_i64, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_i32, c_p, c_i32, c_i32, c_p,
                                  c_i64, c_p, c_i32, c_i32, c_p],
    "t2h_attn_pack": [c_p, c_p, c_p, c_i64, c_i64, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_p, c_p, c_i32, c_p, c_i32,
                      c_i32, c_p, c_i64, c_p, c_i32, c_i32, c_p, c_i64, c_p, c_p, c_i64, c_i32, c_p],
    "t2h_rope_freqs": [c_i32, c_i32, c_f64, c_f64, c_p, c_i32],
    "t2h_rope_phases": [c_p, c_i64, c_i32, c_p, c_i32, c_i32, c_p, c_p, c_i32, c_i32, c_p],
    "t2h_activation": [c_p, c_p, c_p, c_i64, c_i32, c_i32, c_i32, c_p],
    "t2h_qkv_linear_pack": [c_p, c_i64, c_p, c_i64, c_i32, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_p, c_p, c_i32, c_p,
                            c_i32, c_i32, c_p, c_i64, c_p, c_i32, c_i32, c_p, c_i64, c_p, c_p, c_i64, c_i32, c_p],
    "t2h_linear_gate_residual": [c_p, c_i64, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_p, c_i64,
                                 c_p, c_i32, c_i64, c_p],
    "t2h_linear": [c_p, c_i64, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_p],
    "t2h_gate_residual": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_i32, c_p, c_i32, c_i64, c_p],
    "t2h_gate_residual_ln_modulate": [c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_f32, c_i32, c_p, c_p, c_i64, c_i64,
                                      c_i32, c_i32, c_p, c_i32, c_i64, c_p],
    "t2h_timestep_embedding": [c_p, c_p, c_i64, c_i32, c_i32, c_f64, c_p],
    "t2h_coords_to_offsets": [c_p, c_i64, c_i32, c_i32, c_p, c_p, c_p],
    "t2h_modulation_add": [c_p, c_p, c_p, c_i64, c_i64, c_p],
    "t2h_flow_euler_step": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_f64, c_f64, c_f64, c_f64, c_f64, c_p,
                            c_i32, c_p, c_i64, c_p],
    "t2h_flow_euler_step_noalloc": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_f64, c_f64, c_f64, c_f64, c_f64,
                                    c_p, c_i32, c_p],
    "t2h_ln_mod_rows": [c_p, c_p, c_p, c_i64, c_i32, c_i32, c_i32, c_i32, c_p],
    "t2h_gate_add_bias_rows": [c_p, c_p, c_p, c_i64, c_i32, c_i32, c_i32, c_i32, c_p],
    "t2h_block_join_ln": [c_p, c_p, c_p, c_p, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_p],
    "t2h_h_ln_modulate": [c_p, c_p, c_i64, c_i32, c_f32, c_i32, c_p, c_p, c_p, c_i32, c_i64],
    "t2h_h_qk_rmsnorm_rope": [c_p, c_p, c_p, c_p, c_i64, c_i32, c_i32, c_p, c_p, c_i32, c_p, c_i32, c_i32, c_p,
                              c_i64, c_p, c_i32, c_i32],
    "t2h_h_activation": [c_p, c_p, c_p, c_i64, c_i32, c_i32],
    "t2h_h_gate_residual": [c_p, c_p, c_p, c_p, c_p, c_i64, c_i32, c_p, c_i32, c_i64],
    "t2h_h_timestep_embedding": [c_p, c_p, c_i64, c_i32, c_f64],
    "t2h_h_coords_to_offsets": [c_p, c_i64, c_i32, c_i32, c_p],
}
EXPORTED = ["t2h_version", "t2h_last_error", "t2h_flow_euler_workspace", *_SIGNATURES]

_lib = None


class T2HError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg or f"t2h error {code}")
        self.code = code


def load(path: str | None = None):
    """Load libt2h.so (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (bind to torch's HIP runtime first)
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"libt2h.so not found at {path}: run __graft_entry__.build() first")
    L = ctypes.CDLL(path)
    L.t2h_version.restype = c_i32
    L.t2h_version.argtypes = []
    L.t2h_last_error.restype = ctypes.c_char_p
    L.t2h_last_error.argtypes = []
    L.t2h_flow_euler_workspace.restype = c_i64
    L.t2h_flow_euler_workspace.argtypes = [c_i64, c_i64, c_i32]
    for name, args in _SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = c_i32
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != T2H_OK:
        msg = load().t2h_last_error().decode(errors="replace")
        if rc == T2H_EINVAL:
            raise ValueError(msg)
        raise T2HError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
