"""Build recipe for libt2h.so (hipcc, gfx950 only).

Each csrc/*.hip translation unit is compiled in parallel, then linked into
lib/libt2h.so next to this package. The packed-FP32 target feature is turned
off for every HIP compile (the host pass warns that it does not know the
feature; that warning is filtered).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))   # trellis2-mojo_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
BUILD_DIR = os.path.join(PKG_ROOT, "_build")
LIB_DIR = os.path.join(PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libt2h.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", f"-I{INCLUDE}", f"-I{CSRC}",
]
_NOISE = "-packed-fp32-ops' is not a recognized feature"


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if _NOISE not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link lib/libt2h.so. Returns the path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in sources]
    with cf.ThreadPoolExecutor(max_workers=min(len(sources), 8)) as ex:
        futs = [ex.submit(_run, [HIPCC, *CFLAGS, "-c", s, "-o", o]) for s, o in zip(sources, objs)]
        logs = [f.result() for f in futs]
    tmp = LIB_PATH + ".tmp"
    # -z defs: an unresolved symbol (e.g. a kernel whose host stub was not
    # emitted) fails the link here instead of the first dlopen on a GPU box
    logs.append(_run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *objs, "-o", tmp]))
    os.replace(tmp, LIB_PATH)
    if verbose:
        print("\n".join(l for l in logs if l.strip()))
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
