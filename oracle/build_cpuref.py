"""Build oracle/libcpuref.so, the C/OpenMP restatement of the reference's numba
kernels (oracle/cpuref.c). TEST INFRASTRUCTURE: the CPU baseline and a cross-check.

-march=x86-64-v3 (AVX2 + FMA) so the library built here also runs on the GPU
machine's host; -ffast-math stands for numba's fastmath=True.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "cpuref.c"
LIB = HERE / "libcpuref.so"
FLAGS = ["-O3", "-march=x86-64-v3", "-ffast-math", "-fopenmp", "-shared", "-fPIC"]


def build(verbose: bool = True) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    r = subprocess.run(["gcc", *FLAGS, str(SRC), "-o", str(tmp), "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("gcc failed building libcpuref.so:\n" + r.stderr)
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def load():
    """ctypes handle of libcpuref.so with argument types set."""
    import ctypes
    from ctypes import c_int, c_void_p
    L = ctypes.CDLL(str(LIB))
    P, I = c_void_p, c_int
    sigs = {
        "ref_q4_matmul_t": [P, I, P, P, I, I, I, I, P],
        "ref_q8_matmul_t": [P, I, P, P, I, I, I, P],
        "ref_moe_q4": [P, I, P, P, P, P, P, I, I, I, I, I, P],
        "ref_mv_q8_0": [P, I, P, I, I, P],
        "ref_mv_q4_k": [P, I, P, I, I, P],
        "ref_threads": [],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = c_int if name == "ref_threads" else None
    return L


if __name__ == "__main__":
    build()
