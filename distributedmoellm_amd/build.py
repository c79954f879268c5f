"""Build libmoehip.so (the HIP kernels and their C ABI) in-tree for gfx950.

    python -m distributedmoellm_amd.build

One hipcc invocation over csrc/*.hip. Packed-FP32 instruction selection is
switched off (-packed-fp32-ops) on purpose; hipcc's host pass warns that it
does not know the feature, which is harmless.
"""

from __future__ import annotations

import os
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmoehip.so"
ARCH = os.environ.get("MOEHIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    return "hipcc"


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = True) -> Path:
    """Compile every source into libmoehip.so (always recompiles)."""
    srcs = sources()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *map(str, srcs), "-o", str(tmp)]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    errors = [ln for ln in (r.stdout + r.stderr).splitlines()
              if "packed-fp32-ops" not in ln and ln.strip()]
    if r.returncode != 0:
        sys.stderr.write("\n".join(errors) + "\n")
        raise RuntimeError(f"hipcc failed ({r.returncode}) building {LIB.name}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build()
