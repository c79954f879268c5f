"""Build libmoehip.so (the HIP kernels and their C ABI) in-tree for gfx950.

    python -m distributedmoellm_amd.build

Each csrc/*.hip is compiled to an object in a temporary directory, all at
once (one hipcc process per source), then the objects are linked. Packed-FP32
instruction selection is switched off (-packed-fp32-ops) on purpose; hipcc's
host pass warns that it does not know the feature, which is harmless.
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmoehip.so"
ARCH = os.environ.get("MOEHIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    return "hipcc"


# per-source additions: the multi-row GEMM wants its MFMA results in VGPRs
# (the compiler's default puts them in AGPRs and copies them back one by one)
EXTRA_FLAGS = {"rows.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _messages(r) -> list[str]:
    return [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln and ln.strip()]


def build(verbose: bool = True) -> Path:
    """Compile every source into libmoehip.so (always recompiles)."""
    srcs = sources()
    t0 = time.time()
    with tempfile.TemporaryDirectory(prefix="moehip-") as tmpdir:
        objs = [Path(tmpdir) / (src.stem + ".o") for src in srcs]
        procs = [subprocess.Popen([hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)],
                                  stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
                 for src, obj in zip(srcs, objs)]
        failed = []
        for src, p in zip(srcs, procs):
            out, err = p.communicate()
            if p.returncode != 0:
                failed.append(src.name)
                sys.stderr.write("\n".join(_messages(subprocess.CompletedProcess(p.args, p.returncode, out, err)))
                                 + "\n")
        if failed:
            raise RuntimeError(f"hipcc failed on {', '.join(failed)} building {LIB.name}")
        tmp = LIB.with_suffix(".so.tmp")
        r = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
                           capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write("\n".join(_messages(r)) + "\n")
            raise RuntimeError(f"linking {LIB.name} failed ({r.returncode})")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build()
