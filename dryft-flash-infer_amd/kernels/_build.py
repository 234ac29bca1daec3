"""Build ``libqlinear.so`` (the gfx950 C-ABI library) from ``csrc/*.hip`` with hipcc.

Every translation unit is compiled in parallel for gfx950 only, then linked into one
shared library next to this file. No torch types cross the ABI, so no torch headers
are involved. Run ``python -m kernels._build`` (with ``dryft-flash-infer_amd`` on
``sys.path``) or ``__graft_entry__.build()``.
"""

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
CSRC = os.path.join(PKG, "csrc")
OUT_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(HERE, "libqlinear.so")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # IEEE division and no contraction: the quantize kernels must round exactly as torch.
    "-ffp-contract=off",
    # Loadable by the HIP runtime bundled with the torch wheel as well as /opt/rocm.
    "-mcode-object-version=5",
    # No packed-fp32 instructions anywhere: some of their forms have given silently wrong
    # results on the MI355X boxes this library targets.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return path


def _compile(src):
    obj = os.path.join(OUT_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stderr[-4000:]}")
    return obj


def build(verbose=True, jobs=None):
    """Compile every csrc/*.hip for gfx950 and link kernels/libqlinear.so (always rebuilds)."""
    os.makedirs(OUT_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
