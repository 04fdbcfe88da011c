"""Build libapexw_hip.so in-tree with hipcc for gfx950.

    python -m apexw_amd._build            # or __graft_entry__.build()

All HIP sources under apexw_amd/csrc are compiled into one shared library next
to this file.  Flags:
  -O3 --offload-arch=gfx950        CDNA4 code objects only
  -ffp-contract=off                no implicit FMA: kernels write fmaf() exactly
                                   where the reference's torch ops fuse
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                   keep packed fp32 instructions out of the code
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB_NAME = "libapexw_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=False):
    """Compile every HIP source into apexw_amd/libapexw_hip.so (always rebuilds)."""
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
