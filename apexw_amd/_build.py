"""Build libapexw_hip.so (hipcc, gfx950) and the _host module (g++) in-tree.

    python -m apexw_amd._build            # or __graft_entry__.build()

All HIP sources under apexw_amd/csrc are compiled (one hipcc per file, in
parallel) and linked into one shared library next
to this file.  csrc/host.cpp (the per-step scan of a plan's tensors, plain
CPython C API over torch's tensor headers) becomes apexw_amd/_host*.so.
HIP flags:
  -O3 --offload-arch=gfx950        CDNA4 code objects only
  -ffp-contract=off                no implicit FMA: kernels write fmaf() exactly
                                   where the reference's torch ops fuse
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                   keep packed fp32 instructions out of the code
"""

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB_NAME = "libapexw_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


OBJ_DIR = os.path.join(HERE, "_objs")   # per-source objects (git- and gpurun-ignored)
HOST_SRC = os.path.join(CSRC, "host.cpp")
HOST_PATH = os.path.join(HERE, "_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=False):
    """Compile the HIP library and the host module (always rebuilds both)."""
    build_host(verbose)
    return build_hip(verbose)


def build_host(verbose=False):
    """Compile csrc/host.cpp against the installed torch into apexw_amd/_host*.so."""
    import torch
    from torch.utils import cpp_extension as ce
    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = HOST_PATH + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *(f"-I{p}" for p in ce.include_paths()), f"-I{sysconfig.get_paths()['include']}", HOST_SRC,
           f"-L{os.path.join(tdir, 'lib')}", "-ltorch_python", "-ltorch", "-ltorch_cpu", "-lc10",
           f"-Wl,-rpath,{os.path.join(tdir, 'lib')}", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, HOST_PATH)
    return HOST_PATH


def _compile_one(src, obj, verbose):
    cmd = [HIPCC, *FLAGS, "-c", "-I", os.path.join(ROOT, "include"), "-o", obj, src]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, res.returncode, errs


def build_hip(verbose=False):
    """Compile every HIP source (one hipcc per file, in parallel) and link
    apexw_amd/libapexw_hip.so."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s) + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda so: _compile_one(so[0], so[1], verbose), zip(srcs, objs)))
    for src, rc, errs in results:
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({rc}):\n{errs}")
        if verbose and errs.strip():
            print(errs, file=sys.stderr)
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
