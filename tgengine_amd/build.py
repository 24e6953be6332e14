"""Build libtgx.so (HIP, gfx950) in-tree with hipcc.

``python -m tgengine_amd.build`` or ``tgengine_amd.build.build()``.  The library
lands in ``tgengine_amd/_lib/libtgx.so`` so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libtgx.so"
SOURCES = ["tgx_common.hip", "tgx_ring.hip", "tgx_recent.hip", "tgx_csr.hip", "tgx_negpool.hip"]

ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # no packed-FP32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep every fp32/fp64 rounding of the time encoding explicit
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtgx)")


def build_host(verbose: bool = False) -> Path:
    """The torch extension `tgengine_amd._tgx_host` (host glue, plain g++), linked
    against libtgx.so through an $ORIGIN rpath."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension as ce
    out = PKG / ("_tgx_host" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_suffix(".tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-shared", "-fPIC", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_tgx_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in ce.include_paths()], f"-I{sysconfig.get_paths()['include']}",
           # torch's HIP stream API (the caller's current stream); host code only
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
           f"-I{INCLUDE}", str(CSRC / "tgx_host.cpp"), "-o", str(tmp),
           *[f"-L{p}" for p in ce.library_paths()], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-L{OUT_DIR}", "-ltgx", "-Wl,-rpath,$ORIGIN/_lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host glue build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        noisy = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if verbose and noisy:
            print("\n".join(noisy), file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_host(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
