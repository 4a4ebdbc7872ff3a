"""Build recipe for ``logo_amd/liblogo_hip.so`` (gfx950 only) and its
PyTorch operator shim ``logo_amd/_logo_torch.so``.

Compiles every ``csrc/*.hip`` and ``csrc/*.cpp`` with ``hipcc`` into one
C-ABI shared library next to this file.  Packed-FP32 instructions are disabled
for all device code (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
Then compiles ``torch_ops/logo_torch_ops.cpp`` (host code only: the
``TORCH_LIBRARY(logo_hip)`` registration over the C entry points) against the
installed PyTorch, linked to ``liblogo_hip.so`` beside it.

Usage: ``python -m logo_amd.build`` (or ``__graft_entry__.build()``).
"""

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liblogo_hip.so")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results the VALU reads (S, dP) stay in VGPRs instead of AGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-result",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def sources():
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, name))
    return out


TORCH_SHIM_SRC = os.path.join(HERE, "torch_ops", "logo_torch_ops.cpp")
TORCH_SHIM = os.path.join(HERE, "_logo_torch.so")


def build_torch_shim(verbose: bool = False) -> str:
    """Compile the TORCH_LIBRARY shim (host C++) into ``_logo_torch.so``."""
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    for inc in include_paths():
        cmd += ["-I", inc]
    cmd += ["-I", "/opt/rocm/include", TORCH_SHIM_SRC]
    for lib_dir in library_paths():
        cmd += ["-L", lib_dir]
    cmd += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-L", "/opt/rocm/lib", "-lamdhip64",
            "-L", HERE, "-llogo_hip",
            "-Wl,-rpath,$ORIGIN", "-o", TORCH_SHIM + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch shim build failed:\n{res.stderr}")
    os.replace(TORCH_SHIM + ".tmp", TORCH_SHIM)
    return TORCH_SHIM


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compile all sources and link ``liblogo_hip.so``; returns its path."""
    hipcc = _hipcc()
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="logo_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc, *COMMON_FLAGS, "-I", os.path.join(HERE, "..", "include"), "-c", src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
            return obj

        with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
            objs = list(ex.map(compile_one, srcs))
        tmp_lib = LIB + ".tmp"
        cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp_lib]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        os.replace(tmp_lib, LIB)
    build_torch_shim(verbose)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
