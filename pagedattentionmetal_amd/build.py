"""Build libpam.so (HIP kernels for gfx950 + C++ runtime + C ABI) in-tree.

``python -m pagedattentionmetal_amd.build`` or ``build()`` compiles every source
under ``csrc/`` with hipcc into ``_build/`` and links
``pagedattentionmetal_amd/libpam.so``.  hipcc cross-compiles for gfx950 on a host
without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpam.so")
ARCH = "gfx950"

# Packed FP32 VALU forms are disabled for all device code; hipcc's host pass
# warns that it does not know the feature, which is harmless.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# per-source additions: the backward kernels keep their MFMA results in VGPRs
# (with the default AGPR form the compiler copies every score tile out of AGPRs)
FILE_FLAGS = {"backward.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", f"--offload-arch={ARCH}",
          "-fvisibility=hidden"]


def sources():
    out = []
    for sub in ("kernels", "runtime"):
        d = os.path.join(CSRC, sub)
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".cpp")):
                out.append(os.path.join(d, f))
    return out


def _hipcc():
    h = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(h):
        raise RuntimeError("hipcc not found: libpam needs ROCm's hipcc to build")
    return h


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.relpath(src, CSRC).replace(os.sep, "_") + ".o")
    cmd = [_hipcc(), *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [_hipcc(), *COMMON, "-x", "hip", *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    noisy = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noisy:
        sys.stderr.write("\n".join(noisy) + "\n")
    return obj


MODULE_SRC = os.path.join(CSRC, "module", "module_entry.hip")
MODULE = os.path.join(HERE, "libpam_kernels.hsaco")


def _code_object() -> str:
    """libpam_kernels.hsaco: the kernels' named entries as a gfx950 code object
    (an ELF, not a bundle) for hipModuleLoad."""
    tmp = MODULE + ".tmp"
    cmd = [_hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "--cuda-device-only", "--no-gpu-bundle-output",
           *DEVICE_FLAGS, MODULE_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {MODULE_SRC}:\n{r.stderr}")
    os.replace(tmp, MODULE)
    return MODULE


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs) + 1, max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        module = ex.submit(_code_object)
        objs = list(ex.map(_compile, srcs))
        module.result()
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} and {MODULE}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
