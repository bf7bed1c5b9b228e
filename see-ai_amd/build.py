"""Builds libseeai_hip.so, the gfx950 executor, in-tree.

Every .hip source under csrc/ and the host-side C ABI (capi.cpp) is compiled
with hipcc for gfx950 only and linked into ``see-ai_amd/libseeai_hip.so``.

Flags:
  -ffp-contract=off   the epilogue, optimizer and elementwise expressions
                      round where the reference's x86-64 build rounds them
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      keeps the compiler from forming packed-f32 VALU ops
                      (this pool's rule; the host pass warns it does not know
                      the feature, which is harmless)
  -mllvm -amdgpu-mfma-vgpr-form  (k_flash.hip, k_attn16.hip)
                      MFMA accumulators in VGPRs: the attention kernels run
                      VALU softmax on every score tile, and AGPR-resident
                      tiles cost a copy per element each way
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libseeai_hip.so")
PLANGEN_LIB = os.path.join(HERE, "libseeai_plangen.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


PER_FILE = {"k_flash.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
            "k_attn16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


# The host layer above the C ABI (plan reader, backend, engine): C++20,
# no device code.
ROCM = os.path.dirname(os.path.dirname(os.path.realpath(HIPCC)))
HOST_FLAGS = ["-O2", "-fPIC", "-std=c++20", "-Wall", "-Wextra", f"-I{INCLUDE}",
              f"-I{os.path.join(ROCM, 'include')}", "-D__HIP_PLATFORM_AMD__", "-x", "c++"]


def sources():
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith(".hip") or name.endswith(".cpp"):
            out.append(os.path.join(CSRC, name))
    for name in sorted(os.listdir(HOST)):
        if name.endswith(".cc"):
            out.append(os.path.join(HOST, name))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if os.path.dirname(src) == HOST:
        cmd = [HIPCC, *HOST_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, *PER_FILE.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if src.endswith(".cpp"):  # the C ABI over the kernels: host code beside HIP launches
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    # The plan writer's bulk generator (host code only).
    gen_src = os.path.join(HERE, "plangen", "plangen.cc")
    gen_tmp = PLANGEN_LIB + ".tmp"
    r = subprocess.run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-pthread",
                        "-ffp-contract=off", "-o", gen_tmp, gen_src], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on plangen.cc:\n{r.stderr[-6000:]}")
    os.replace(gen_tmp, PLANGEN_LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    for lib in (LIB, PLANGEN_LIB):
        if os.path.exists(lib):
            os.remove(lib)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
