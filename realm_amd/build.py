"""Build the gfx950 code object and the C-ABI host library, in-tree.

    realm_amd/lib/realm_kernels.hsaco   hipcc --genco --offload-arch=gfx950
    realm_amd/lib/librealm_hip.so       g++, embeds the code object, links libamdhip64

Run as ``python -m realm_amd.build`` (or through ``__graft_entry__.build()``).
Builds always recompile; they cross-compile without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
LIB_DIR = os.path.join(PKG, "lib")
KDIR = os.path.join(PKG, "csrc", "kernels")
HDIR = os.path.join(PKG, "csrc", "host")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(LIB_DIR, "realm_kernels.hsaco")
LIBSO = os.path.join(LIB_DIR, "librealm_hip.so")

# Packed-FP32 instructions are kept out of every kernel (they have produced
# silent wrong results on these machines); hipcc's host pass warns that it
# does not know the feature, which is harmless.
HIP_FLAGS = [
    "--genco", "--offload-arch=gfx950", "--no-gpu-bundle-output", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "unknown target feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_hsaco(out: str = HSACO, defines: tuple = ()) -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, *[f"-D{d}" for d in defines],
          "-I", KDIR, os.path.join(KDIR, "realm_kernels.hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host(out: str = LIBSO, hsaco: str = HSACO) -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
          "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__", f"-DREALM_HSACO_FILE={hsaco}",
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(REPO, "include"),
          "-I", KDIR,
          os.path.join(HDIR, "realm_hip.cpp"), "-o", tmp,
          "-L", os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-lamdhip64", "-lpthread"])
    os.replace(tmp, out)
    return out


def build() -> str:
    build_hsaco()
    return build_host()


if __name__ == "__main__":
    print(build())
