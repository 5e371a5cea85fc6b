"""Build the gfx950 code object and the C-ABI host library, in-tree.

    realm_amd/lib/realm_kernels.hsaco   hipcc --genco --offload-arch=gfx950
    realm_amd/lib/librealm_hip.so       g++ (realm_hip.cpp, gguf.cpp) plus the hipcc
                                        object of noalloc.hip (the no-allocation
                                        entry point's device array), embeds the code
                                        objects, links libamdhip64

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

# code objects: the non-GEMV kernels, the GEMV variants per format and token
# count (1, 2, 4) and the LDS-tiled GEMM (compiled in parallel; the host library embeds all of them)
HSACO_UNITS = [("realm_kernels", "realm_kernels.hip", ()),
               ("realm_gemv_q4k", "gemv_fmt.hip", ("REALM_GEMV_FMT=0",)),
               ("realm_gemv_q6k", "gemv_fmt.hip", ("REALM_GEMV_FMT=1",)),
               ("realm_gemv_q80", "gemv_fmt.hip", ("REALM_GEMV_FMT=2",)),
               ("realm_gemv_q4k_t2", "gemv_fmt.hip", ("REALM_GEMV_FMT=0", "REALM_GEMV_NT=2")),
               ("realm_gemv_q6k_t2", "gemv_fmt.hip", ("REALM_GEMV_FMT=1", "REALM_GEMV_NT=2")),
               ("realm_gemv_q80_t2", "gemv_fmt.hip", ("REALM_GEMV_FMT=2", "REALM_GEMV_NT=2")),
               ("realm_gemv_q4k_t4", "gemv_fmt.hip", ("REALM_GEMV_FMT=0", "REALM_GEMV_NT=4")),
               ("realm_gemv_q6k_t4", "gemv_fmt.hip", ("REALM_GEMV_FMT=1", "REALM_GEMV_NT=4")),
               ("realm_gemv_q80_t4", "gemv_fmt.hip", ("REALM_GEMV_FMT=2", "REALM_GEMV_NT=4")),
               ("realm_gemv_q8m", "gemv_fmt.hip", ("REALM_GEMV_FMT=3",)),
               ("realm_gemv_q8m_t2", "gemv_fmt.hip", ("REALM_GEMV_FMT=3", "REALM_GEMV_NT=2")),
               ("realm_gemv_q8m_t4", "gemv_fmt.hip", ("REALM_GEMV_FMT=3", "REALM_GEMV_NT=4")),
               ("realm_gemv_q4k_pre", "gemv_fmt.hip", ("REALM_GEMV_FMT=0", "REALM_GEMV_PRE")),
               ("realm_gemv_q6k_pre", "gemv_fmt.hip", ("REALM_GEMV_FMT=1", "REALM_GEMV_PRE")),
               ("realm_gemv_q80_pre", "gemv_fmt.hip", ("REALM_GEMV_FMT=2", "REALM_GEMV_PRE")),
               ("realm_gemm_tiled", "gemm_tiled.hip", ()),
               ("realm_gemm_tiled_q80", "gemm_tiled.hip", ("REALM_TILED_Q80",))]
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
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "unknown target feature" not in l and "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_hsaco(out: str = HSACO, defines: tuple = (), src: str = "realm_kernels.hip") -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, *[f"-D{d}" for d in defines],
          "-I", KDIR, os.path.join(KDIR, src), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_all_hsaco(out_dir: str = LIB_DIR, defines: tuple = ()) -> list:
    """Every code object of HSACO_UNITS, compiled in parallel; returns paths."""
    import concurrent.futures as cf
    jobs = [(os.path.join(out_dir, name + ".hsaco"), tuple(defs) + tuple(defines), src)
            for name, src, defs in HSACO_UNITS]
    with cf.ThreadPoolExecutor(len(jobs)) as ex:
        return list(ex.map(lambda j: build_hsaco(*j), jobs))


def build_noalloc_object(out_dir: str = LIB_DIR) -> str:
    """hipcc object (host code + gfx950 device code) holding the fixed
    scratch array of the no-allocation entry point and its address lookup."""
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "noalloc.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", "-fvisibility=hidden",
          "--offload-arch=gfx950", "-O2",
          "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", HDIR, os.path.join(HDIR, "noalloc.hip"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_host(out: str = LIBSO, hsacos: list | None = None) -> str:
    if hsacos is None:
        hsacos = [os.path.join(LIB_DIR, name + ".hsaco") for name, _, _ in HSACO_UNITS]
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    embeds = [f"-DREALM_HSACO_FILE{i}={p}" for i, p in enumerate(hsacos)]
    noalloc = build_noalloc_object(os.path.dirname(out))
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
          "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__", f"-DREALM_HSACO_COUNT={len(hsacos)}", *embeds,
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(REPO, "include"),
          "-I", KDIR, "-I", HDIR,
          os.path.join(HDIR, "realm_hip.cpp"), os.path.join(HDIR, "gguf.cpp"), noalloc,
          "-o", tmp,
          "-L", os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-lamdhip64", "-lpthread"])
    os.replace(tmp, out)
    return out


def build() -> str:
    return build_host(hsacos=build_all_hsaco())


if __name__ == "__main__":
    print(build())
