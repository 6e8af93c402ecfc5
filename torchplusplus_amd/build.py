"""Build recipe for the gfx950 kernel library and its torch extension.

Produces, in-tree (so the files travel with the source tree):
  torchplusplus_amd/libtorchpp_hip.so   -- every HIP kernel + the C ABI of include/tpp.h
  torchplusplus_amd/_C<EXT_SUFFIX>      -- pybind11/torch binding over that C ABI

The reference built five CUDAExtension modules with nvcc for sm_80
(/root/reference/setup.py:39-89). Here one hipcc invocation per source file
targets gfx950 only; no CUTLASS/CK is compiled. The library links ROCm's
hipBLASLt for the plain GEMMs it dispatches there (csrc/gemm_lt.hip).

Usage: python -m torchplusplus_amd.build  [--lib-only] [-j N]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(REPO_DIR, "_build")
LIB_NAME = "libtorchpp_hip.so"
ARCH = os.environ.get("TORCHPP_ARCH", "gfx950")
ROCM_PATH = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM_PATH, "bin", "hipcc"))

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32; the host
# pass prints a harmless "not a recognized feature" warning for it.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    "-Wno-unused-command-line-argument",
]


def kernel_sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n{' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_lib(jobs: int = 8) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = kernel_sources()
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD_DIR, os.path.basename(s) + ".o")
        objs.append(o)
        cmds.append([HIPCC, *DEVICE_FLAGS, "-c", s, "-o", o])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    out = os.path.join(PKG_DIR, LIB_NAME)
    tmp = out + ".tmp"
    rocm_lib = os.path.join(ROCM_PATH, "lib")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, f"-L{rocm_lib}", "-lhipblaslt",
          f"-Wl,-rpath,{rocm_lib}", "-o", tmp])
    os.replace(tmp, out)
    return out


def build_ext() -> str:
    import torch  # noqa: F401  (only for its include/lib paths)
    from torch.utils import cpp_extension

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG_DIR, "_C" + ext_suffix)
    tmp = out + ".tmp"
    incs = cpp_extension.include_paths(device_type="cuda")
    libs = cpp_extension.library_paths(device_type="cuda")
    torch_lib = libs[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        HIPCC,
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-x", "c++",
        os.path.join(CSRC, "ext", "bindings.cpp"),
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-Wno-unused-command-line-argument",
        "-Wno-deprecated-declarations",
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{REPO_DIR}",
        *[f"-I{p}" for p in incs],
        *[f"-L{p}" for p in libs],
        f"-L{PKG_DIR}",
        "-ltorchpp_hip",
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        "-lamdhip64",
        f"-Wl,-rpath,{torch_lib}",
        "-Wl,-rpath,$ORIGIN",
        "-o", tmp,
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all(jobs: int = 8, lib_only: bool = False) -> None:
    lib = build_lib(jobs)
    print(f"built {os.path.relpath(lib, REPO_DIR)}")
    if not lib_only:
        ext = build_ext()
        print(f"built {os.path.relpath(ext, REPO_DIR)}")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    build_all(a.j, a.lib_only)
    sys.exit(0)
