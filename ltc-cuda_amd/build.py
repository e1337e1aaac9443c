"""Compile libltc_hip.so (the C-ABI library) for gfx950 with hipcc, in-tree.

Usage:  python ltc-cuda_amd/build.py [--verbose]

The library is linked against the HIP runtime by SONAME only (no rpath), so
a process that has already imported torch resolves it to torch's bundled
libamdhip64.so.7 and only one HIP runtime is ever mapped.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libltc_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ("ltc_device.hip", "ltc_capi.hip")
ARCH = os.environ.get("LTC_OFFLOAD_ARCH", "gfx950")


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.isfile(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def source_files() -> list:
    """Every file the library and the torch extension are built from."""
    inc = os.path.join(os.path.dirname(HERE), "include", "ltc_capi.h")
    return [os.path.join(CSRC, s) for s in SOURCES] + [
        os.path.join(CSRC, "ltc_internal.h"), os.path.join(CSRC, "ltc_torch_ext.cpp"), inc]


def command(out: str = LIB_PATH, arch: str = ARCH) -> list:
    return [
        hipcc_path(),
        f"--offload-arch={arch}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-mcode-object-version=5",
        # Resolve libamdhip64.so.7 by SONAME (torch's copy once torch is loaded).
        "-fno-rtlib-add-rpath",
        # Fixed SONAME: the torch extension and ctypes then share one instance.
        "-Wl,-soname," + LIB_NAME,
        # No packed-FP32 (v_pk_*_f32) instructions anywhere in device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        "-o", out,
        *[os.path.join(CSRC, s) for s in SOURCES],
    ]


EXT_SRC = os.path.join(CSRC, "ltc_torch_ext.cpp")
EXT_NAME = "_ltc_torch"


def ext_path() -> str:
    import sysconfig
    return os.path.join(HERE, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def ext_command(out: str) -> list:
    """Host-only C++ build of the torch glue (the autograd node of the
    fused module path), linked against libltc_hip.so through $ORIGIN."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension as ce
    incs = ce.include_paths("cuda") + [sysconfig.get_paths()["include"]]
    libs = ce.library_paths("cuda")[:1]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-fvisibility=hidden", "-w",
        # The HIP headers torch includes select their AMD half with this macro.
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        *[f"-I{d}" for d in incs], EXT_SRC, "-o", out,
        f"-L{HERE}", "-lltc_hip", *[f"-L{d}" for d in libs],
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN", "-Wl,--no-as-needed",
    ]


def build_ext(verbose: bool = False) -> str:
    out = ext_path()
    tmp = out + ".tmp"
    cmd = ext_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("torch extension build failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False, arch: str = ARCH) -> str:
    """Compile libltc_hip.so for `arch`, then the torch extension; returns the
    library path."""
    tmp = LIB_PATH + ".tmp"
    cmd = command(tmp, arch)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, LIB_PATH)
    build_ext(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
