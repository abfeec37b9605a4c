"""Build the native parts of spira_amd in-tree.

* ``spira_amd/libspira_hip.so`` -- the gfx950 kernel library (hipcc), whose C
  ABI is declared in ``include/spira_hip.h``;
* ``spira_amd/nn/functional/_C*.so`` -- the torch host layer (g++ against
  PyTorch-ROCm), linked to the kernel library.

Run ``python -m spira_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
HIP_DIR = os.path.join(PKG, "csrc", "hip")
HOST_DIR = os.path.join(PKG, "csrc", "host")
BUILD_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libspira_hip.so")
EXT = os.path.join(PKG, "nn", "functional", "_C" + sysconfig.get_config_var("EXT_SUFFIX"))

ARCH = os.environ.get("SPIRA_HIP_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 vector ops are kept out of every device code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _torch_flags():
    import torch
    from torch.utils import cpp_extension as ce
    inc = ce.include_paths(device_type="cuda")
    libs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations"]
    cflags += [f"-I{p}" for p in inc] + [f"-I{sysconfig.get_paths()['include']}"]
    ldflags = [f"-L{p}" for p in libs] + [f"-Wl,-rpath,{p}" for p in libs]
    ldflags += ["-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip", "-lamdhip64"]
    return cflags, ldflags


def build(verbose: bool = False) -> None:
    os.makedirs(BUILD_DIR, exist_ok=True)
    hip_srcs = sorted(f for f in os.listdir(HIP_DIR) if f.endswith(".hip"))
    host_srcs = sorted(f for f in os.listdir(HOST_DIR) if f.endswith(".cpp"))
    cflags, ldflags = _torch_flags()
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for f in hip_srcs:
            obj = os.path.join(BUILD_DIR, f[:-4] + ".o")
            jobs.append(ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", os.path.join(HIP_DIR, f), "-o", obj]))
        for f in host_srcs:
            obj = os.path.join(BUILD_DIR, "host_" + f[:-4] + ".o")
            jobs.append(ex.submit(_run, [CXX, *cflags, "-c", os.path.join(HOST_DIR, f), "-o", obj]))
        for j in jobs:
            out = j.result()
            if verbose and out.strip():
                print(out)
    hip_objs = [os.path.join(BUILD_DIR, f[:-4] + ".o") for f in hip_srcs]
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *hip_objs, "-o", LIB])
    host_objs = [os.path.join(BUILD_DIR, "host_" + f[:-4] + ".o") for f in host_srcs]
    _run([CXX, "-shared", "-fPIC", *host_objs, "-o", EXT, f"-L{PKG}", "-l:libspira_hip.so",
          "-Wl,-rpath,$ORIGIN/../..", *ldflags])
    if verbose:
        print(f"built {LIB}\nbuilt {EXT}")


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
