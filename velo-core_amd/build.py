"""Build the gfx950 code object and the C-ABI host library in-tree.

  velokv/velokv_gfx950.co  hipcc --offload-arch=gfx950 --offload-device-only (raw code object)
  velokv/libvelokv.so      g++ over the HIP runtime API (host code only)

Run `python velo-core_amd/build.py` or __graft_entry__.build().
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "velokv")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "--offload-device-only", "--no-gpu-bundle-output", "-O3", "-std=c++17",
    # no packed-fp32 (v_pk_*_f32) instructions anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-pass-failed",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    return r.stdout


def build_code_object():
    out = os.path.join(PKG, "velokv_gfx950.co")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, f"-I{CSRC}", f"-I{INCLUDE}",
          os.path.join(CSRC, "velokv_kernels.hip"), "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host_library():
    out = os.path.join(PKG, "libvelokv.so")
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{INCLUDE}", f"-I{CSRC}",
          os.path.join(CSRC, "velokv_host.cpp"), os.path.join(CSRC, "velokv_radix.cpp"), "-o", tmp,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl"])
    os.replace(tmp, out)
    return out


def build():
    co = build_code_object()
    so = build_host_library()
    return co, so


if __name__ == "__main__":
    for p in build():
        print(p)
