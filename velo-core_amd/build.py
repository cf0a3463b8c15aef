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


OBJ_DIR = os.path.join(HERE, "_build")


def build_noalloc_object():
    """velokv_noalloc.hip: host code plus the per-device scratch array of
    vk_paged_decode_noalloc (a gfx950 fat binary linked into libvelokv.so)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    out = os.path.join(OBJ_DIR, "velokv_noalloc.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-c",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument",
          f"-I{CSRC}", f"-I{INCLUDE}", os.path.join(CSRC, "velokv_noalloc.hip"), "-o", out])
    return out


def build_host_library(sanitize: bool = False):
    """libvelokv.so (or, with sanitize, libvelokv_asan.so: the host C++ under
    AddressSanitizer + UndefinedBehaviorSanitizer, for the CPU test suite)."""
    out = os.path.join(PKG, "libvelokv_asan.so" if sanitize else "libvelokv.so")
    tmp = out + ".tmp"
    noalloc = build_noalloc_object()
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"] if sanitize else []
    _run(["g++", "-O1" if sanitize else "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-Wno-unused-parameter", *san,
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{INCLUDE}", f"-I{CSRC}",
          os.path.join(CSRC, "velokv_host.cpp"), os.path.join(CSRC, "velokv_radix.cpp"), noalloc, "-o", tmp,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl"])
    os.replace(tmp, out)
    return out


def build():
    co = build_code_object()
    so = build_host_library()
    return co, so


def sanitizer_runtime():
    """LD_PRELOAD value for a Python process that loads the sanitized libraries
    (the interpreter itself is not instrumented, so the runtimes come first)."""
    libs = []
    for name in ("libasan.so", "libubsan.so"):
        p = subprocess.run(["g++", f"-print-file-name={name}"], stdout=subprocess.PIPE, text=True).stdout.strip()
        libs.append(os.path.realpath(p))
    return ":".join(libs)


def build_sanitized(run_tests: bool = False) -> int:
    """Host library and oracle under AddressSanitizer + UndefinedBehaviorSanitizer
    (host code only; the GPU code object is not involved), then optionally the
    CPU test suite (pytest -m "not gpu") loading them."""
    build_host_library(sanitize=True)
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "asan"])
    if not run_tests:
        return 0
    env = dict(os.environ, VELOKV_SANITIZE="1", LD_PRELOAD=sanitizer_runtime(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-m", "not gpu",
                           "-p", "no:cacheprovider"], env=env, cwd=ROOT).returncode


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        sys.exit(build_sanitized(run_tests="--run-tests" in sys.argv))
    for p in build():
        print(p)
