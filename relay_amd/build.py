"""Builds librelay_hip.so in-tree: the gfx950 kernels (hipcc) and the C++ host backend
(g++ against the HIP runtime API), linked with rocBLAS.

    python -m relay_amd.build            # build (always recompiles)

The library lands next to this file (relay_amd/librelay_hip.so), so it travels with the
source tree; object files go to relay_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librelay_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_SOURCES = ["decode_attention.hip", "flash_prefill.hip", "gemv.hip", "gemm_w8.hip", "layer_ops.hip"]
HOST_SOURCES = ["host/hip_backend.cpp", "host/lt_gemm.cpp", "host/capi.cpp", "host/config.cpp", "host/backend_defaults.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter",
    # No packed fp32 instructions (v_pk_*_f32) anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter", "-D__HIP_PLATFORM_AMD__",
              f"-I{ROCM}/include", f"-I{CSRC}/host", f"-I{REPO}/include"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the device-only feature flag.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs.append(["g++", *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for cmd in jobs:
            if verbose:
                print(" ".join(cmd), flush=True)
        list(ex.map(_run, jobs))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, f"-L{ROCM}/lib", "-lhipblaslt", "-lrocblas",
          "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> None:
    """The CPU oracle (test infrastructure) and, where the reference tree exists, the
    reference CPU backend built from it (oracle/_ref)."""
    oracle = os.path.join(REPO, "oracle")
    subprocess.run(["make", "-s", "-C", oracle, "-B", "all"], check=True)
    if os.path.isdir("/root/reference/engine"):
        subprocess.run(["make", "-s", "-C", oracle, "-j8", "ref"], check=True)
        # relay's Engine driving the HIP backend (needs the kernel objects of build())
        subprocess.run(["make", "-s", "-C", oracle, "-j8", "engine-hip"], check=True)
        # relay's own test programs with the RELAY_TEST_BACKEND=hip branch of check.h
        subprocess.run(["make", "-s", "-C", oracle, "-j8", "ref-tests-hip"], check=True)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
