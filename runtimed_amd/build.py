"""Build librq.so (the HIP kernels and the C ABI of include/rq.h) for gfx950.

Run as ``python -m runtimed_amd.build`` or through ``__graft_entry__.build()``.
Objects go to runtimed_amd/_build/, the library to runtimed_amd/librq.so.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "librq.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["csrc/rq_api.cpp", "csrc/rq_dequant.hip", "csrc/rq_gemv.hip", "csrc/rq_gemv_mx.hip", "csrc/rq_fp8.hip",
           "csrc/rq_gemm.hip", "csrc/rq_smallm.hip", "csrc/rq_smallm_codes.hip", "csrc/rq_marlin.hip", "csrc/rq_kv.hip", "csrc/rq_upload.hip",
           "csrc/rq_workspace.cpp", "csrc/rq_noalloc.hip", "host/rq_host.cpp"]
ROOT = PKG.parent
HOST_TEST_SRC = ROOT / "tests" / "cpp" / "test_host.cpp"
HOST_TEST_BIN = ROOT / "tests" / "cpp" / "test_host"

# Packed FP32 ops stay off: the compiler must not emit v_pk_{add,mul,fma}_f32.
COMMON = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str) -> Path:
    obj = OUT / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(PKG / src), "-o", str(obj)]
    started = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    # the object is as old as the sources it was compiled from: an edit made
    # while it compiled leaves it stale for an incremental build
    os.utime(obj, (started, started))
    return obj


def _stale(src: str) -> bool:
    """An object older than its source or than any header it may include."""
    obj = OUT / (Path(src).stem + ".o")
    if not obj.exists():
        return True
    deps = [PKG / src, *CSRC.glob("*.h"), *(PKG / "host").glob("*.hpp"), *(ROOT / "include").glob("*.h")]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps)


def build(verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every source (or, with incremental, only sources whose object
    is stale) and link librq.so."""
    OUT.mkdir(exist_ok=True)
    srcs = [s for s in SOURCES if (PKG / s).exists()]
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    objs = [OUT / (Path(s).stem + ".o") for s in srcs]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_host_tests(verbose: bool = False) -> Path:
    """The C++ test program of the host layer; links librq.so and the oracle
    (test infrastructure) through rpaths relative to the binary."""
    oracle_dir = ROOT / "oracle"
    cmd = [HIPCC, "-O2", "-std=c++17", f"--offload-arch={ARCH}", "-x", "hip", str(HOST_TEST_SRC),
           "-o", str(HOST_TEST_BIN), f"-L{PKG}", "-lrq", f"-L{oracle_dir}", "-lrq_oracle",
           "-Wl,-rpath,$ORIGIN/../../runtimed_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"host test build failed:\n{res.stderr}")
    if verbose:
        print(f"built {HOST_TEST_BIN}")
    return HOST_TEST_BIN


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
