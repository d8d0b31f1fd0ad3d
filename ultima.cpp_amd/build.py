"""Build the native libraries of the package in-tree.

    libultima_hsamp.so   -- HIP kernels for gfx950 + the C ABI (include/ultima_hsamp.h)
    libultima_hsamp_noalloc.so -- the allocation-free entry (include/ultima_hsamp_noalloc.h)
    libultima_sampler.so -- the ultima::sampler C++ drop-in (include/ultima/sampler/sampler.hpp)
    dropin_driver        -- tests/cpp/dropin_driver.cpp linked against the drop-in
    tests/cpp/libdevice_expf.so -- test kit evaluating the device expf
    tests/cpp/libxsum_kit.so    -- test kit running the exact-sum engine of k_full

Every call compiles from scratch (no staleness checks): the outputs are small
and the compile takes well under a minute.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INC = ROOT / "include"
BUILD = PKG / "_build"

HSAMP_SO = PKG / "libultima_hsamp.so"
NOALLOC_SO = PKG / "libultima_hsamp_noalloc.so"
SAMPLER_SO = PKG / "libultima_sampler.so"
CPP_TEST = PKG / "dropin_driver"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# Device code: gfx950 only, IEEE float semantics (no contraction, correctly
# rounded f32 division), no packed-FP32 instructions.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-rdc", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INC}", f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")
    noise = [ln for ln in (r.stdout + r.stderr).splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "not a recognized feature" not in ln]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build_all() -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    objs = {
        "hsamp_kernels.o": CSRC / "hsamp_kernels.hip",
        "hsamp_api.o": CSRC / "hsamp_api.cpp",
        "hsamp_head.o": CSRC / "hsamp_head.hip",
        "hsamp_headq.o": CSRC / "hsamp_headq.hip",
        "hsamp_history.o": CSRC / "hsamp_history.hip",
        "hsamp_callers.o": CSRC / "hsamp_callers.hip",
    }
    with ThreadPoolExecutor(max_workers=4) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-x", "hip", "-c", str(src), "-o", str(BUILD / o)])
                for o, src in [*objs.items(), ("hsamp_noalloc.o", CSRC / "hsamp_noalloc.hip")]]
        for f in futs:
            f.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-fno-gpu-rdc",
          *[str(BUILD / o) for o in objs], "-o", str(HSAMP_SO)])
    # its device array is held only by processes that load this library
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-fno-gpu-rdc", str(BUILD / "hsamp_noalloc.o"),
          "-o", str(NOALLOC_SO), f"-L{PKG}", "-lultima_hsamp", "-Wl,-rpath,$ORIGIN"])
    # The C++ drop-in: host code only, reference-compatible flags.
    cxx = ["g++", "-std=c++20", "-O2", "-fPIC", "-fno-rtti", "-fno-exceptions", "-Wall", "-Wextra",
           f"-I{INC}"]
    _run([*cxx, "-shared", str(CSRC / "sampler.cpp"), "-o", str(SAMPLER_SO),
          f"-L{PKG}", "-lultima_hsamp", "-Wl,-rpath,$ORIGIN"])
    _run([HIPCC, *HIP_FLAGS, "-shared", "-x", "hip", str(ROOT / "tests" / "cpp" / "device_expf.hip"),
          "-o", str(ROOT / "tests" / "cpp" / "libdevice_expf.so")])
    _run([HIPCC, *HIP_FLAGS, "-shared", "-x", "hip", str(ROOT / "tests" / "cpp" / "xsum_kit.hip"),
          "-o", str(ROOT / "tests" / "cpp" / "libxsum_kit.so")])
    # the test driver also allocates device memory itself (sample_batch)
    _run([*cxx, "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", str(ROOT / "tests" / "cpp" / "dropin_driver.cpp"),
          "-o", str(CPP_TEST), f"-L{PKG}", "-lultima_sampler", "-lultima_hsamp", f"-L{ROCM / 'lib'}", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN"])


if __name__ == "__main__":
    build_all()
