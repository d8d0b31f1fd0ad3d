"""The product's expf (ultima.cpp_amd/csrc/libm_expf.h) against glibc expf.

The header is compiled for the host here (g++, FMA enabled, no contraction)
and evaluated on every non-NaN float; the result must equal the host libm's
expf bit for bit. The same source compiles for gfx950; the GPU parity tests
check the device build against the oracle.
"""
import subprocess
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

SRC = textwrap.dedent(r"""
    #include <cmath>
    #include <cstdio>
    #include <cstring>
    #include <cstdint>
    #include "libm_expf.h"
    int main() {
        unsigned long long bad = 0, n = 0;
        #pragma omp parallel for reduction(+:bad,n) schedule(static, 1 << 16)
        for (long long i = 0; i <= 0xffffffffLL; ++i) {
            uint32_t u = (uint32_t)i; float x; std::memcpy(&x, &u, 4);
            if (std::isnan(x)) continue;
            float a = hsamp::libm_expf(x), b = expf(x);
            uint32_t ua, ub; std::memcpy(&ua, &a, 4); std::memcpy(&ub, &b, 4);
            bad += (ua != ub); ++n;
        }
        std::printf("%llu %llu\n", n, bad);
        return 0;
    }
""")


def test_libm_expf_matches_host_expf_on_every_float(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text(SRC)
    exe = tmp_path / "t"
    cmd = ["g++", "-std=c++20", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp",
           f"-I{ROOT / 'ultima.cpp_amd' / 'csrc'}", str(src), "-o", str(exe)]
    subprocess.run(cmd, check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600)
    n, bad = map(int, out.stdout.split())
    assert n == 2**32 - 2 * (2**23 - 1)          # every float but the NaNs
    assert bad == 0, f"{bad} of {n} floats differ from libm expf"
