"""The CMake build of the sampler (ultima.cpp_amd/CMakeLists.txt), used the way
Ultima.cpp uses its own: a consumer project adds the directory and links the
STATIC target `ultima_sampler` (reference src/sampler/CMakeLists.txt:1-15),
exactly as the reference's server, CLI and tests link theirs. CPU only: the
kernels are cross-compiled for gfx950 and the consumer runs host code only
(SamplerParams defaults and identity(), sampler.hpp:16-47)."""
import shutil
import subprocess
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "ultima.cpp_amd"

CONSUMER_MAIN = r"""
#include <cstdio>
#include "ultima/sampler/sampler.hpp"
int main() {
    const ultima::sampler::SamplerParams d{};
    const ultima::sampler::SamplerParams id = ultima::sampler::SamplerParams::identity();
    // reference defaults (sampler.hpp:16-45) and identity() (sampler.cpp:192-205)
    const bool ok = d.temperature == 0.2f && d.top_k == 40 && d.top_p == 0.95f && d.min_p == 0.05f &&
                    d.rep_penalty == 1.1f && d.repeat_last_n == 64 && d.dry_multiplier == 0.8f &&
                    id.temperature == 1.0f && id.top_k == 0 && id.top_p == 1.0f && id.min_p == 0.0f &&
                    id.rep_penalty == 1.0f && id.repeat_last_n == 0 && id.dry_multiplier == 0.0f;
    std::printf("%s\n", ok ? "consumer ok" : "consumer mismatch");
    return ok ? 0 : 1;
}
"""


def _run(cmd, cwd):
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, f"{' '.join(map(str, cmd))} failed:\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}"
    return r.stdout


@pytest.mark.skipif(shutil.which("cmake") is None or not Path("/opt/rocm/llvm/bin/clang++").exists(),
                    reason="needs cmake and the ROCm clang")
def test_consumer_links_ultima_sampler_through_cmake(tmp_path):
    proj = tmp_path / "consumer"
    proj.mkdir()
    (proj / "main.cpp").write_text(CONSUMER_MAIN)
    (proj / "CMakeLists.txt").write_text(textwrap.dedent(f"""\
        cmake_minimum_required(VERSION 3.21)
        project(consumer LANGUAGES CXX)
        add_subdirectory({PKG.as_posix()} ultima_amd)
        add_executable(consumer main.cpp)
        target_link_libraries(consumer PRIVATE ultima_sampler)
        """))
    build = tmp_path / "build"
    _run(["cmake", "-S", str(proj), "-B", str(build)], tmp_path)
    _run(["cmake", "--build", str(build), "-j", "8"], tmp_path)
    lib = build / "ultima_amd" / "libultima_sampler.a"
    assert lib.exists(), "ultima_sampler must be a static library, as the reference's target is"
    syms = _run(["nm", "-C", "--defined-only", str(lib)], tmp_path)
    for name in ("ultima::sampler::sample(", "ultima::sampler::argmax(", "ultima::sampler::SamplerParams::identity()"):
        assert name in syms, f"{name} missing from libultima_sampler.a"
    out = _run([str(build / "consumer")], tmp_path)
    assert "consumer ok" in out
