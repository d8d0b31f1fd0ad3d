"""pytest setup: the `gpu` marker, import paths and shared fixtures.

CPU tests (-m "not gpu") pin the oracle and check the library's host side;
GPU tests (-m gpu) are the parity tests proper and call the HIP sampler
through its C ABI.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def wl(pkg):
    return pkg.workloads


@pytest.fixture(scope="session")
def hs(pkg):
    """The C ABI binding with a handle on cuda:0 (GPU tests only)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X: torch.cuda.is_available() is False")
    return pkg.hsamp


@pytest.fixture(scope="session")
def _samplers(hs):
    cache = {}
    yield cache
    for s in cache.values():
        s.close()


OVERRIDES = ("ULTIMA_HSAMP_EXACT", "ULTIMA_HSAMP_EXACT_TILES", "ULTIMA_HSAMP_SLICES")


@pytest.fixture
def sampler(hs, _samplers, request):
    """A library handle shared by the GPU parity tests, one per setting of the
    diagnostics overrides (which a handle reads when it is created): a test
    that takes kernel_mode gets the handle of its mode."""
    import os
    if "kernel_mode" in request.fixturenames:
        request.getfixturevalue("kernel_mode")
    key = tuple(os.environ.get(k) for k in OVERRIDES)
    if key not in _samplers:
        _samplers[key] = hs.Sampler(0, max_rows=1024, max_vocab=1 << 18)
    return _samplers[key]


@pytest.fixture(params=["default", "exact", "exact2", "exact4", "general"])
def kernel_mode(request, monkeypatch):
    """Runs a test five times: with the library's own choice of kernels and
    slicing (no override: what every caller and bench.py get), with exact
    lists over slices of one tile, of two tiles and of four tiles
    (ULTIMA_HSAMP_EXACT_TILES, the fewest slices; four: aligned bf16 rows,
    whose history counts are then kept by rank; two: other aligned rows;
    unaligned rows keep one tile), and with ULTIMA_HSAMP_EXACT=0, which sends
    every batch to the general stream and merge kernels."""
    monkeypatch.delenv("ULTIMA_HSAMP_EXACT", raising=False)
    monkeypatch.delenv("ULTIMA_HSAMP_SLICES", raising=False)
    if request.param == "default":
        monkeypatch.delenv("ULTIMA_HSAMP_EXACT_TILES", raising=False)
    elif request.param == "general":
        monkeypatch.setenv("ULTIMA_HSAMP_EXACT", "0")
        monkeypatch.delenv("ULTIMA_HSAMP_EXACT_TILES", raising=False)
    else:
        monkeypatch.setenv("ULTIMA_HSAMP_EXACT_TILES", {"exact2": "2", "exact4": "4"}.get(request.param, "1"))
    return request.param
