"""ultima.cpp_amd -- the MI355X (gfx950) token sampler of Ultima.cpp.

Native parts (built in-tree by build.py):
    libultima_hsamp.so    HIP kernels + the C ABI of include/ultima_hsamp.h
    libultima_sampler.so  the ultima::sampler C++ drop-in (include/ultima/sampler/sampler.hpp)
Python parts:
    hsamp      ctypes binding of the C ABI (tests, bench)
    workloads  seeded synthetic workloads of the five benchmark configurations

The directory name is not a Python identifier; __graft_entry__.load_package()
imports it as `ultima_cpp_amd`.
"""
from . import hsamp, workloads  # noqa: F401
