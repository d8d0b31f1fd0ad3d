// Test kit: evaluates the product's device expf (ultima.cpp_amd/csrc/libm_expf.h)
// over a contiguous range of float bit patterns, so tests can compare it with
// the host libm bit for bit.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "libm_expf.h"

__global__ void k_expf_range(uint32_t start, float* out, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) out[i] = hsamp::libm_expf(__uint_as_float(start + (uint32_t)i));
}

extern "C" int device_expf_range(uint32_t start, float* out_dev, int n, void* stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_expf_range, dim3((n + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), start, out_dev, n);
    return (int)hipGetLastError();
}
