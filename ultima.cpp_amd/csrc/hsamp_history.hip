// Device-side history for the penalties: each row's recent-token window kept
// in device memory and appended on the GPU with the step's sampled token
// (reference SamplerContext::push_recent, src/sampler/sampler.cpp:213, called
// after every sample() by src/server/http_server.cpp:183 and
// apps/ultima-cli/main.cpp:679).
//
// k_history_push: one wave per row. A full row (length >= stride) first keeps
// its last `keep` ids at its front (keep <= stride / 2: source and
// destination do not overlap), then the token goes to position length and
// the length advances. The sampler reads the rows and the lengths where they
// are (ultima_hsamp_batch.hist, .hist_len_dev).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ultima_hsamp.h"

namespace hsamp {
namespace {

__global__ __launch_bounds__(64) void k_history_push(int32_t* __restrict__ hist, int64_t stride,
                                                     int32_t* __restrict__ len, const int32_t* __restrict__ tokens,
                                                     int rows, int keep) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    int32_t* h = hist + (int64_t)r * stride;
    // the length and the token go out together: one memory round trip
    int L = len[r];
    const int32_t tok = tokens[r];
    L = L < 0 ? 0 : L;
    if (L >= stride) {
        // [L - keep, L) -> [0, keep): L = stride here, keep <= stride / 2
        const int64_t from = stride - keep;
        // eight ids per thread in flight, then their stores (the ranges do not
        // overlap: from >= keep)
        for (int i0 = 0; i0 < keep; i0 += 8 * 64) {
            int32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * 64 + (int)threadIdx.x;
                v[j] = h[from + min(i, keep - 1)];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * 64 + (int)threadIdx.x;
                if (i < keep) h[i] = v[j];
            }
        }
        L = keep;
    }
    if (threadIdx.x == 0) {
        h[L] = tok;
        len[r] = L + 1;
    }
}

}  // namespace
}  // namespace hsamp

extern "C" int ultima_hsamp_history_push(int32_t* hist, int64_t hist_stride, int32_t* hist_len_dev,
                                         const int32_t* tokens, int32_t rows, int32_t keep, void* hip_stream) {
    if (hist == nullptr || hist_len_dev == nullptr || tokens == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    if (rows < 1 || hist_stride < 2 || keep < 1 || (int64_t)keep > hist_stride / 2 || hist_stride > INT32_MAX)
        return ULTIMA_HSAMP_ERR_INVALID;
    hipLaunchKernelGGL(hsamp::k_history_push, dim3(rows), dim3(64), 0, static_cast<hipStream_t>(hip_stream), hist,
                       hist_stride, hist_len_dev, tokens, (int)rows, (int)keep);
    return hipGetLastError() == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}
