// Test kit for the exact-sum engine of k_full (ultima.cpp_amd/csrc/hsamp_xsum.h):
// one block of kFT threads takes a sequence x[0, n) of floats >= 0 (padded
// with +0 to Vp = a whole number of 512 * G windows) and returns
//   out[0]  its sequential float32 sum in index order (exact_index_sum),
// and, when thr > 0, the top-p driver's answer for x as probabilities:
//   outi[0] whether the running sum in descending order reaches thr,
//   outi[1] how many values that takes, out[1] the last one, out[2] the sum,
//   outi[2] how many values are larger than the last one, outi[3] how many
//   equal it.
// rlo / rhi: the smallest and largest float bits above 0 in x when the caller
// gives them (rhi 0: the driver finds them).
// tests/test_gpu_xsum.py compares them with numpy's sequential float32 sums.
#include <hip/hip_runtime.h>

#include "hsamp_xsum.h"

using namespace hsamp;

__global__ __launch_bounds__(kFT) void k_xsum(const float* x, int n, int Vp, int G, float thr, uint32_t rlo,
                                              uint32_t rhi, float* out, int* outi) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ FullShared st;
    const FullLds f = full_lds(smem);
    const int lane = lane_id(), wid = wave_id();
    const int WS = kFWin * G, nW = Vp / WS;
    for (int w = wid; w < nW; w += kFW) {
        float ws = 0.0f;
        for (int i = lane; i < WS; i += 64) ws += x[(size_t)w * WS + i];
        ws = wave_tree_prefix_f(ws);
        if (lane == 63) f.winA[w] = ws;
    }
    __syncthreads();
    const XState s = exact_index_sum(x, nW, G, f, st);
    if (threadIdx.x == 0) out[0] = xs_value(s);
    if (thr > 0.0f) {
        uint32_t ck = 0u;
        int cc = 0, cg = 0, ce = 0;
        const bool ok = full_top_p(x, n, Vp, 1.0f, thr, f, st, rlo, rhi, &ck, &cc, &cg, &ce);
        if (threadIdx.x == 0) {
            outi[0] = ok ? 1 : 0;
            outi[1] = cc;
            outi[2] = cg;
            outi[3] = ce;
            out[1] = __uint_as_float(ck);
            out[2] = (float)st.dS;
        }
    }
}

// xinc2 and xinc2f (integer and float arithmetic) for x[i] at binade E:
// out[4 i .. 4 i + 3] = xinc2's pair, xinc2f's pair (or two pairs that
// differ when xinc and xincf disagree).
__global__ void k_xinc(const float* x, int n, int E, uint32_t* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const XPair a = xinc2(x[i], E);
    bool t;
    const XPair b = xinc2f(x[i], E, t);
    // xincf's increment, tie and big flags against xinc's (a mismatch shows as
    // an impossible pair)
    // and xinc1f's: the pair's common increment away from one half, the same tie flag
    bool t1, g1, t2, g2, t3;
    const uint32_t i1 = xinc(x[i], E, t1, g1), i2 = xincf(x[i], E, t2, g2), i3 = xinc1f(x[i], E, t3);
    if (i1 != i2 || t1 != t2 || g1 != g2 || t3 != t || (!t && (i3 != b.d0 || b.d0 != b.d1))) {
        out[4 * i] = 0xFFFFFFFFu;
        out[4 * i + 1] = 0u;
        out[4 * i + 2] = 0u;
        out[4 * i + 3] = 0xFFFFFFFFu;
        return;
    }
    out[4 * i] = a.d0;
    out[4 * i + 1] = a.d1;
    out[4 * i + 2] = b.d0;
    out[4 * i + 3] = b.d1;
}

extern "C" int xinc_run(const float* x, int n, int E, uint32_t* out) {
    hipLaunchKernelGGL(k_xinc, dim3((n + 255) / 256), dim3(256), 0, nullptr, x, n, E, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    return (int)hipDeviceSynchronize();
}

extern "C" int xsum_run(const float* x, int n, int Vp, int G, float thr, uint32_t rlo, uint32_t rhi, float* out,
                        int* outi) {
    hipLaunchKernelGGL(k_xsum, dim3(1), dim3(kFT), kFullLdsBytes, nullptr, x, n, Vp, G, thr, rlo, rhi, out, outi);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    return (int)hipDeviceSynchronize();
}
