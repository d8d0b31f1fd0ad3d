// The logits producer on gfx950: final rmsnorm + lm-head matvec, feeding the
// sampler's [rows, V] logits in device memory (reference
// src/model/qwen_model.cpp:182-207).
//
// Results are the reference's bits. Its kernels are AVX2 + FMA loops
// (src/kernels/rmsnorm.cpp:21-52, matvec_f32_f32.cpp:22-50,
// matvec_bf16_f32.cpp:48-68), so every dot product here is evaluated in their
// order: eight partials, partial l a chain of fused multiply-adds over
// elements l, l + 8, ...; the horizontal sum (p_i + p_{i+4}, then
// (s_0 + s_1) + (s_2 + s_3)); then the n % 8 tail as GCC compiles it for the
// reference's flags (f32 loops: the first four products rounded on their own
// and added in order when four or more remain, the rest fused; the bf16 tail:
// fused, summed on its own and added last).
//
// k_head_norm: one wave per row; lanes 0-7 run the eight chains of the sum of
//   squares over LDS copies of the row, then every lane writes its share of
//   (x * scale) * inv_rms.
// k_head_gemv: HBM-bound (V x H weights read once per group of up to four
//   rows). A block takes 32 vocabulary rows at a time; thread (row, chain)
//   runs one of the eight chains of one row. The weights go through LDS in
//   256-column chunks (coalesced 16-byte loads, the next chunk's in flight
//   while the chains run, rows padded so that the chains' strided reads are
//   free of bank conflicts), the normed rows' columns too.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "hsamp_wave.h"
#include "ultima_hsamp.h"

#pragma clang fp contract(off)

namespace hsamp {
namespace {

#ifndef HSAMP_HEAD_KC
#define HSAMP_HEAD_KC 256
#endif
constexpr int kHT = 256;        // threads of a gemv block
constexpr int kHR = 32;         // vocabulary rows per gemv block (8 chains each)
constexpr int kHKC = HSAMP_HEAD_KC;   // columns per LDS chunk

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// acc + a(0) b(0) + ... + a(t-1) b(t-1) as the reference's vectorised f32 tail
// (t < 8): when t >= 4 the first four products are rounded on their own.
template <class A, class B>
__device__ __forceinline__ float tail_f32(float acc, A a, B b, int t) {
    int i = 0;
    if (t >= 4)
        for (; i < 4; ++i) acc = acc + a(i) * b(i);
    for (; i < t; ++i) acc = __builtin_fmaf(a(i), b(i), acc);
    return acc;
}

// The horizontal sum of the eight partials held by lanes 8g .. 8g + 7 (lane
// 8g + l holds partial l); every lane of the group gets it.
__device__ __forceinline__ float hsum8_lanes(float p) {
    const float s = p + __shfl_xor(p, 4, 64);        // lanes l < 4: s_l = p_l + p_{l+4}
    const float s01 = s + __shfl_xor(s, 1, 64);      // lane 0: s_0 + s_1, lane 2: s_2 + s_3
    const float s23 = __shfl_xor(s01, 2, 64);
    const int l = lane_id() & 7;
    // (s_0 + s_1) + (s_2 + s_3), formed on lane 0 of the group and broadcast
    const float tot = (l & 2) ? s23 + s01 : s01 + s23;
    return __shfl(tot, lane_id() & ~7, 64);
}

constexpr int kHNC = 4096;      // hidden elements one k_head_norm pass stages in LDS

__global__ __launch_bounds__(64) void k_head_norm(const float* __restrict__ hidden, int64_t hstride, int H,
                                                 const float* __restrict__ scale, float eps,
                                                 float* __restrict__ normed) {
    __shared__ float xs[kHNC];
    const int r = blockIdx.x, lane = lane_id();
    const float* x = hidden + (int64_t)r * hstride;
    float* y = normed + (int64_t)r * H;
    const int H8 = H / 8 * 8;
    // the eight chains (lanes 0-7) over LDS copies of the row, kHNC at a time
    // (the whole wave copies; the chains' reads are independent of their sums)
    float p = 0.0f;
    for (int c0 = 0; c0 < H8; c0 += kHNC) {
        const int n = min(kHNC, H8 - c0);
        for (int i = lane; i < n; i += 64) xs[i] = x[c0 + i];
        __syncthreads();
        if (lane < 8) {
            // sixteen reads ahead of their multiply-adds (n is a multiple of 8)
            int k = lane;
            for (; k + 8 * 15 < n; k += 8 * 16) {
                float v[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) v[q] = xs[k + 8 * q];
#pragma unroll
                for (int q = 0; q < 16; ++q) p = __builtin_fmaf(v[q], v[q], p);
            }
            for (; k < n; k += 8) p = __builtin_fmaf(xs[k], xs[k], p);
        }
        __syncthreads();
    }
    float ss = __shfl(hsum8_lanes(p), 0, 64);
    ss = tail_f32(ss, [&](int i) { return x[H8 + i]; }, [&](int i) { return x[H8 + i]; }, H - H8);
    const float mean_sq = ss / (float)H;
    const float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (int i = lane; i < H; i += 64) y[i] = (x[i] * scale[i]) * inv_rms;
}

// WB: bf16 weights (else f32). BB: batch rows per block (1, 2 or 4). VEC:
// weight rows sit on 16-byte boundaries (16-byte loads; else element loads).
// Blocks stride over the 32-row tiles of the vocabulary. Per 256-column
// chunk, the weights and the normed rows' columns go from registers to LDS
// chain-major -- entry (row, column 8j + l) at [row][l][j] -- so that a
// chain reads eight of its steps with one 16-byte LDS read; the chunk after
// next is already in flight while this one's chains run.
template <bool WB, int BB, bool VEC>
__global__ __launch_bounds__(kHT) void k_head_gemv(const void* __restrict__ weight, int V, int H,
                                                   const float* __restrict__ normed, int rows,
                                                   float logit_scale, float* __restrict__ logits,
                                                   int64_t lstride) {
    using W = typename std::conditional<WB, uint16_t, float>::type;
    constexpr int ES = sizeof(W);
    constexpr int NJ = kHKC / 8;                      // steps of a chain per chunk
    constexpr int CS = NJ * ES + 16;                  // bytes per (row, chain), padded: conflict-free
    constexpr int RS = 8 * CS;                        // bytes per row
    constexpr int XS = NJ * 4 + 16;                   // bytes per (batch row, chain) of the normed rows
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* xsm = smem + kHR * RS;             // [BB][8][NJ] f32, chain-major
    const int tid = threadIdx.x;
    const int b0 = blockIdx.y * BB;
    const int nb = min(BB, rows - b0);
    const int ml = tid >> 3, l = tid & 7;
    const W* wb = static_cast<const W*>(weight);
    const int H8 = H / 8 * 8;
    const int nC = (H8 + kHKC - 1) / kHKC;
    const int nT = (V + kHR - 1) / kHR;
    const bool scaled = logit_scale != 1.0f && logit_scale != 0.0f;
    const float inv = scaled ? 1.0f / logit_scale : 1.0f;

    constexpr int VPR = kHKC * ES / 16;               // 16-byte vectors per tile row
    constexpr int NV = kHR * VPR / kHT;               // per thread
    constexpr int NX = (BB * kHKC + kHT - 1) / kHT;   // normed values per thread
    constexpr int EPV = 16 / ES;                      // elements per vector
    // two chunks in flight: A holds the even chunks, B the odd ones
    uint4 regA[NV], regB[NV];
    float xrA[NX], xrB[NX];
    // chunk c of tile rows m0 .. m0 + 31 into registers (past H8, past V: 0)
    auto load = [&](uint4 (&reg)[NV], float (&xr)[NX], int m0, int c) {
        const int c0 = c * kHKC;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = tid + i * kHT;
            const int row = v / VPR, col = (v % VPR) * EPV;   // first column of the vector
            const int m = m0 + row;
            uint4 q = make_uint4(0u, 0u, 0u, 0u);
            if (m < V) {
                const W* src = wb + (int64_t)m * H + c0 + col;
                if (VEC && c0 + col + EPV <= H8) {
                    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                    q = make_uint4(t.x, t.y, t.z, t.w);
                } else {
                    W e[EPV];
#pragma unroll
                    for (int j = 0; j < EPV; ++j) e[j] = (c0 + col + j < H8) ? src[j] : W(0);
                    q = *reinterpret_cast<const uint4*>(e);
                }
            }
            reg[i] = q;
        }
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int e = tid + i * kHT;
            const int b = e / kHKC, k = e % kHKC;
            xr[i] = (e < BB * kHKC && b < nb && c0 + k < H8) ? normed[(int64_t)(b0 + b) * H + c0 + k] : 0.0f;
        }
    };
    // registers -> LDS, chain-major: vector (row, columns col .. col + EPV - 1)
    // holds step col / 8 of chains col % 8 ...
    auto store = [&](const uint4 (&reg)[NV], const float (&xr)[NX]) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = tid + i * kHT;
            const int row = v / VPR, col = (v % VPR) * EPV;
            const W* e = reinterpret_cast<const W*>(&reg[i]);
#pragma unroll
            for (int q = 0; q < EPV; ++q) {
                const int cc = col + q;                   // column within the chunk
                *reinterpret_cast<W*>(smem + row * RS + (cc & 7) * CS + (cc >> 3) * ES) = e[q];
            }
        }
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int e = tid + i * kHT;
            if (e < BB * kHKC) {
                const int b = e / kHKC, k = e % kHKC;
                *reinterpret_cast<float*>(xsm + (b * 8 + (k & 7)) * XS + (k >> 3) * 4) = xr[i];
            }
        }
    };

    for (int t = blockIdx.x; t < nT; t += gridDim.x) {
        const int m0 = t * kHR;
        float acc[BB];
#pragma unroll
        for (int b = 0; b < BB; ++b) acc[b] = 0.0f;
        // this chunk's steps of the thread's chain, eight per LDS read
        auto chains = [&](int c) {
            const int nj = min(kHKC, H8 - c * kHKC) >> 3;
            const unsigned char* wrow = smem + ml * RS + l * CS;
            for (int j0 = 0; j0 < nj; j0 += 8) {
                float w[8];
                if (WB) {
                    const uint4 q = *reinterpret_cast<const uint4*>(wrow + j0 * 2);
                    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        w[2 * i] = __uint_as_float(d[i] << 16);
                        w[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
                    }
                } else {
                    const float4 q0 = *reinterpret_cast<const float4*>(wrow + j0 * 4);
                    const float4 q1 = *reinterpret_cast<const float4*>(wrow + j0 * 4 + 16);
                    w[0] = q0.x; w[1] = q0.y; w[2] = q0.z; w[3] = q0.w;
                    w[4] = q1.x; w[5] = q1.y; w[6] = q1.z; w[7] = q1.w;
                }
                const int jn = min(8, nj - j0);
#pragma unroll
                for (int b = 0; b < BB; ++b) {
                    const unsigned char* xrow = xsm + (b * 8 + l) * XS + j0 * 4;
                    const float4 x0 = *reinterpret_cast<const float4*>(xrow);
                    const float4 x1 = *reinterpret_cast<const float4*>(xrow + 16);
                    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    if (jn == 8) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) acc[b] = __builtin_fmaf(w[i], x[i], acc[b]);
                    } else {
                        for (int i = 0; i < jn; ++i) acc[b] = __builtin_fmaf(w[i], x[i], acc[b]);
                    }
                }
            }
        };
        if (nC > 0) load(regA, xrA, m0, 0);
        if (nC > 1) load(regB, xrB, m0, 1);
        for (int c = 0; c < nC; c += 2) {
            store(regA, xrA);
            __syncthreads();
            if (c + 2 < nC) load(regA, xrA, m0, c + 2);   // in flight for two chunks' chains
            chains(c);
            __syncthreads();                             // before the next chunk overwrites them
            if (c + 1 < nC) {
                store(regB, xrB);
                __syncthreads();
                if (c + 3 < nC) load(regB, xrB, m0, c + 3);
                chains(c + 1);
                __syncthreads();
            }
        }
        const int m = m0 + ml;
#pragma unroll
        for (int b = 0; b < BB; ++b) {
            const float hs = hsum8_lanes(acc[b]);
            if (b < nb && l == 0 && m < V) {
                const W* row = wb + (int64_t)m * H;
                const float* x = normed + (int64_t)(b0 + b) * H;
                const int tl = H - H8;
                float y;
                if (WB) {
                    float tail = 0.0f;
                    for (int i = 0; i < tl; ++i)
                        tail = __builtin_fmaf(bf16f(((const uint16_t*)row)[H8 + i]), x[H8 + i], tail);
                    y = hs + tail;
                } else {
                    y = tail_f32(hs, [&](int i) { return ((const float*)row)[H8 + i]; },
                                 [&](int i) { return x[H8 + i]; }, tl);
                }
                if (scaled) y = y * inv;
                logits[(int64_t)(b0 + b) * lstride + m] = y;
            }
        }
    }
}

template <bool WB, int BB>
hipError_t launch_gemv_bb(const ultima_hsamp_head* h, bool vec, int cus, hipStream_t s) {
    // enough blocks to fill every CU several times over, each striding over tiles
    const int tiles = (h->vocab + kHR - 1) / kHR;
    const dim3 grid(std::min(tiles, 8 * cus), (h->rows + BB - 1) / BB);
    constexpr int ES = WB ? 2 : 4;
    constexpr int NJ = kHKC / 8;
    const size_t lds = (size_t)kHR * 8 * (NJ * ES + 16) + (size_t)BB * 8 * (NJ * 4 + 16);
    if (vec)
        hipLaunchKernelGGL((k_head_gemv<WB, BB, true>), grid, dim3(kHT), lds, s, h->weight, h->vocab, h->hidden_dim,
                           h->normed, h->rows, h->logit_scale, h->logits, h->logits_stride);
    else
        hipLaunchKernelGGL((k_head_gemv<WB, BB, false>), grid, dim3(kHT), lds, s, h->weight, h->vocab,
                           h->hidden_dim, h->normed, h->rows, h->logit_scale, h->logits, h->logits_stride);
    return hipGetLastError();
}

// batch rows per block: one weight pass per group of up to four rows
template <bool WB>
hipError_t launch_gemv(const ultima_hsamp_head* h, bool vec, int cus, hipStream_t s) {
    if (h->rows == 1) return launch_gemv_bb<WB, 1>(h, vec, cus, s);
    if (h->rows == 2) return launch_gemv_bb<WB, 2>(h, vec, cus, s);
    return launch_gemv_bb<WB, 4>(h, vec, cus, s);
}

}  // namespace
}  // namespace hsamp

extern "C" int ultima_hsamp_lm_head(const ultima_hsamp_head* h, void* hip_stream) {
    using namespace hsamp;
    if (h == nullptr || h->hidden == nullptr || h->norm_scale == nullptr || h->weight == nullptr ||
        h->normed == nullptr || h->logits == nullptr)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (h->rows < 1 || h->hidden_dim < 1 || h->vocab < 1 || h->hidden_stride < h->hidden_dim ||
        h->logits_stride < h->vocab)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (h->weight_dtype != ULTIMA_HSAMP_F32 && h->weight_dtype != ULTIMA_HSAMP_BF16) return ULTIMA_HSAMP_ERR_INVALID;
    if (!(h->eps == h->eps) || !(h->logit_scale == h->logit_scale)) return ULTIMA_HSAMP_ERR_INVALID;
    // row offsets must fit the kernels' 32-bit index arithmetic within a row
    if ((int64_t)h->vocab * h->hidden_dim >= (int64_t)1 << 40) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    hipLaunchKernelGGL(k_head_norm, dim3(h->rows), dim3(64), 0, s, h->hidden, h->hidden_stride, h->hidden_dim,
                       h->norm_scale, h->eps, h->normed);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return ULTIMA_HSAMP_ERR_HIP;
    const int es = h->weight_dtype == ULTIMA_HSAMP_BF16 ? 2 : 4;
    const bool vec = (reinterpret_cast<uintptr_t>(h->weight) % 16 == 0) && (((int64_t)h->hidden_dim * es) % 16 == 0);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    }
    e = h->weight_dtype == ULTIMA_HSAMP_BF16 ? launch_gemv<true>(h, vec, cus, s) : launch_gemv<false>(h, vec, cus, s);
    return e == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}
