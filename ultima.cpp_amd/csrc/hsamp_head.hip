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
// k_head_norm: one 512-thread block per row; the row goes to LDS chain-major
//   (16 loads in flight per thread), lanes 0-7 run the eight chains of the
//   sum of squares with 16-byte LDS reads, then every thread writes its share
//   of (x * scale) * inv_rms from registers.
// k_head_gemv: HBM-bound (V x H weights read once per group of up to four
//   rows). One wave per 64 vocabulary rows, lane i running the eight chains
//   of its own row: the weights go through a row-major LDS tile in chunks of
//   128 bytes per row (coalesced 16-byte loads two chunks ahead, 16-byte
//   stores, 16-byte reads of one step of all eight chains).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "hsamp_wave.h"
#include "ultima_hsamp.h"

#pragma clang fp contract(off)

namespace hsamp {
namespace {

constexpr int kGRowBytes = 128;              // bytes of each weight row per gemv chunk
constexpr int kGRS = kGRowBytes + 16;         // LDS bytes per row of the gemv tile (padded)

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

constexpr int kNT = 512;                  // threads of a k_head_norm block
constexpr int kNQ = 16;                   // row elements per thread and pass
constexpr int kHNC = kNT * kNQ;           // row elements one pass stages in LDS (8192)
constexpr int kNCS = kHNC / 8 + 8;        // LDS stride of one chain (padded: conflict-free stores)

__global__ __launch_bounds__(kNT) void k_head_norm(const float* __restrict__ hidden, int64_t hstride, int H,
                                                  const float* __restrict__ scale, float eps,
                                                  float* __restrict__ normed) {
    // the row chain-major: element 8j + l of a pass at [l][j], so that chain l
    // reads four of its steps with one 16-byte LDS read
    __shared__ __attribute__((aligned(16))) float xs[8 * kNCS];
    __shared__ float ssum;
    const int r = blockIdx.x, tid = threadIdx.x;
    const float* x = hidden + (int64_t)r * hstride;
    float* y = normed + (int64_t)r * H;
    const int H8 = H / 8 * 8;
    float v[kNQ] = {}, g[kNQ];
    // every load of the thread's share in flight at once; the scale's too
    // (the output pass of a one-pass row takes x from these registers)
    auto load = [&](float (&d)[kNQ], const float* src, int c0, int n) {
#pragma unroll
        for (int q = 0; q < kNQ; ++q) {
            const int i = c0 + tid + q * kNT;
            d[q] = i < n ? src[i] : 0.0f;
        }
    };
    float p = 0.0f;   // chain l = tid (tid < 8)
    if (H <= kHNC) load(g, scale, 0, H);
    for (int c0 = 0; c0 < H8; c0 += kHNC) {
        const int n = min(kHNC, H8 - c0);
        load(v, x, c0, c0 + n);
        if (c0 > 0) __syncthreads();   // the previous pass's chains are done with xs
#pragma unroll
        for (int q = 0; q < kNQ; ++q) {
            const int i = tid + q * kNT;   // element i of the pass: chain i & 7, step i >> 3
            if (i < n) xs[(i & 7) * kNCS + (i >> 3)] = v[q];
        }
        __syncthreads();
        if (tid < 8) {
            // 16 steps per group of four 16-byte reads, the next group's reads
            // issued before this group's multiply-adds (n / 8 steps in all)
            const float4* c = reinterpret_cast<const float4*>(xs + tid * kNCS);
            const int n4 = n / 128;   // whole groups of 16 steps (n / 8 steps)
            float4 a[4], b[4];
            if (n4 > 0)
#pragma unroll
                for (int q = 0; q < 4; ++q) a[q] = c[q];
            for (int t = 0; t < n4; ++t) {
                if (t + 1 < n4)
#pragma unroll
                    for (int q = 0; q < 4; ++q) b[q] = c[4 * (t + 1) + q];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    p = __builtin_fmaf(a[q].x, a[q].x, p);
                    p = __builtin_fmaf(a[q].y, a[q].y, p);
                    p = __builtin_fmaf(a[q].z, a[q].z, p);
                    p = __builtin_fmaf(a[q].w, a[q].w, p);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) a[q] = b[q];
            }
            const float* cs = xs + tid * kNCS;
            for (int k = n4 * 16; k < n / 8; ++k) p = __builtin_fmaf(cs[k], cs[k], p);
        }
    }
    if (tid < 64) {
        float ss = __shfl(hsum8_lanes(p), 0, 64);
        ss = tail_f32(ss, [&](int i) { return x[H8 + i]; }, [&](int i) { return x[H8 + i]; }, H - H8);
        if (tid == 0) ssum = ss;
    }
    __syncthreads();
    const float mean_sq = ssum / (float)H;
    const float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    if (H <= kHNC) {
        // the row's x in v (its H8 part) and its scale in g
#pragma unroll
        for (int q = 0; q < kNQ; ++q) {
            const int i = tid + q * kNT;
            if (i < H) y[i] = ((i < H8 ? v[q] : x[i]) * g[q]) * inv_rms;
        }
    } else {
        for (int i = tid; i < H; i += kNT) y[i] = (x[i] * scale[i]) * inv_rms;
    }
}

// WB: bf16 weights (else f32). BB: batch rows per block (1, 2 or 4). VEC:
// weight rows sit on 16-byte boundaries (16-byte loads; else element loads).
// One wave per 64 vocabulary rows, lane i running the eight chains of row
// m0 + i. The weights arrive in chunks of 128 bytes of each row: coalesced
// 16-byte loads (eight lanes per row segment) into registers, two chunks
// ahead, then 16-byte stores into a row-major LDS tile (rows padded to 144
// bytes: conflict-free), from which each lane reads its own row 16 bytes at a
// time -- one step of all eight chains (bf16), or half a step (f32). The
// normed rows' columns of the chunk go through LDS too and are read as
// broadcasts. The block is the one wave: no barrier waits on another wave.
template <bool WB, int BB, bool VEC>
__global__ __launch_bounds__(64) void k_head_gemv(const void* __restrict__ weight, int V, int H,
                                                  const float* __restrict__ normed, int rows,
                                                  float logit_scale, float* __restrict__ logits,
                                                  int64_t lstride) {
    using W = typename std::conditional<WB, uint16_t, float>::type;
    constexpr int ES = sizeof(W);
    constexpr int KC = kGRowBytes / ES;               // columns per chunk
    constexpr int EPV = 16 / ES;                      // columns per 16-byte vector
    constexpr int NV = 64 * (kGRowBytes / 16) / 64;   // vectors per lane per chunk (8)
    constexpr int SB = 8 * ES;                        // bytes of one step (eight chains)
    __shared__ __attribute__((aligned(16))) unsigned char wl[64 * kGRS];
    __shared__ __attribute__((aligned(16))) float xl[BB][KC];
    const int lane = threadIdx.x;
    const int m0 = blockIdx.x * 64;
    const int b0 = blockIdx.y * BB;
    const int nb = min(BB, rows - b0);
    const W* wb = static_cast<const W*>(weight);
    const int H8 = H / 8 * 8;
    const int nC = (H8 + KC - 1) / KC;
    const bool scaled = logit_scale != 1.0f && logit_scale != 0.0f;
    const float inv = scaled ? 1.0f / logit_scale : 1.0f;

    // chunk c into registers: vector i of the lane is segment v % 8 of tile
    // row v / 8 (v = lane + 64 i); past H8 or past V: 0
    auto load = [&](uint4 (&reg)[NV], float (&xr)[BB], int c) {
        const int c0 = c * KC;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = lane + i * 64;
            const int m = m0 + (v >> 3), col = c0 + (v & 7) * EPV;
            uint4 q = make_uint4(0u, 0u, 0u, 0u);
            if (m < V) {
                const W* src = wb + (int64_t)m * H + col;
                if (VEC && col + EPV <= H8) {
                    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
                    q = make_uint4(t.x, t.y, t.z, t.w);
                } else {
                    W e[EPV];
#pragma unroll
                    for (int j = 0; j < EPV; ++j) e[j] = (col + j < H8) ? src[j] : W(0);
                    q = *reinterpret_cast<const uint4*>(e);
                }
            }
            reg[i] = q;
        }
#pragma unroll
        for (int b = 0; b < BB; ++b)
            xr[b] = (b < nb && lane < KC && c0 + lane < H8) ? normed[(int64_t)(b0 + b) * H + c0 + lane] : 0.0f;
    };
    auto store = [&](const uint4 (&reg)[NV], const float (&xr)[BB]) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = lane + i * 64;
            *reinterpret_cast<uint4*>(wl + (v >> 3) * kGRS + (v & 7) * 16) = reg[i];
        }
#pragma unroll
        for (int b = 0; b < BB; ++b)
            if (lane < KC) xl[b][lane] = xr[b];
    };
    float acc[BB][8];
#pragma unroll
    for (int b = 0; b < BB; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[b][l] = 0.0f;
    // the chunk's steps of the lane's eight chains
    auto chains = [&](int c) {
        const int nj = min(KC, H8 - c * KC) >> 3;
        const unsigned char* wr = wl + lane * kGRS;
        auto one = [&](int j) {
            float w[8];
            if (WB) {
                const uint4 q = *reinterpret_cast<const uint4*>(wr + j * SB);
                const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w[2 * i] = __uint_as_float(d[i] << 16);
                    w[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
                }
            } else {
                const float4 q0 = *reinterpret_cast<const float4*>(wr + j * SB);
                const float4 q1 = *reinterpret_cast<const float4*>(wr + j * SB + 16);
                w[0] = q0.x; w[1] = q0.y; w[2] = q0.z; w[3] = q0.w;
                w[4] = q1.x; w[5] = q1.y; w[6] = q1.z; w[7] = q1.w;
            }
#pragma unroll
            for (int b = 0; b < BB; ++b) {
                const float4 x0 = *reinterpret_cast<const float4*>(&xl[b][8 * j]);
                const float4 x1 = *reinterpret_cast<const float4*>(&xl[b][8 * j + 4]);
                const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[b][l] = __builtin_fmaf(w[l], x[l], acc[b][l]);
            }
        };
        if (nj == KC / 8) {
#pragma unroll
            for (int j = 0; j < KC / 8; ++j) one(j);
        } else {
            for (int j = 0; j < nj; ++j) one(j);
        }
    };
    // two chunks in flight: A holds the even chunks, B the odd ones (a third
    // set, and the compiler's own fences of a wave, measured slower)
    uint4 regA[NV], regB[NV];
    float xrA[BB], xrB[BB];
    auto step = [&](uint4 (&reg)[NV], float (&xr)[BB], int c) {
        store(reg, xr);
        __syncthreads();                                 // (the block is one wave)
        if (c + 2 < nC) load(reg, xr, c + 2);
        chains(c);
        __syncthreads();                                 // the reads are done before the next stores
    };
    if (nC > 0) load(regA, xrA, 0);
    if (nC > 1) load(regB, xrB, 1);
    for (int c = 0; c < nC; c += 2) {
        step(regA, xrA, c);
        if (c + 1 < nC) step(regB, xrB, c + 1);
    }
    // the horizontal sum, the tail, the logit scale; one row per lane
    const int m = m0 + lane;
    if (m >= V) return;
    const W* row = wb + (int64_t)m * H;
    const int tl = H - H8;
#pragma unroll
    for (int b = 0; b < BB; ++b) {
        if (b >= nb) break;
        const float* p = acc[b];
        const float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
        const float hs = (s0 + s1) + (s2 + s3);
        const float* x = normed + (int64_t)(b0 + b) * H;
        float y;
        if (WB) {
            float tail = 0.0f;
            for (int i = 0; i < tl; ++i) tail = __builtin_fmaf(bf16f(((const uint16_t*)row)[H8 + i]), x[H8 + i], tail);
            y = hs + tail;
        } else {
            y = tail_f32(hs, [&](int i) { return ((const float*)row)[H8 + i]; }, [&](int i) { return x[H8 + i]; }, tl);
        }
        if (scaled) y = y * inv;
        logits[(int64_t)(b0 + b) * lstride + m] = y;
    }
}

template <bool WB, int BB>
hipError_t launch_gemv_bb(const ultima_hsamp_head* h, bool vec, hipStream_t s) {
    // one wave per 64 vocabulary rows: every wave the same work, all resident
    // at once for real vocabularies (151936 rows: 2374 waves)
    const dim3 grid((h->vocab + 63) / 64, (h->rows + BB - 1) / BB);
    if (vec)
        hipLaunchKernelGGL((k_head_gemv<WB, BB, true>), grid, dim3(64), 0, s, h->weight, h->vocab, h->hidden_dim,
                           h->normed, h->rows, h->logit_scale, h->logits, h->logits_stride);
    else
        hipLaunchKernelGGL((k_head_gemv<WB, BB, false>), grid, dim3(64), 0, s, h->weight, h->vocab,
                           h->hidden_dim, h->normed, h->rows, h->logit_scale, h->logits, h->logits_stride);
    return hipGetLastError();
}

// batch rows per block: one weight pass per group of up to four rows
template <bool WB>
hipError_t launch_gemv(const ultima_hsamp_head* h, bool vec, hipStream_t s) {
    if (h->rows == 1) return launch_gemv_bb<WB, 1>(h, vec, s);
    if (h->rows == 2) return launch_gemv_bb<WB, 2>(h, vec, s);
    return launch_gemv_bb<WB, 4>(h, vec, s);
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
    hipLaunchKernelGGL(k_head_norm, dim3(h->rows), dim3(kNT), 0, s, h->hidden, h->hidden_stride, h->hidden_dim,
                       h->norm_scale, h->eps, h->normed);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return ULTIMA_HSAMP_ERR_HIP;
    const int es = h->weight_dtype == ULTIMA_HSAMP_BF16 ? 2 : 4;
    const bool vec = (reinterpret_cast<uintptr_t>(h->weight) % 16 == 0) && (((int64_t)h->hidden_dim * es) % 16 == 0);
    e = h->weight_dtype == ULTIMA_HSAMP_BF16 ? launch_gemv<true>(h, vec, s) : launch_gemv<false>(h, vec, s);
    return e == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}
