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
// k_head_gemv, one kernel for both: HBM-bound (V x H weights read once per
//   group of up to four rows). One wave per 64 vocabulary rows, lane i
//   running the eight chains of its own row: the weights go through a
//   row-major LDS tile in chunks of 128 bytes per row (coalesced 16-byte
//   loads one chunk ahead, 16-byte stores, 16-byte reads of one step of all
//   eight chains). Every wave first computes the rmsnorm of its batch rows
//   itself (the sum of squares' eight chains over chain-major LDS pieces of
//   the hidden rows, while its first weight chunk is in flight) and forms
//   the normed values chunk by chunk; the first waves also write the normed
//   rows out.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "hsamp_head.h"
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

// WB: bf16 weights (else f32). BB: batch rows per block (1, 2 or 4). VEC:
// weight rows sit on 16-byte boundaries (16-byte loads; else element loads).
// PRE: `hidden` already holds the head's input (normed and folded by
// k_head_prep): no norm here, the values are used as they are.
// One wave per 64 vocabulary rows, lane i running the eight chains of row
// m0 + i. The weights arrive in chunks of 128 bytes of each row: coalesced
// 16-byte loads (eight lanes per row segment) into registers, one chunk
// ahead, then 16-byte stores into a row-major LDS tile (rows padded to 144
// bytes: conflict-free), from which each lane reads its own row 16 bytes at a
// time -- one step of all eight chains (bf16), or half a step (f32). The
// normed rows' columns of the chunk go through LDS too and are read as
// broadcasts. The block is the one wave: no barrier waits on another wave.
template <bool WB, int BB, bool VEC, bool PRE>
__global__ __launch_bounds__(64) void k_head_gemv(const void* __restrict__ weight, int V, int H,
                                                  const float* __restrict__ hidden, int64_t hstride,
                                                  const float* __restrict__ scale, float eps,
                                                  float* __restrict__ normed, int rows,
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
    auto xrow = [&](int b) { return hidden + (int64_t)(b0 + min(b, nb - 1)) * hstride; };

    // chunk c into registers: vector i of the lane is segment v % 8 of tile
    // row v / 8 (v = lane + 64 i); with it the hidden values and the scale of
    // the chunk's column c0 + lane. Every load is unconditional, from an
    // address clamped into its array (rows past V read row V - 1, columns
    // past H8 the row's last whole vector): their values feed only rows that
    // are not stored and steps the chains skip. A branch around a load would
    // make the compiler wait for it at the join; these loads stay in flight
    // together.
    auto load = [&](uint4 (&reg)[NV], float (&xr)[BB], float& sr, int c) {
        const int c0 = c * KC;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = lane + i * 64;
            const int m = min(m0 + (v >> 3), V - 1), col = c0 + (v & 7) * EPV;
            const W* rowp = wb + (int64_t)m * H;
            if (VEC) {
                typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp + min(col, H8 - EPV)));
                reg[i] = make_uint4(t.x, t.y, t.z, t.w);
            } else {
                W e[EPV];
#pragma unroll
                for (int j = 0; j < EPV; ++j) e[j] = rowp[min(col + j, H8 - 1)];
                reg[i] = *reinterpret_cast<const uint4*>(e);
            }
        }
        const int k = min(c0 + lane, H8 - 1);
#pragma unroll
        for (int b = 0; b < BB; ++b) xr[b] = xrow(b)[k];
        sr = scale[k];
    };
    uint4 reg[NV];
    float xr[BB], sr;

    // The final rmsnorm of the wave's batch rows, computed by every wave (the
    // same bits as one kernel computing it once: the reference's eight chains
    // of x * x, its horizontal sum and tail, mean, 1 / sqrt(mean + eps)).
    // The rows go through the LDS tile in pieces of 2048 elements (2048 / BB
    // of each row), chain-major; lanes 8b + l run chain l of row b. The
    // first piece's loads are issued ahead of the first weight chunk's, so
    // that waiting for them leaves the weights in flight while the chains
    // run.
    constexpr int PE = 2048 / BB;                     // elements of each row per piece
    constexpr int PS = PE / 8 + 8;                    // LDS floats per (row, chain), padded
    constexpr int PT = 2048 / 64;                     // piece elements per lane
    float* xp = reinterpret_cast<float*>(wl);         // [BB][8][PS]
    float pv[PT];
    auto piece_load = [&](int p0) {
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            const int e = lane + 64 * t, b = e / PE, k = p0 + e % PE;
            pv[t] = xrow(b)[min(k, H8 - 1)];
        }
    };
    float p = 0.0f;   // lane 8b + l: chain l of batch row b
    const int nP = PRE ? 0 : (H8 + PE - 1) / PE;
    if (nP > 0) piece_load(0);
    __builtin_amdgcn_sched_barrier(0);
    if (nC > 0) load(reg, xr, sr, 0);
    __builtin_amdgcn_sched_barrier(0);
    for (int q = 0; q < nP; ++q) {
        const int p0 = q * PE;
        if (q > 0) __syncthreads();                      // the previous piece's chains are done
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            const int e = lane + 64 * t, b = e / PE, k = e % PE;   // k % 8 = lane % 8: chain lane % 8
            xp[(b * 8 + (k & 7)) * PS + (k >> 3)] = pv[t];
        }
        __syncthreads();
        if (q + 1 < nP) piece_load(p0 + PE);            // in flight while this piece's chains run
        const int n = min(PE, H8 - p0) >> 3;            // steps of this piece
        if (lane < 8 * BB) {
            const float4* cs = reinterpret_cast<const float4*>(xp + (lane >> 3) * 8 * PS + (lane & 7) * PS);
            // sixteen steps per group, the group's four reads issued together
            int g = 0;
            for (; 16 * (g + 1) <= n; ++g) {
                float4 v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = cs[4 * g + i];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p = __builtin_fmaf(v[i].x, v[i].x, p);
                    p = __builtin_fmaf(v[i].y, v[i].y, p);
                    p = __builtin_fmaf(v[i].z, v[i].z, p);
                    p = __builtin_fmaf(v[i].w, v[i].w, p);
                }
            }
            const float* cf = reinterpret_cast<const float*>(cs);
            for (int j = 16 * g; j < n; ++j) p = __builtin_fmaf(cf[j], cf[j], p);
        }
    }
    __syncthreads();                                     // the tile is free for the weights
    float rinv[BB];   // 1 / rms of each batch row (every lane)
    if (PRE) {
#pragma unroll
        for (int bb = 0; bb < BB; ++bb) rinv[bb] = 1.0f;
    } else {
        const float hs8 = hsum8_lanes(p);                 // lanes 8b .. 8b + 7: row b's horizontal sum
        const int b = min(lane >> 3, nb - 1);
        const float* x = xrow(b);
        const float ss = tail_f32(hs8, [&](int i) { return x[H8 + i]; }, [&](int i) { return x[H8 + i]; }, H - H8);
        const float mean_sq = ss / (float)H;
        const float r = 1.0f / sqrtf(mean_sq + eps);
#pragma unroll
        for (int bb = 0; bb < BB; ++bb) rinv[bb] = __shfl(r, 8 * bb, 64);
    }
    // the normed rows themselves (an output), 64 columns per wave
    if (!PRE && blockIdx.x * 64 < H) {
        for (int i = blockIdx.x * 64 + lane; i < H; i += gridDim.x * 64) {
            const float g = scale[i];
#pragma unroll
            for (int b = 0; b < BB; ++b)
                if (b < nb) normed[(int64_t)(b0 + b) * H + i] = (xrow(b)[i] * g) * rinv[b];
        }
    }
    // registers -> LDS; the normed values (x * scale) * (1 / rms), those of
    // columns past H8 (and of batch rows past the last) as 0
    auto store = [&](const uint4 (&reg)[NV], const float (&xr)[BB], float sr, int c) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = lane + i * 64;
            *reinterpret_cast<uint4*>(wl + (v >> 3) * kGRS + (v & 7) * 16) = reg[i];
        }
        const int c0 = c * KC;
#pragma unroll
        for (int b = 0; b < BB; ++b)
            if (lane < KC) xl[b][lane] = (b < nb && c0 + lane < H8) ? (PRE ? xr[b] : (xr[b] * sr) * rinv[b]) : 0.0f;
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
    // One chunk in flight while the chains run on the one before: chunk c to
    // LDS, chunk c + 1's loads issued into the registers just freed, then
    // c's chain steps. (Measured: two or three chunks ahead are slower --
    // 64 rows x 128 bytes per chunk spread each wave's requests over many
    // DRAM rows, and more of them in flight lowers the rate; a wave holds
    // 8 KB in flight, the chip ~19 MB, more than the latency asks for.)
    // No lane-dependent condition around a load: the compiler's waits are exact.
    for (int c = 0; c < nC; ++c) {
        store(reg, xr, sr, c);
        __syncthreads();                                 // (the block is one wave)
        if (c + 1 < nC) load(reg, xr, sr, c + 1);
        chains(c);
        __syncthreads();                                 // the reads are done before the next stores
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
        const float* x = xrow(b);
        auto xn = [&](int i) { return PRE ? x[H8 + i] : (x[H8 + i] * scale[H8 + i]) * rinv[b]; };   // normed value H8 + i
        float y;
        if (WB) {
            float tail = 0.0f;
            for (int i = 0; i < tl; ++i) tail = __builtin_fmaf(bf16f(((const uint16_t*)row)[H8 + i]), xn(i), tail);
            y = hs + tail;
        } else {
            y = tail_f32(hs, [&](int i) { return ((const float*)row)[H8 + i]; }, xn, tl);
        }
        if (scaled) y = y * inv;
        logits[(int64_t)(b0 + b) * lstride + m] = y;
    }
}

template <bool WB, int BB, bool PRE>
hipError_t launch_gemv_bb(const ultima_hsamp_head* h, bool vec, hipStream_t s) {
    // one wave per 64 vocabulary rows: every wave the same work, all resident
    // at once for real vocabularies (151936 rows: 2374 waves)
    const dim3 grid((h->vocab + 63) / 64, (h->rows + BB - 1) / BB);
    // PRE: the head's input is the prepared rows in `normed`
    const float* in = PRE ? h->normed : h->hidden;
    const int64_t in_stride = PRE ? h->hidden_dim : h->hidden_stride;
    if (vec)
        hipLaunchKernelGGL((k_head_gemv<WB, BB, true, PRE>), grid, dim3(64), 0, s, h->weight, h->vocab, h->hidden_dim,
                           in, in_stride, h->norm_scale, h->eps, h->normed, h->rows,
                           h->logit_scale, h->logits, h->logits_stride);
    else
        hipLaunchKernelGGL((k_head_gemv<WB, BB, false, PRE>), grid, dim3(64), 0, s, h->weight, h->vocab, h->hidden_dim,
                           in, in_stride, h->norm_scale, h->eps, h->normed, h->rows,
                           h->logit_scale, h->logits, h->logits_stride);
    return hipGetLastError();
}

// batch rows per block: one weight pass per group of up to four rows
template <bool WB, bool PRE>
hipError_t launch_gemv(const ultima_hsamp_head* h, bool vec, hipStream_t s) {
    if (h->rows == 1) return launch_gemv_bb<WB, 1, PRE>(h, vec, s);
    if (h->rows == 2) return launch_gemv_bb<WB, 2, PRE>(h, vec, s);
    return launch_gemv_bb<WB, 4, PRE>(h, vec, s);
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
    const bool dense = h->weight_dtype == ULTIMA_HSAMP_F32 || h->weight_dtype == ULTIMA_HSAMP_BF16;
    if (!dense && head_block_values(h->weight_dtype) == 0) return ULTIMA_HSAMP_ERR_INVALID;
    // PQ2_0's block sums of the activation are kept in LDS: at most 512 blocks
    if (h->weight_dtype == ULTIMA_HSAMP_HEAD_PQ2_0 && h->hidden_dim > 512 * 128) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    if (!(h->eps == h->eps) || !(h->logit_scale == h->logit_scale)) return ULTIMA_HSAMP_ERR_INVALID;
    // the fold's block: 0 (none) or a power of two the prep kernel's LDS holds
    if (h->fold_block < 0 || (h->fold_block & (h->fold_block - 1)) != 0) return ULTIMA_HSAMP_ERR_INVALID;
    if (h->fold_block > ULTIMA_HSAMP_MAX_FOLD_BLOCK) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    // row offsets must fit the kernels' 32-bit index arithmetic within a row
    if ((int64_t)h->vocab * h->hidden_dim >= (int64_t)1 << 40) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    // the fold applies when its block divides H (else the reference leaves
    // the rows as they are)
    const bool fold = h->fold_block > 0 && h->hidden_dim % h->fold_block == 0;
    hipError_t e = hipSuccess;
    if (!dense) {
        e = launch_head_prep(h, s);
        if (e == hipSuccess) e = launch_head_quant(h, s);
        return e == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
    }
    const int es = h->weight_dtype == ULTIMA_HSAMP_BF16 ? 2 : 4;
    const bool vec = (reinterpret_cast<uintptr_t>(h->weight) % 16 == 0) && (((int64_t)h->hidden_dim * es) % 16 == 0);
    if (fold) {
        e = launch_head_prep(h, s);
        if (e == hipSuccess)
            e = h->weight_dtype == ULTIMA_HSAMP_BF16 ? launch_gemv<true, true>(h, vec, s) : launch_gemv<false, true>(h, vec, s);
    } else {
        e = h->weight_dtype == ULTIMA_HSAMP_BF16 ? launch_gemv<true, false>(h, vec, s) : launch_gemv<false, false>(h, vec, s);
    }
    return e == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}
