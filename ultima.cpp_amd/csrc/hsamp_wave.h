// Wave-wide helpers of the gfx950 kernels (wave64): lane/wave ids, DPP scans
// and reductions, readlanes, and the wave-local LDS ordering fence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "libm_expf.h"

namespace hsamp {

using u64 = unsigned long long;

// Diagnostics: with HSAMP_PHASE_CLOCKS defined, thread 0 of each block records
// the 100 MHz real-time clock at numbered points of the stream and merge
// kernels (slot = block * 16 + point; stream blocks by logical id, merge
// blocks from 8192 + row); hsamp_phase_read copies the clocks out. Off by
// default: the macro then expands to nothing.
#ifdef HSAMP_PHASE_CLOCKS
__device__ unsigned long long g_phase[16384 * 16];
#define HSAMP_PHASE(blk, i)                                                          \
    do {                                                                             \
        if (threadIdx.x == 0) g_phase[(blk) * 16 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define HSAMP_PHASE(blk, i) ((void)0)
#endif

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ---- wave-wide reductions and scans through DPP ---------------------------------
// Shifts within 16-lane rows (row_shr 1, 2, 4, 8), then row_bcast:15 and
// row_bcast:31 across rows: an inclusive scan over the 64 lanes in six VALU
// steps, without the LDS crossbar that shuffles use. Lanes whose source lies
// outside the row keep `id` (the operation's identity); lane 63 ends with the
// whole wave's result.
template <int CTRL, int ROWM>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t id, uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)x, CTRL, ROWM, 0xF, false);
}
template <typename F>
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x, uint32_t id, F op) {
    x = op(x, dpp_u32<0x111, 0xF>(id, x));
    x = op(x, dpp_u32<0x112, 0xF>(id, x));
    x = op(x, dpp_u32<0x114, 0xF>(id, x));
    x = op(x, dpp_u32<0x118, 0xF>(id, x));
    x = op(x, dpp_u32<0x142, 0xA>(id, x));
    x = op(x, dpp_u32<0x143, 0xC>(id, x));
    return x;
}
__device__ __forceinline__ int wave_incl_sum_i(int x) {
    return (int)wave_scan_u32((uint32_t)x, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    x = wave_scan_u32(x, 0u, [](uint32_t a, uint32_t b) { return max(a, b); });
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
    x = wave_scan_u32(x, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return min(a, b); });
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
template <int CTRL, int ROWM>
__device__ __forceinline__ float dpp_f32(float id, float x) {
    return __uint_as_float(dpp_u32<CTRL, ROWM>(__float_as_uint(id), __float_as_uint(x)));
}
template <int CTRL, int ROWM>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = dpp_u32<CTRL, ROWM>(0u, (uint32_t)b), hi = dpp_u32<CTRL, ROWM>(0u, (uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// Inclusive scans (tree association: only for decisions taken with a margin).
__device__ __forceinline__ float wave_tree_prefix_f(float x) {
    x = x + dpp_f32<0x111, 0xF>(0.0f, x);
    x = x + dpp_f32<0x112, 0xF>(0.0f, x);
    x = x + dpp_f32<0x114, 0xF>(0.0f, x);
    x = x + dpp_f32<0x118, 0xF>(0.0f, x);
    x = x + dpp_f32<0x142, 0xA>(0.0f, x);
    x = x + dpp_f32<0x143, 0xC>(0.0f, x);
    return x;
}
__device__ __forceinline__ double wave_tree_prefix_d(double x) {
    x = x + dpp_f64<0x111, 0xF>(x);
    x = x + dpp_f64<0x112, 0xF>(x);
    x = x + dpp_f64<0x114, 0xF>(x);
    x = x + dpp_f64<0x118, 0xF>(x);
    x = x + dpp_f64<0x142, 0xA>(x);
    x = x + dpp_f64<0x143, 0xC>(x);
    return x;
}

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t b = f64_to_bits(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return bits_to_f64(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float wave_max_f(float v) {
    // (no NaN reaches it)
    v = fmaxf(v, dpp_f32<0x111, 0xF>(-__builtin_inff(), v));
    v = fmaxf(v, dpp_f32<0x112, 0xF>(-__builtin_inff(), v));
    v = fmaxf(v, dpp_f32<0x114, 0xF>(-__builtin_inff(), v));
    v = fmaxf(v, dpp_f32<0x118, 0xF>(-__builtin_inff(), v));
    v = fmaxf(v, dpp_f32<0x142, 0xA>(-__builtin_inff(), v));
    v = fmaxf(v, dpp_f32<0x143, 0xC>(-__builtin_inff(), v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// The value of lane (lane ^ M): DPP quad permutes for M = 1, 2, the
// swizzle's xor mode (within 32 lanes, no LDS memory) up to 16, a permute
// for 32.
template <int M>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t x) {
    if constexpr (M == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);
    else if constexpr (M <= 16) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, (M << 10) | 0x1F);
    else return (uint32_t)__shfl_xor((int)x, M, 64);
}
template <int M>
__device__ __forceinline__ u64 xor_lane_u64(u64 x) {
    return ((u64)xor_lane_u32<M>((uint32_t)(x >> 32)) << 32) | xor_lane_u32<M>((uint32_t)x);
}

// Orders the wave's LDS accesses around a cross-lane exchange. LDS operations
// of one wave complete in program order; the fences keep the compiler from
// moving accesses across.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace hsamp
