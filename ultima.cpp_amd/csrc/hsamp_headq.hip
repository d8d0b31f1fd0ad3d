// The logits producer's quantised heads and its Hadamard fold on gfx950
// (reference src/model/qwen_model.cpp:182-207, src/model/weight_dispatch.cpp:106-146).
//
// k_head_prep, one block per batch row: the final rmsnorm in the reference's
//   order (src/kernels/rmsnorm.cpp:21-52: eight fused chains of x * x, their
//   horizontal sum and tail, mean, 1 / sqrt(mean + eps), (x * scale) * inv),
//   then, for a folded head, the Hadamard fold (src/kernels/hadamard.cpp:9-44:
//   signs, the butterflies a + b / a - b over each block, * fl(1 / sqrt(block)))
//   in LDS; the head's input rows are written to `normed`.
//
// k_head_q<T, NWB, AL>, the quantised matvec: HBM-bound streams of GGUF blocks
//   whose per-element work (unpacking, the scale's rounding, the fused
//   multiply-add into the kernel's own partial sums) keeps the VALUs busy too.
//   The reference's AVX2 kernels fix each row's evaluation order -- for every
//   type a set of partial sums (8 to 64), each a chain of fused multiply-adds
//   over the row in a fixed element order, and a fixed reduction of them -- so
//   one lane runs one vocabulary row: all of that row's chains, in registers.
//   A wave takes 64 rows. Their bytes arrive in chunks of whole blocks (about
//   140-210 bytes per row): coalesced 16-byte buffer loads of the 64 rows'
//   aligned spans, one chunk ahead in registers, then into a row-major LDS tile
//   (rows padded to an odd number of dwords: lanes reading their own rows hit
//   different banks), from which each lane reads its row's dwords (a byte
//   shift by alignbyte where a block starts inside a dword). The activation is
//   the same for every lane: the chunk's values go through LDS with the
//   weights and are read as broadcasts. (Scalar loads would share the LDS
//   reads' wait counter and flat loads both counters: either makes a wait for
//   a tile read also wait for the next chunk in flight.) NWB waves share one
//   tile, each running a different batch row. Values are unpacked a dword at
//   a time into one value per byte (masks and shifts over four values at once)
//   and converted by byte.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "hsamp_head.h"
#include "ultima_hsamp.h"

#pragma clang fp contract(off)

namespace hsamp {
namespace {

// ---- exact IEEE half -> float (subnormals, Inf/NaN with their payload) -------
__device__ __forceinline__ float half_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return __uint_as_float(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        const float f = (float)m * 0x1p-24f;          // exact: m < 2^10
        return sign ? -f : f;
    }
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

__device__ __forceinline__ float hsum8(const float* p) {
    const float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
    return (s0 + s1) + (s2 + s3);
}

// signed byte e of w (one sign-extending convert), unsigned byte e of w as a
// float (one v_cvt_f32_ubyte), unsigned bit field [o, o + n) of w
__device__ __forceinline__ int sbyte(uint32_t w, int e) { return (int)(w << (24 - 8 * e)) >> 24; }
__device__ __forceinline__ float ubytef(uint32_t w, int e) { return (float)((w >> (8 * e)) & 0xFFu); }
__device__ __forceinline__ uint32_t ubits(uint32_t w, int o, int n) { return (w >> o) & ((1u << n) - 1u); }
// bits 0..3 of t, one to a byte (bit k -> bit 0 of byte k)
__device__ __forceinline__ uint32_t spread4(uint32_t t) { return ((t & 15u) * 0x00204081u) & 0x01010101u; }

// ---- the row's bytes in the LDS tile ------------------------------------------
// A lane's row chunk starts at byte `sh` (0..15) of its tile slot. AL = 1: the
// rows' chunk starts are dword-aligned in memory up to the chunk's shift class
// SC (0 or 2, known per chunk), so every dword read is one LDS read, plus an
// alignbyte by a constant where a field starts mid-dword; AL = 0: any byte
// alignment (two reads and an alignbyte by the lane's shift).
template <int AL>
struct RowBytes {
    const uint32_t* dw;   // the lane's slot + (sh >> 2) dwords
    int s3;               // sh & 3 (AL = 0 only)
    template <int SC>
    __device__ __forceinline__ uint32_t ld32(int off) const {
        if (AL) {
            const int o = SC + off;
            const int i = o >> 2, r = o & 3;
            if (r == 0) return dw[i];
            return __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], (uint32_t)r);
        }
        const int o = s3 + off;
        const int i = o >> 2;
        return __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], (uint32_t)(o & 3));
    }
};

// ---- the formats -----------------------------------------------------------------
// BE values per block, BB bytes per block, BPC blocks per chunk, NA partial
// sums per row. chunk(...) runs the lane's chains over one chunk of nblk
// blocks; x(i) is the chunk's activation value i (wave-uniform); final() the
// reference's reduction of the partial sums.

// Q8_0 (matvec_q8_0_f32.cpp:83-117): per block, lane l of a block accumulator
// takes values 8c + l (c = 0..3) from zero; then row partial l += d * it.
struct FQ8_0 {
    static constexpr int BE = 32, BB = 34, BPC = 4, NA = 8;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int nblk) {
#pragma unroll
        for (int j = 0; j < BPC; ++j) {
            if (j >= nblk) break;
            const int bo = j * BB;
            const float d = half_to_f32(rb.template ld32<SC>(bo) & 0xFFFFu);
            float bk[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) bk[l] = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t w = rb.template ld32<SC>(bo + 2 + 4 * t);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * t + e;
                    bk[i & 7] = __builtin_fmaf((float)sbyte(w, e), x(j * BE + i), bk[i & 7]);
                }
            }
#pragma unroll
            for (int l = 0; l < 8; ++l) a[l] = __builtin_fmaf(d, bk[l], a[l]);
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum8(a); }
};

// reduction of four eight-lane accumulators a[8g + l]
__device__ __forceinline__ float hsum4x8(const float* a) {
    float t[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) t[l] = (a[l] + a[8 + l]) + (a[16 + l] + a[24 + l]);
    return hsum8(t);
}
// reduction of eight eight-lane accumulators a[8g + l]
__device__ __forceinline__ float hsum8x8(const float* a) {
    float t[8];
#pragma unroll
    for (int l = 0; l < 8; ++l)
        t[l] = ((a[l] + a[8 + l]) + (a[16 + l] + a[24 + l])) + ((a[32 + l] + a[40 + l]) + (a[48 + l] + a[56 + l]));
    return hsum8(t);
}

// Q4_1 (matvec_q4_1_f32.cpp:47-75 over dequant_q4_1.cpp:46-54): value j =
// fl(nib * d + m) (fused as GCC compiles it), j + 16 the high nibble; value i
// into partial i.
struct FQ4_1 {
    static constexpr int BE = 32, BB = 20, BPC = 8, NA = 32;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int nblk) {
#pragma unroll
        for (int j = 0; j < BPC; ++j) {
            if (j >= nblk) break;
            const int bo = j * BB;
            const uint32_t h = rb.template ld32<SC>(bo);
            const float d = half_to_f32(h & 0xFFFFu), m = half_to_f32(h >> 16);
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t q = rb.template ld32<SC>(bo + 4 + 4 * t);
                lo[t] = q & 0x0F0F0F0Fu;
                hi[t] = (q >> 4) & 0x0F0F0F0Fu;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float v = __builtin_fmaf(ubytef(lo[i >> 2], i & 3), d, m);
                a[i] = __builtin_fmaf(v, x(j * BE + i), a[i]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float v = __builtin_fmaf(ubytef(hi[i >> 2], i & 3), d, m);
                a[16 + i] = __builtin_fmaf(v, x(j * BE + 16 + i), a[16 + i]);
            }
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum4x8(a); }
};

// Q5_0 (matvec_q5_0_f32.cpp:108-150): value i = (nib | bit i of qh << 4) - 16,
// scaled fl(q * d) on its own, into partial i.
struct FQ5_0 {
    static constexpr int BE = 32, BB = 22, BPC = 8, NA = 32;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int nblk) {
#pragma unroll
        for (int j = 0; j < BPC; ++j) {
            if (j >= nblk) break;
            const int bo = j * BB;
            const float d = half_to_f32(rb.template ld32<SC>(bo) & 0xFFFFu);
            const uint32_t qh = rb.template ld32<SC>(bo + 2);
            // the five-bit values, one to a byte: nibble | fifth bit << 4
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t q = rb.template ld32<SC>(bo + 6 + 4 * t);
                lo[t] = (q & 0x0F0F0F0Fu) | (spread4(qh >> (4 * t)) << 4);
                hi[t] = ((q >> 4) & 0x0F0F0F0Fu) | (spread4(qh >> (16 + 4 * t)) << 4);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float v = (ubytef(lo[i >> 2], i & 3) - 16.0f) * d;   // q - 16 exactly, then fl(q * d)
                a[i] = __builtin_fmaf(v, x(j * BE + i), a[i]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float v = (ubytef(hi[i >> 2], i & 3) - 16.0f) * d;
                a[16 + i] = __builtin_fmaf(v, x(j * BE + 16 + i), a[16 + i]);
            }
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum4x8(a); }
};

// the six-bit scale and min j of a Q4_K / Q5_K super-block's 12-byte table
// (bytes 4..15 of the block, in s[0..2]); matvec_q4k_f32.cpp:45-55
__device__ __forceinline__ void scale_min_k4(const uint32_t* s, int j, uint32_t& sc, uint32_t& mn) {
    auto byte = [&](int k) { return (s[k >> 2] >> (8 * (k & 3))) & 0xFFu; };
    if (j < 4) {
        sc = byte(j) & 63u;
        mn = byte(j + 4) & 63u;
    } else {
        sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Q4_K (matvec_q4k_f32.cpp:108-160): pair j's low nibbles are values 64j + l
// (partial l), its high nibbles 64j + 32 + l (partial 32 + l); each value
// fl(nib * d1 - m1) fused.
struct FQ4_K {
    static constexpr int BE = 256, BB = 144, BPC = 1, NA = 64;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int) {
        const uint32_t h = rb.template ld32<SC>(0);
        const float d = half_to_f32(h & 0xFFFFu), dmin = half_to_f32(h >> 16);
        uint32_t s[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) s[k] = rb.template ld32<SC>(4 + 4 * k);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t sc0, mn0, sc1, mn1;
            scale_min_k4(s, 2 * j, sc0, mn0);
            scale_min_k4(s, 2 * j + 1, sc1, mn1);
            const float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
            const float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t q = rb.template ld32<SC>(16 + 32 * j + 4 * t);
                lo[t] = q & 0x0F0F0F0Fu;
                hi[t] = (q >> 4) & 0x0F0F0F0Fu;
            }
#pragma unroll
            for (int l = 0; l < 32; ++l) {
                const float v = __builtin_fmaf(ubytef(lo[l >> 2], l & 3), d1, -m1);
                a[l] = __builtin_fmaf(v, x(64 * j + l), a[l]);
            }
#pragma unroll
            for (int l = 0; l < 32; ++l) {
                const float v = __builtin_fmaf(ubytef(hi[l >> 2], l & 3), d2, -m2);
                a[32 + l] = __builtin_fmaf(v, x(64 * j + 32 + l), a[32 + l]);
            }
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum8x8(a); }
};

// Q5_K (matvec_q5k_f32.cpp:48-80 over dequant_q5k.cpp:57-93): value e of the
// super-block = fl(d1 * q - m1) (fused as GCC compiles it) into partial e % 32,
// in increasing e.
struct FQ5_K {
    static constexpr int BE = 256, BB = 176, BPC = 1, NA = 32;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int) {
        const uint32_t h = rb.template ld32<SC>(0);
        const float d = half_to_f32(h & 0xFFFFu), dmin = half_to_f32(h >> 16);
        uint32_t s[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) s[k] = rb.template ld32<SC>(4 + 4 * k);
        uint32_t qh[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) qh[t] = rb.template ld32<SC>(16 + 4 * t);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t sc0, mn0, sc1, mn1;
            scale_min_k4(s, 2 * j, sc0, mn0);
            scale_min_k4(s, 2 * j + 1, sc1, mn1);
            const float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
            const float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
            // the five-bit values, one to a byte
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t q = rb.template ld32<SC>(48 + 32 * j + 4 * t);
                lo[t] = (q & 0x0F0F0F0Fu) | (((qh[t] >> (2 * j)) & 0x01010101u) << 4);
                hi[t] = ((q >> 4) & 0x0F0F0F0Fu) | (((qh[t] >> (2 * j + 1)) & 0x01010101u) << 4);
            }
#pragma unroll
            for (int l = 0; l < 32; ++l)
                a[l] = __builtin_fmaf(__builtin_fmaf(d1, ubytef(lo[l >> 2], l & 3), -m1), x(64 * j + l), a[l]);
#pragma unroll
            for (int l = 0; l < 32; ++l)
                a[l] = __builtin_fmaf(__builtin_fmaf(d2, ubytef(hi[l >> 2], l & 3), -m2), x(64 * j + 32 + l), a[l]);
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum4x8(a); }
};

// Q6_K (matvec_q6k_f32.cpp:99-169): per half, runs r = 0..3 of 32 six-bit
// values q - 32, value l of run r scaled fl(q * fl(d * sc[2r + l / 16])) on its
// own and fused into partial (r % 2) * 32 + l, runs in order.
struct FQ6_K {
    static constexpr int BE = 256, BB = 210, BPC = 1, NA = 64;
    template <int SC, class RB, class X>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, float* a, int) {
        const float d = half_to_f32(rb.template ld32<SC>(208) & 0xFFFFu);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t sw0 = rb.template ld32<SC>(192 + 8 * half), sw1 = rb.template ld32<SC>(196 + 8 * half);
            float s[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) s[i] = d * (float)sbyte(i < 4 ? sw0 : sw1, i & 3);
            // per dword of ql / qh: four six-bit values of each run, one to a byte
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t l0 = rb.template ld32<SC>(64 * half + 4 * t);
                const uint32_t l1 = rb.template ld32<SC>(64 * half + 32 + 4 * t);
                const uint32_t h = rb.template ld32<SC>(128 + 32 * half + 4 * t);
                uint32_t q[4];
                q[0] = (l0 & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
                q[1] = (l1 & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
                q[2] = ((l0 >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
                q[3] = ((l1 >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int l = 4 * t + e;
                        const int p = (r & 1) * 32 + l;
                        const float v = (ubytef(q[r], e) - 32.0f) * s[2 * r + (l >> 4)];   // q - 32 exactly
                        a[p] = __builtin_fmaf(v, x(128 * half + 32 * r + l), a[p]);
                    }
            }
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return hsum8x8(a); }
};

// PQ2_0 (matvec_pq2_0_f32.cpp:111-184, its vectorised path): per block, lane
// l of one accumulator takes, for code position j = 0..3 and byte group
// g = 0..3, byte i = 8g + l's code j times x[4i + j] (fused, from zero); the
// row sum += d * (horizontal sum - the block's plain sequential sum of x)
// (fused as GCC compiles it). a[0] holds the row sum; the block sums come
// from bs(j).
struct FPQ2_0 {
    static constexpr int BE = 128, BB = 34, BPC = 4, NA = 1;
    template <int SC, class RB, class X, class BS>
    __device__ __forceinline__ static void chunk(const RB& rb, const X& x, const BS& bs, float* a, int nblk) {
#pragma unroll
        for (int jb = 0; jb < BPC; ++jb) {
            if (jb >= nblk) break;
            const int bo = jb * BB;
            const float d = half_to_f32(rb.template ld32<SC>(bo) & 0xFFFFu);
            uint32_t c[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) c[t] = rb.template ld32<SC>(bo + 2 + 4 * t);
            float acc[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
            // lane l of the accumulator: code position j outer, byte group g
            // inner, byte i = 8g + l's code times x[4i + j]
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t cj = (c[t] >> (2 * j)) & 0x03030303u;   // codes j of bytes 4t .. 4t + 3
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * t + e, l = i & 7;
                        acc[l] = __builtin_fmaf(ubytef(cj, e), x(jb * BE + 4 * i + j), acc[l]);
                    }
                }
            a[0] = __builtin_fmaf(d, hsum8(acc) - bs(jb), a[0]);
        }
    }
    __device__ __forceinline__ static float final(const float* a) { return a[0]; }
};

template <int T> struct FmtOf;
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q4_K> { using F = FQ4_K; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q5_K> { using F = FQ5_K; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q6_K> { using F = FQ6_K; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q8_0> { using F = FQ8_0; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q4_1> { using F = FQ4_1; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_Q5_0> { using F = FQ5_0; };
template <> struct FmtOf<ULTIMA_HSAMP_HEAD_PQ2_0> { using F = FPQ2_0; };

constexpr int kMaxPqBlocks = 512;   // PQ2_0 block sums kept in LDS: H <= 65536

// T: head type; NWB: waves (batch rows) per block; AL: every row's chunk
// starts dword-aligned up to the chunk's shift class (see RowBytes).
// The block's 64 rows are read through one buffer resource based at the
// block's first row (16-byte aligned down; `delta` bytes before it): 32-bit
// offsets, loads past the head's end read 0, and the loads count only in the
// vector memory counter (waits for LDS reads do not wait for them).
template <int T, int NWB, int AL>
__global__ __launch_bounds__(64 * NWB) void k_head_q(const unsigned char* __restrict__ w, int V, int H, int64_t rb,
                                                     const float* __restrict__ xin, int rows, float logit_scale,
                                                     float* __restrict__ logits, int64_t lstride) {
    using F = typename FmtOf<T>::F;
    constexpr int CE = F::BE * F::BPC;                 // values per chunk
    constexpr int CB = F::BB * F::BPC;                 // bytes per chunk (whole blocks)
    constexpr int NVR = (CB + 15 + 15) / 16;           // 16-byte vectors of a row's aligned span
    constexpr int SLOT = 4 * NVR + 3;                  // dwords per tile row (odd: banks)
    constexpr int NV_T = (64 * NVR + 64 * NWB - 1) / (64 * NWB);   // vectors per thread per chunk
    constexpr int NX = (CE * 4 / 16 + 63) / 64;        // 16-byte vectors of the activation per lane per chunk
    constexpr bool PQ = T == ULTIMA_HSAMP_HEAD_PQ2_0;
    __shared__ uint32_t tile[64 * SLOT + 4];
    __shared__ __attribute__((aligned(16))) float xl[NWB][CE];
    __shared__ float bsum[PQ ? NWB * kMaxPqBlocks : 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = blockIdx.x * 64;
    const int b = blockIdx.y * NWB + wave;
    const int bb = b < rows ? b : rows - 1;
    const int nb = H / F::BE;                          // blocks per row
    const int nC = (nb + F::BPC - 1) / F::BPC;

    // the block's rows: [base, base + nrec) with base 16-byte aligned and nrec
    // rounded up to 16 bytes (a 16-byte load is out of range as a whole when
    // it reaches past nrec: the granule holding the rows' last byte is read in
    // full; it lies in that byte's page)
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(w) + (uintptr_t)((int64_t)m0 * rb);
    const uint32_t delta = (uint32_t)(b0 & 15u);
    const int64_t rows_here = min(64, V - m0);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(b0 - delta), (short)0, (int)((delta + rows_here * rb + 15) & ~(int64_t)15), 0x00020000);
    // the wave's activation row
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(xin + (int64_t)bb * H), (short)0, H * 4, 0x00020000);

    if (PQ) {
        // the activation's block sums, plain sequential float sums, lane k
        // taking blocks k, k + 64, ...
        const float* xrow = xin + (int64_t)bb * H;
        for (int k = lane; k < nb; k += 64) {
            const float* xs = xrow + (int64_t)k * F::BE;
            float sum = 0.0f;
            for (int i = 0; i < F::BE; i += 8) {
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = xs[i + e];
#pragma unroll
                for (int e = 0; e < 8; ++e) sum = sum + v[e];
            }
            bsum[wave * kMaxPqBlocks + k] = sum;
        }
    }

    // vector i of this thread: 16 bytes seg of tile row r's aligned span;
    // its offset within the block's resource for chunk c is
    // ((rofs + c CB) & ~15) + 16 seg
    uint32_t rofs[NV_T];
    int vseg[NV_T];
#pragma unroll
    for (int i = 0; i < NV_T; ++i) {
        const int v = min(tid + 64 * NWB * i, 64 * NVR - 1);
        const int r = v / NVR;
        vseg[i] = v - r * NVR;
        rofs[i] = delta + (uint32_t)((int64_t)r * rb);
    }
    uint4 reg[NV_T];
    uint4 xv[NX];
    // Only the granules of the row's span are asked for (an offset past the
    // resource's range makes the rest read 0 without touching memory), and
    // the loads keep the default cache policy: a chunk's span shares its
    // first and last 128-byte lines with the chunks before and after it,
    // which then find them in L2.
    auto load = [&](int c) {
        const uint32_t nbytes = (uint32_t)(min(F::BPC, nb - c * F::BPC) * F::BB);
#pragma unroll
        for (int i = 0; i < NV_T; ++i) {
            const uint32_t a0 = rofs[i] + (uint32_t)(c * CB);
            const uint32_t lo = a0 & ~15u, end = a0 + nbytes;
            uint32_t o = lo + 16u * (uint32_t)vseg[i];
            o = o < end ? o : 0xFFFFFFF0u;
            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(wr, o, 0, 0);
            reg[i] = make_uint4(t.x, t.y, t.z, t.w);
        }
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)(16 * (lane + 64 * i)), c * CE * 4, 0);
            xv[i] = make_uint4(t.x, t.y, t.z, t.w);
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int i = 0; i < NV_T; ++i) {
            const int v = tid + 64 * NWB * i;
            if ((64 * NVR) % (64 * NWB) == 0 || v < 64 * NVR) {
                const int r = v / NVR, seg = v - r * NVR;
                uint32_t* s = tile + r * SLOT + 4 * seg;
                s[0] = reg[i].x;
                s[1] = reg[i].y;
                s[2] = reg[i].z;
                s[3] = reg[i].w;
            }
        }
#pragma unroll
        for (int i = 0; i < NX; ++i)
            if ((CE * 4 / 16) % 64 == 0 || lane + 64 * i < CE * 4 / 16)
                *reinterpret_cast<uint4*>(&xl[wave][4 * (lane + 64 * i)]) = xv[i];
    };

    float a[F::NA];
#pragma unroll
    for (int i = 0; i < F::NA; ++i) a[i] = 0.0f;
    const uint32_t lofs = delta + (uint32_t)((int64_t)lane * rb);   // the lane's row in the resource
    if (nC > 0) load(0);
    for (int c = 0; c < nC; ++c) {
        store();
        __syncthreads();
        if (c + 1 < nC) load(c + 1);
        const int nblk = min(F::BPC, nb - c * F::BPC);
        const int sh = (int)((lofs + (uint32_t)(c * CB)) & 15u);
        RowBytes<AL> rbx;
        rbx.dw = tile + lane * SLOT + (sh >> 2);
        rbx.s3 = sh & 3;
        const float* xw = xl[wave];
        auto x = [&](int i) { return xw[i]; };
        auto run = [&](auto sc) {
            constexpr int S = decltype(sc)::value;
            if constexpr (PQ) {
                const float* bsw = bsum + wave * kMaxPqBlocks + c * F::BPC;
                auto bs = [&](int j) { return bsw[j]; };
                F::template chunk<S>(rbx, x, bs, a, nblk);
            } else {
                F::template chunk<S>(rbx, x, a, nblk);
            }
        };
        // the chunk's shift class: chunk starts move by CB % 4 bytes per chunk
        if (AL && (CB & 3) && (c & 1))
            run(std::integral_constant<int, 2>());
        else
            run(std::integral_constant<int, 0>());
        __syncthreads();
    }
    const int m = m0 + lane;
    if (b >= rows || m >= V) return;
    float y = F::final(a);
    if (logit_scale != 1.0f && logit_scale != 0.0f) y = y * (1.0f / logit_scale);
    logits[(int64_t)b * lstride + m] = y;
}

template <int T, int NWB>
hipError_t launch_q_nwb(const ultima_hsamp_head* h, const float* xin, int64_t rb, bool al, hipStream_t s) {
    const dim3 grid((h->vocab + 63) / 64, (h->rows + NWB - 1) / NWB);
    const unsigned char* wp = static_cast<const unsigned char*>(h->weight);
    if (al)
        hipLaunchKernelGGL((k_head_q<T, NWB, 1>), grid, dim3(64 * NWB), 0, s, wp, h->vocab, h->hidden_dim, rb, xin,
                           h->rows, h->logit_scale, h->logits, h->logits_stride);
    else
        hipLaunchKernelGGL((k_head_q<T, NWB, 0>), grid, dim3(64 * NWB), 0, s, wp, h->vocab, h->hidden_dim, rb, xin,
                           h->rows, h->logit_scale, h->logits, h->logits_stride);
    return hipGetLastError();
}

template <int T>
hipError_t launch_q(const ultima_hsamp_head* h, const float* xin, int64_t rb, bool al, hipStream_t s) {
    if (h->rows == 1) return launch_q_nwb<T, 1>(h, xin, rb, al, s);
    if (h->rows == 2) return launch_q_nwb<T, 2>(h, xin, rb, al, s);
    return launch_q_nwb<T, 4>(h, xin, rb, al, s);
}

// ---- the norm and the fold -------------------------------------------------------

constexpr int kPrepThreads = 1024;

// One block per batch row. The sum of squares' eight chains run on eight
// threads of wave 0 (the reference's order: chain l over elements l, l + 8,
// ...); the normed row goes to LDS when a fold follows (one fold block at a
// time), else straight out.
__global__ __launch_bounds__(kPrepThreads) void k_head_prep(const float* __restrict__ hidden, int64_t hstride,
                                                            const float* __restrict__ scale, float eps, int H,
                                                            int fold_block, const float* __restrict__ signs,
                                                            float* __restrict__ normed) {
    __shared__ float red[8];
    __shared__ float buf[ULTIMA_HSAMP_MAX_FOLD_BLOCK];
    const int row = blockIdx.x;
    const float* x = hidden + (int64_t)row * hstride;
    float* y = normed + (int64_t)row * H;
    const int tid = threadIdx.x;
    const int H8 = H / 8 * 8;
    if (tid < 8) {
        float p = 0.0f;
        int k = tid;
        for (; k + 8 * 7 < H8; k += 64) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = x[k + 8 * e];
#pragma unroll
            for (int e = 0; e < 8; ++e) p = __builtin_fmaf(v[e], v[e], p);
        }
        for (; k < H8; k += 8) p = __builtin_fmaf(x[k], x[k], p);
        red[tid] = p;
    }
    __syncthreads();
    float ss = hsum8(red);
    // the tail as GCC compiles the reference's vectorised loop: the first four
    // products rounded on their own when four or more remain, the rest fused
    {
        const int t = H - H8;
        int i = 0;
        if (t >= 4)
            for (; i < 4; ++i) ss = ss + x[H8 + i] * x[H8 + i];
        for (; i < t; ++i) ss = __builtin_fmaf(x[H8 + i], x[H8 + i], ss);
    }
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    const bool fold = fold_block > 0 && H % fold_block == 0;
    if (!fold) {
        for (int i = tid; i < H; i += kPrepThreads) y[i] = (x[i] * scale[i]) * inv;
        return;
    }
    const float finv = 1.0f / sqrtf((float)fold_block);
    for (int off = 0; off < H; off += fold_block) {
        for (int i = tid; i < fold_block; i += kPrepThreads) {
            const float v = (x[off + i] * scale[off + i]) * inv;
            buf[i] = signs != nullptr ? v * signs[off + i] : v;
        }
        __syncthreads();
        for (int len = 1; len < fold_block; len <<= 1) {
            for (int p = tid; p < fold_block / 2; p += kPrepThreads) {
                const int j = (p / len) * 2 * len + (p % len);
                const float u = buf[j], v = buf[j + len];
                buf[j] = u + v;
                buf[j + len] = u - v;
            }
            __syncthreads();
        }
        for (int i = tid; i < fold_block; i += kPrepThreads) y[off + i] = fold_block >= 2 ? buf[i] * finv : buf[i];
        __syncthreads();
    }
}

// logits of 0 (a hidden size that is not a whole number of the type's blocks)
__global__ void k_head_zero(float* __restrict__ logits, int64_t lstride, int V) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < V) logits[(int64_t)blockIdx.y * lstride + i] = 0.0f;
}

}  // namespace

int head_block_values(int dtype) {
    switch (dtype) {
        case ULTIMA_HSAMP_HEAD_Q4_K: case ULTIMA_HSAMP_HEAD_Q5_K: case ULTIMA_HSAMP_HEAD_Q6_K: return 256;
        case ULTIMA_HSAMP_HEAD_Q8_0: case ULTIMA_HSAMP_HEAD_Q4_1: case ULTIMA_HSAMP_HEAD_Q5_0: return 32;
        case ULTIMA_HSAMP_HEAD_PQ2_0: return 128;
        default: return 0;
    }
}

int head_block_bytes(int dtype) {
    switch (dtype) {
        case ULTIMA_HSAMP_HEAD_Q4_K: return 144;
        case ULTIMA_HSAMP_HEAD_Q5_K: return 176;
        case ULTIMA_HSAMP_HEAD_Q6_K: return 210;
        case ULTIMA_HSAMP_HEAD_Q8_0: return 34;
        case ULTIMA_HSAMP_HEAD_Q4_1: return 20;
        case ULTIMA_HSAMP_HEAD_Q5_0: return 22;
        case ULTIMA_HSAMP_HEAD_PQ2_0: return 34;
        default: return 0;
    }
}

hipError_t launch_head_prep(const ultima_hsamp_head* h, hipStream_t s) {
    hipLaunchKernelGGL(k_head_prep, dim3(h->rows), dim3(kPrepThreads), 0, s, h->hidden, h->hidden_stride,
                       h->norm_scale, h->eps, h->hidden_dim, h->fold_block, h->fold_signs, h->normed);
    return hipGetLastError();
}

hipError_t launch_head_quant(const ultima_hsamp_head* h, hipStream_t s) {
    const int be = head_block_values(h->weight_dtype);
    const int64_t H = h->hidden_dim;
    if (H % be != 0) {
        hipLaunchKernelGGL(k_head_zero, dim3((h->vocab + 255) / 256, h->rows), dim3(256), 0, s, h->logits,
                           h->logits_stride, h->vocab);
        return hipGetLastError();
    }
    const int64_t rb = H / be * head_block_bytes(h->weight_dtype);
    // dword-aligned rows: every chunk starts at a multiple of 4 bytes, up to
    // the shift class its index gives
    const bool al = reinterpret_cast<uintptr_t>(h->weight) % 4 == 0 && rb % 4 == 0;
    switch (h->weight_dtype) {
        case ULTIMA_HSAMP_HEAD_Q4_K: return launch_q<ULTIMA_HSAMP_HEAD_Q4_K>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_Q5_K: return launch_q<ULTIMA_HSAMP_HEAD_Q5_K>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_Q6_K: return launch_q<ULTIMA_HSAMP_HEAD_Q6_K>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_Q8_0: return launch_q<ULTIMA_HSAMP_HEAD_Q8_0>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_Q4_1: return launch_q<ULTIMA_HSAMP_HEAD_Q4_1>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_Q5_0: return launch_q<ULTIMA_HSAMP_HEAD_Q5_0>(h, h->normed, rb, al, s);
        case ULTIMA_HSAMP_HEAD_PQ2_0: return launch_q<ULTIMA_HSAMP_HEAD_PQ2_0>(h, h->normed, rb, al, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace hsamp
