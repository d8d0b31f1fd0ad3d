// Exact sequential float32 sums in parallel, and the full-vocabulary row
// machinery built on them (block helpers, LDS tables, the top-p driver). Used
// by k_full in hsamp_kernels.hip and by the test kit that pins the engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hsamp_plan.h"
#include "hsamp_wave.h"

namespace hsamp {

#ifdef HSAMP_PHASE_CLOCKS
__device__ __forceinline__ void g_phase_lv(int blk, int level) { g_phase[(14000 + blk) * 16 + level] = __builtin_amdgcn_s_memrealtime(); }
#else
__device__ __forceinline__ void g_phase_lv(int, int) {}
#endif

// ---- full-vocabulary rows ---------------------------------------------------------
// Sampling rows whose top-k is off (top_k == 0 or >= V) or above kLimitK: the
// whole transformed row goes through softmax, top-p, min-p and the draw
// (sampler.cpp:109-182). One block of kFT threads per row; the row's
// transformed logits and softmax numerators live in global scratch (fullv,
// fullp, padded to whole windows).
//
// Exact sequential float sums. softmax_probs (sampler.cpp:124-142) divides by
// a float sum taken in index order, and apply_top_p (:146-164) compares a
// float running sum taken in (p desc, index asc) order with top_p. Both are
// chains of up to V roundings, reproduced here exactly and in parallel: while
// a running sum s >= 0 stays in one binade [2^E, 2^(E+1)) (E = -126 also
// covers the subnormals), s = M * 2^(E-23) for an integer M < 2^24, and
// adding x >= 0 adds x rounded to a multiple of 2^(E-23): an integer
// increment that depends on x alone, except when x lies exactly half-way
// between two multiples (then M's parity decides: round half to even).
// Groups of values (windows of consecutive ids, buckets of probability keys)
// are summed as integers at the binade an approximate prefix predicts; the
// few groups where the sum leaves its binade, a half-way value occurs, the
// prediction fails or (top-p) the threshold is reached are replayed value by
// value from the exact state, in 64-value steps of one wave.

constexpr int kFT = 1024;             // threads of a k_full block
constexpr int kFW = kFT / 64;         // its waves
constexpr int kFWin = 512;            // ids of an index-order window per 512-step (64 lanes x 8)
constexpr int kFMaxWin = 2048;        // windows the LDS tables hold
constexpr int kFNB = 4096;            // top-p buckets
constexpr int kFSort = 512;           // bucket values one wave sorts in LDS

// Exact state of a running float32 sum of values >= 0: s = M * 2^(E-23),
// E >= -126, M < 2^24, M >= 2^23 unless E == -126.
struct XState {
    int E;
    uint32_t M;
};

// x = X * 2^(ex-23) with ex >= -126 (subnormals: ex = -126, X < 2^23).
__device__ __forceinline__ void fparts(float x, int& ex, uint32_t& X) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t f = (b >> 23) & 255u;
    ex = (int)max(f, 1u) - 127;
    X = (b & 0x7FFFFFu) | (f != 0u ? 0x800000u : 0u);
}

__device__ __forceinline__ float xs_value(XState s) {
    return s.M >= 0x800000u ? __uint_as_float(((uint32_t)(s.E + 127) << 23) | (s.M & 0x7FFFFFu))
                            : __uint_as_float(s.M);
}

// Increment of x >= 0 at binade E in units of 2^(E-23), half-way values
// rounded up (tie: round half to even then decides by parity); big: x >= 2^E
// or more, the sum leaves the binade.
__device__ __forceinline__ uint32_t xinc(float x, int E, bool& tie, bool& big) {
    int ex;
    uint32_t X;
    fparts(x, ex, X);
    const int d = E - ex;
    tie = false;
    big = false;
    if (X == 0u || d > 24) return 0u;
    if (d < 0) {
        big = true;
        return 0u;
    }
    if (d == 0) return X;
    const uint32_t half = 1u << (d - 1);
    const uint32_t r = X & ((half << 1) - 1u);
    tie = r == half;
    return (X >> d) + (r >= half ? 1u : 0u);
}

// xinc by float arithmetic: t = x * 2^(23-E) is exact for every x whose
// increment is not 0 (a power-of-two scale; t below 2^-126, where it could
// round, means an increment of 0), K = floor(t) and the fraction decide:
// K + 1 from one half up (tie: exactly one half), big: t >= 2^24.
__device__ __forceinline__ uint32_t xincf(float x, int E, bool& tie, bool& big) {
    const float t = ldexpf(x, 23 - E);
    const float fl = floorf(t);
    const float fr = t - fl;
    big = !(t < 16777216.0f);
    tie = fr == 0.5f;
    return big ? 0u : (uint32_t)fl + (fr >= 0.5f ? 1u : 0u);
}

// s + x, rounded to nearest even, exactly (integer arithmetic only).
__device__ XState xs_add(XState s, float x) {
    int ex;
    uint32_t X;
    fparts(x, ex, X);
    if (X == 0u) return s;
    if (s.M == 0u) return XState{ex, X};
    const int d = s.E - ex;
    uint64_t N;
    int base;
    if (d >= 0) {
        if (d > 25) return s;                        // x below a quarter of s's ulp
        N = ((uint64_t)s.M << d) + X;
        base = ex;
    } else {
        if (-d > 25) return XState{ex, X};           // s below a quarter of x's ulp
        N = ((uint64_t)X << (-d)) + s.M;
        base = s.E;
    }
    const int len = 64 - __clzll((long long)N);
    if (len <= 24) {
        // exact: normalise down to binade -126 at most
        const int Eb = max(-126, base - (24 - len));
        return XState{Eb, (uint32_t)(N << (base - Eb))};
    }
    const int sh = len - 24;
    uint64_t mant = N >> sh;
    const uint64_t rem = N & ((1ull << sh) - 1ull), half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (mant & 1ull))) ++mant;
    int E2 = base + sh;
    if (mant == (1ull << 24)) {
        mant >>= 1;
        ++E2;
    }
    return XState{E2, (uint32_t)mant};
}

// The smallest M at binade E with M * 2^(E-23) >= t (t > 0 float); 2^24 when
// no M of the binade reaches t.
__device__ __forceinline__ uint32_t xs_thr(float t, int E) {
    int et;
    uint32_t T;
    fparts(t, et, T);
    const int d = E - et;
    if (d < 0) return 1u << 24;
    if (d == 0) return T;
    if (d > 24) return 1u;
    return (T + (1u << d) - 1u) >> d;
}

// The binade of an approximate sum (E = -126 for 0 and subnormals).
__device__ __forceinline__ int xs_binade(float a) {
    const uint32_t f = (__float_as_uint(a) >> 23) & 255u;
    return (int)max(f, 1u) - 127;
}

// ---- block-wide helpers of k_full (kFT threads) ----

struct FullShared {
    float rf[kFW];
    uint32_t ru[kFW];
    int ri[kFW];
    double rd[kFW];
    uint64_t expT[32];
    double u;
    int flags;
    int tok;
    int sel_d, sel_need;
    XState xs;         // exact sum result
    int found;         // top-p: the threshold was reached
    int fpos;          // ... at this position of the group order (group start + offset)
    uint32_t fkey;     // ... by a value with this key
    int fgroup;        // ... in this group
    int fgt, feq;      // ... after fgt (group start + offset) larger keys, with feq of that key
    int redo;
    double dS;
    float m;
    int wtok[kFW];     // the draw, one window per wave: the id its running sum reaches u at (-1: none)
    double wds[kFW];   // ... that id's distance from u (before or after it)
    double wcp[kFW];   // ... the running sum at the window's end
};

__device__ __forceinline__ float fblock_max(float v, FullShared& st) {
    v = wave_max_f(v);
    if (lane_id() == 0) st.rf[wave_id()] = v;
    __syncthreads();
    float r = st.rf[0];
#pragma unroll
    for (int i = 1; i < kFW; ++i) r = fmaxf(r, st.rf[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t fblock_max_u(uint32_t v, FullShared& st) {
    v = wave_max_u32(v);
    if (lane_id() == 0) st.ru[wave_id()] = v;
    __syncthreads();
    uint32_t r = st.ru[0];
#pragma unroll
    for (int i = 1; i < kFW; ++i) r = max(r, st.ru[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t fblock_min_u(uint32_t v, FullShared& st) {
    v = wave_min_u32(v);
    if (lane_id() == 0) st.ru[wave_id()] = v;
    __syncthreads();
    uint32_t r = st.ru[0];
#pragma unroll
    for (int i = 1; i < kFW; ++i) r = min(r, st.ru[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int fblock_sum_i(int v, FullShared& st) {
    v = wave_incl_sum_i(v);
    if (lane_id() == 63) st.ri[wave_id()] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < kFW; ++i) r += st.ri[i];
    __syncthreads();
    return r;
}

// Exclusive scan over the block in thread order; *total gets the sum.
__device__ __forceinline__ int fblock_excl_scan(int v, int* total, FullShared& st) {
    const int incl = wave_incl_sum_i(v);
    if (lane_id() == 63) st.ri[wave_id()] = incl;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kFW; ++i) {
        const int s = st.ri[i];
        base += (i < wave_id()) ? s : 0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return base + incl - v;
}

__device__ __forceinline__ double wave_sum_d(double x) {
    x = wave_tree_prefix_d(x);
    return readlane_d(x, 63);
}

// LDS-qualified views of pointers into the block's shared memory: functions
// that receive them as plain pointers would otherwise access them with flat
// instructions.
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) float lds_f32;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_u4;
__device__ __forceinline__ uint32_t lds_add(lds_u32* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_or(lds_u32* p, uint32_t v) {
    __hip_atomic_fetch_or(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// 16 bytes of a row in global memory (16-byte aligned) by a global load: a
// plain pointer that reaches a function as an argument is read with flat
// loads, which the LDS waits then wait on too.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f32x4 gbl_f32x4;
__device__ __forceinline__ float4 gload4(const float* p) {
    const f32x4 v = *(const gbl_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

// ---- passes over a row (latency hidden: loads issued ahead of the work) ----

// f(i, x[i]) for every i in [0, n) (n a multiple of 4, x 16-byte aligned),
// over the block: each thread loads four 16-byte groups of four (sixteen
// values in flight) before using any of them. (Loading the next sixteen while
// f runs measured slower in k_full's top-p passes.)
template <class F>
__device__ __forceinline__ void fpass(const float* __restrict__ x, int n, F&& f) {
    const int n4 = n >> 2;
    for (int b = (int)threadIdx.x; b < n4; b += 4 * kFT) {
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = gload4(x + 4 * min(b + q * kFT, n4 - 1));   // (clamped: no branch around a load)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = b + q * kFT;
            if (i < n4) {
                f(4 * i, v[q].x);
                f(4 * i + 1, v[q].y);
                f(4 * i + 2, v[q].z);
                f(4 * i + 3, v[q].w);
            }
        }
    }
}

// f(w, g, v) for each 512-step g of each window w of this wave (windows wid,
// wid + kFW, ...; steps in order), v the lane's 8 values x[w * 512G + g * 512
// + lane * 8 + j]; the next step's values are loaded before f runs.
template <class F>
__device__ __forceinline__ void wpass(const float* __restrict__ x, int nW, int G, F&& f) {
    const int lane = lane_id();
    const int WS = kFWin * G;
    int w = wave_id(), g = 0;
    if (w >= nW) return;
    const float* p0 = x + (size_t)w * WS + lane * 8;
    float4 c0 = gload4(p0), c1 = gload4(p0 + 4);
    for (;;) {
        int nw = w, ng = g + 1;
        if (ng == G) {
            ng = 0;
            nw = w + kFW;
        }
        // (past the last window: the last again, unused; no branch around a load)
        const float* pn = x + (size_t)min(nw, nW - 1) * WS + ng * kFWin + lane * 8;
        const float4 n0 = gload4(pn), n1 = gload4(pn + 4);
        const float v[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        f(w, g, v);
        if (nw >= nW) break;
        w = nw;
        g = ng;
        c0 = n0;
        c1 = n1;
    }
}

// wpass over two arrays at once (same windows): f(w, g, v, y).
template <class F>
__device__ __forceinline__ void wpass2(const float* __restrict__ x, const float* __restrict__ z, int nW, int G,
                                       F&& f) {
    const int lane = lane_id();
    const int WS = kFWin * G;
    int w = wave_id(), g = 0;
    if (w >= nW) return;
    const size_t o0 = (size_t)w * WS + lane * 8;
    float4 c0 = gload4(x + o0), c1 = gload4(x + o0 + 4);
    float4 d0 = gload4(z + o0), d1 = gload4(z + o0 + 4);
    for (;;) {
        int nw = w, ng = g + 1;
        if (ng == G) {
            ng = 0;
            nw = w + kFW;
        }
        // (past the last window: the last again, unused; no branch around a load)
        const size_t on = (size_t)min(nw, nW - 1) * WS + ng * kFWin + lane * 8;
        const float4 n0 = gload4(x + on), n1 = gload4(x + on + 4);
        const float4 m0 = gload4(z + on), m1 = gload4(z + on + 4);
        const float v[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float y[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
        f(w, g, v, y);
        if (nw >= nW) break;
        w = nw;
        g = ng;
        c0 = n0;
        c1 = n1;
        d0 = m0;
        d1 = m1;
    }
}

// ---- the exact sequential sum engine (one wave) ----

// min(a + b, 2^25): the running prefixes only matter up to 2^24.
__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, 1u << 25); }

// What adding some values in order does to M at a fixed binade: d0 when M
// starts even, d1 when odd. A half-way value with lower multiple K rounds to
// the even neighbour, (K + (K & 1), K + 1 - (K & 1)); any other value adds
// its increment whatever the parity; one that leaves the binade saturates.
// Composing is associative, so sequences are scanned like sums.
struct XPair {
    uint32_t d0, d1;
};
__device__ __forceinline__ XPair xinc2(float x, int E) {
    bool t, b;
    const uint32_t i = xinc(x, E, t, b);
    if (b) return XPair{1u << 25, 1u << 25};
    if (!t) return XPair{i, i};
    const uint32_t K = i - 1u;
    return XPair{K + (K & 1u), K + 1u - (K & 1u)};
}
// xinc2 by float arithmetic: t = x * 2^(23-E) is exact (a power-of-two
// scale; t falls below 2^-126, where it could round, only for values that add
// nothing), its integer part K and fraction r give the increment -- K, or
// K + 1 above one half; exactly one half (tie) the pair (K + (K & 1),
// K + 1 - (K & 1)) -- and t >= 2^24 leaves the binade (saturated). The same
// pairs as xinc2 (x >= 0 finite).
__device__ __forceinline__ XPair xinc2f(float x, int E, bool& tie) {
    const float t = ldexpf(x, 23 - E);
    const float fl = floorf(t);
    const float fr = t - fl;
    const uint32_t K = t < 16777216.0f ? (uint32_t)fl : (1u << 25);
    tie = fr == 0.5f;
    const uint32_t i = K + (fr > 0.5f ? 1u : 0u);
    const uint32_t lo = K + (K & 1u), hi = K + 1u - (K & 1u);
    return (tie && K < (1u << 25)) ? XPair{lo, hi} : XPair{min(i, 1u << 25), min(i, 1u << 25)};
}

// xinc2f's increment when x is not half-way (both halves of its pair), and
// whether x is: the common case, without the pair's parity arithmetic.
__device__ __forceinline__ uint32_t xinc1f(float x, int E, bool& tie) {
    const float t = ldexpf(x, 23 - E);
    const float r = rintf(t);   // (t - r is exact; away from one half, round half up is this)
    tie = fabsf(t - r) == 0.5f;
    return t < 16777216.0f ? (uint32_t)r : (1u << 25);
}

// a, then b
__device__ __forceinline__ XPair xcomp(XPair a, XPair b) {
    return XPair{sat_add(a.d0, (a.d0 & 1u) ? b.d1 : b.d0), sat_add(a.d1, (a.d1 & 1u) ? b.d0 : b.d1)};
}
__device__ __forceinline__ uint32_t xat(XPair a, uint32_t M) { return (M & 1u) ? a.d1 : a.d0; }

// Inclusive scan of pairs over the wave in lane order (DPP, as wave_scan_u32).
template <int CTRL, int ROWM>
__device__ __forceinline__ XPair xcomp_dpp(XPair x) {
    const XPair l{dpp_u32<CTRL, ROWM>(0u, x.d0), dpp_u32<CTRL, ROWM>(0u, x.d1)};
    return xcomp(l, x);
}
__device__ __forceinline__ XPair wave_scan_pair(XPair x) {
    x = xcomp_dpp<0x111, 0xF>(x);
    x = xcomp_dpp<0x112, 0xF>(x);
    x = xcomp_dpp<0x114, 0xF>(x);
    x = xcomp_dpp<0x118, 0xF>(x);
    x = xcomp_dpp<0x142, 0xA>(x);
    x = xcomp_dpp<0x143, 0xC>(x);
    return x;
}
// Inclusive scan of pairs, by plain sums when no lane's pair differs by parity.
__device__ __forceinline__ XPair wave_scan_pair_any(XPair x) {
    if (__ballot(x.d0 != x.d1) != 0ull) return wave_scan_pair(x);
    const uint32_t u = wave_scan_u32(x.d0, 0u, [](uint32_t a, uint32_t b) { return a + b; });
    return XPair{u, u};
}

// Replays v[lane * 8 + j] (in that order; absent values +0) onto s, from
// position `start` on. With thr_on, stops at the first value after which the
// sum reaches thr and returns its position (0..511); else returns -1.
// Without thr the values are added one by one as float adds, the running sum
// handed from lane to lane (eight adds, then a readlane, per lane): the chain
// the sum is defined by, 512 steps whatever binades it crosses. With thr each
// step takes every remaining value at s's binade at once (lanes' increments
// scanned, then each lane's values in order from its exact start) and applies
// them up to the first value that leaves the binade or reaches thr, which is
// added exactly; a step without half-way values scans plain saturating sums,
// one with them the parity pairs.
__device__ int xs_replay(XState& s, const float (&v)[8], int start, bool thr_on, float thr) {
    const int lane = lane_id();
    if (!thr_on) {
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = lane * 8 + j >= start ? v[j] : 0.0f;
        float acc = xs_value(s);
        for (int l = start >> 3; l < 64; ++l) {
            float b = acc;
#pragma unroll
            for (int j = 0; j < 8; ++j) b = b + w[j];
            acc = readlane_f(b, l);
        }
        int ex;
        uint32_t X;
        fparts(acc, ex, X);
        s = XState{ex, X};
        return -1;
    }
    for (;;) {
        const int E = s.E;
        const uint32_t M = s.M;
        const uint32_t thrM = thr_on ? xs_thr(thr, E) : 0xFFFFFFFFu;
        uint32_t inc[8];
        bool tie = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            bool t, b;
            const uint32_t i = xinc(v[j], E, t, b);
            const bool on = lane * 8 + j >= start;
            inc[j] = on ? (b ? (1u << 25) : i) : 0u;
            tie |= on && t;
        }
        int first = 8;
        uint32_t at = 0u, cur;
        if (__ballot(tie) == 0ull) {
            // no half-way value: every increment adds whatever M's parity
            uint32_t ls = 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) ls = sat_add(ls, inc[j]);
            const uint32_t incl = wave_scan_u32(ls, 0u, [](uint32_t a, uint32_t b) { return sat_add(a, b); });
            const uint32_t prev = (uint32_t)__shfl_up((int)incl, 1, 64);
            cur = sat_add(M, lane == 0 ? 0u : prev);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t after = sat_add(cur, inc[j]);
                if (first == 8 && lane * 8 + j >= start && (after >= (1u << 24) || after >= thrM)) {
                    first = j;
                    at = cur;
                }
                cur = after;
            }
        } else {
            XPair e[8];
            XPair lp{0u, 0u};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                e[j] = (lane * 8 + j >= start) ? xinc2(v[j], E) : XPair{0u, 0u};
                lp = xcomp(lp, e[j]);
            }
            const XPair incl = wave_scan_pair(lp);
            const XPair prev{(uint32_t)__shfl_up((int)incl.d0, 1, 64), (uint32_t)__shfl_up((int)incl.d1, 1, 64)};
            cur = sat_add(M, lane == 0 ? 0u : xat(prev, M));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t after = sat_add(cur, xat(e[j], cur));
                if (first == 8 && lane * 8 + j >= start && (after >= (1u << 24) || after >= thrM)) {
                    first = j;
                    at = cur;
                }
                cur = after;
            }
        }
        const u64 em = __ballot(first < 8);
        if (em == 0ull) {
            s.M = (uint32_t)__builtin_amdgcn_readlane((int)cur, 63);
            return -1;
        }
        const int L = __ffsll((long long)em) - 1;
        const int jf = __builtin_amdgcn_readlane(first, L);
        float xv = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) xv = (j == jf) ? v[j] : xv;
        xv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv), L));
        s.M = (uint32_t)__builtin_amdgcn_readlane((int)at, L);
        s = xs_add(s, xv);
        const int pos = L * 8 + jf;
        if (thr_on && xs_value(s) >= thr) return pos;
        start = pos + 1;
        if (start >= 512) return -1;
    }
}

// Group table entry: (E + 256) | flags << 16 with the group's pair at E in
// D0/D1 (saturated at 2^25). Flags: 1 = the group must be replayed value by
// value (its order is not known, and a half-way value makes it matter; or
// too many values for the sums), 2 = empty group, 4 = an index-order window
// with lane tables (each lane's pair at E and at E + 1; it is predicted to
// leave its binade once), 8 = a top-p bucket whose increments are summed
// value by value, 16 = a top-p bucket whose copied keys are sorted in place,
// 32 = a top-p bucket whose keys the increments pass copies (the compose
// reads none of 4, 8, 16 and 32).
constexpr uint32_t kGCare = 1u, kGEmpty = 2u, kGLanes = 4u, kGInc = 8u, kGSorted = 16u, kGGath = 32u;
__device__ __forceinline__ uint32_t gpack(int E, uint32_t flags) { return (uint32_t)(E + 256) | (flags << 16); }

// Composes groups 0 .. n-1 in order onto s by one wave: whole groups at once
// while their tables say they stay in s's binade (and below thr); any other
// group goes to slow(g, s), which replays it exactly and returns true when
// the composition has to stop there (threshold reached, or the caller takes
// over). Starts at group c. Returns the group it stopped at, or -1.
template <class P, class Slow>
__device__ int xs_compose(int n, P EF, P D0, P D1, bool thr_on, float thr,
                          XState& s, Slow&& slow, int c = 0) {
    const int lane = lane_id();
    while (c < n) {
        const int g = c + lane;
        const bool valid = g < n;
        const uint32_t ef = valid ? EF[g] : 0u;
        const int Eg = (int)(ef & 0xFFFFu) - 256;
        const uint32_t fl = (ef >> 16) & ~(kGLanes | kGInc | kGSorted | kGGath);
        const bool empty = valid && (fl & kGEmpty) != 0u;
        const bool ok = empty || (valid && fl == 0u && Eg == s.E);
        const XPair d = (ok && !empty) ? XPair{D0[g], D1[g]} : XPair{0u, 0u};
        const XPair pre = wave_scan_pair(d);
        const uint32_t thrM = thr_on ? xs_thr(thr, s.E) : 0xFFFFFFFFu;
        const uint32_t tot = sat_add(s.M, xat(pre, s.M));
        const bool bad = !ok || tot >= (1u << 24) || tot >= thrM;
        const u64 bm = __ballot(bad);
        const int f = bm ? __ffsll((long long)bm) - 1 : 64;
        if (f > 0) s.M = (uint32_t)__builtin_amdgcn_readlane((int)tot, f - 1);
        if (f == 64) {
            c += 64;
            continue;
        }
        const int gs = c + f;
        if (gs >= n) break;
        if (slow(gs, s)) return gs;
        c = gs + 1;
    }
    return -1;
}

// ---- k_full phases ----

// LDS of a k_full block after the penalty table (when it lives there):
// window tables, bucket tables, one wave's sort buffer.
struct FullLds {
    float* winA;        // [kFMaxWin] approximate window sums (the draw: winA..winD0 as doubles)
    uint32_t* winD0;    // [kFMaxWin]
    uint32_t* winD1;    // [kFMaxWin]
    uint32_t* winEF;    // [kFMaxWin]
    uint32_t* gath;     // [kFGather] top-p: keys of the buckets replayed value by value (the window tables' space)
    uint32_t* bcnt;     // [kFNB + 1] bucket counts, then starts
    uint32_t* bfill;    // [kFNB] top-p: the binades where a bucket's values fall half-way (bits; see
                        // full_top_p); the index-order compose stages windows over bcnt .. gfill
    uint32_t* bD;       // [kFNB]
    uint32_t* bEF;      // [kFNB]
    uint32_t* gst;      // [kFNB] start of the bucket's keys in gath, or kNoGath
    uint32_t* gfill;    // [kFNB] their fill positions
    uint32_t* sortb;    // [kFSort] one bucket's keys, sorted
};
constexpr int kFGather = 4 * kFMaxWin;
constexpr uint32_t kNoGath = 0xFFFFFFFFu;
constexpr size_t kFullLdsBytes = 4 * (((4 * kFMaxWin + kFNB + 1 + 5 * kFNB + 3) & ~3) + kFSort) + 64;

__device__ __forceinline__ FullLds full_lds(unsigned char* base) {
    FullLds f;
    uint32_t* p = reinterpret_cast<uint32_t*>(base);
    f.winA = reinterpret_cast<float*>(p);
    f.winD0 = p + kFMaxWin;
    f.winD1 = p + 2 * kFMaxWin;
    f.winEF = p + 3 * kFMaxWin;
    f.gath = p;
    f.bcnt = p + 4 * kFMaxWin;
    f.bfill = f.bcnt + kFNB + 1;
    f.bD = f.bfill + kFNB;
    f.bEF = f.bfill + 2 * kFNB;
    f.gst = f.bfill + 3 * kFNB;
    f.gfill = f.bfill + 4 * kFNB;
    f.sortb = p + ((4 * kFMaxWin + kFNB + 1 + 5 * kFNB + 3) & ~3);   // (16-byte aligned)
    return f;
}

// Exclusive float scan over the block in thread order (approximate sums).
__device__ __forceinline__ float fblock_excl_scan_f(float v, float* total, FullShared& st) {
    const float incl = wave_tree_prefix_f(v);
    if (lane_id() == 63) st.rf[wave_id()] = incl;
    __syncthreads();
    float base = 0.0f, tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kFW; ++i) {
        const float s = st.rf[i];
        base += (i < wave_id()) ? s : 0.0f;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return base + incl - v;
}

// A kept-set predicate over numerators e (id i): e stays when the bits of
// e * inv (its p) are above key, or equal to it with i below ilim; else it
// reads as +0 (key 0 keeps every e >= 0).
struct Keep {
    float inv;
    uint32_t key;
    int32_t ilim;
    __device__ __forceinline__ float operator()(float e, int i) const {
        const uint32_t k = __float_as_uint(e * inv);
        return (k > key || (k == key && i < ilim)) ? e : 0.0f;
    }
};
constexpr Keep kKeepAll{1.0f, 0u, 0x7FFFFFFF};

// The exact index-order float sum of keep(x[i]) over [0, nW * 512 * G) (values
// >= 0, the padding +0), given each window's approximate sum in f.winA:
// predicted binades from the approximate prefixes, the windows' pairs at them,
// then one wave composes (replaying the windows where the prediction fails or
// the sum leaves its binade). With lanes (windows of one step), a window whose
// approximate end lies in a higher binade (or within 0.1% below one) also
// leaves each lane's pairs at E and E + 1 there, as k_fs_exp does, for the
// compose to resolve it by.
__device__ __forceinline__ XState exact_index_compose(const float* x, int nW, int G, FullLds f, FullShared& st,
                                                      const uint4* lanes = nullptr, Keep keep = kKeepAll);

__device__ __noinline__ XState exact_index_sum(const float* x, int nW, int G, FullLds f, FullShared& st,
                                               Keep keep = kKeepAll, uint4* lanes = nullptr) {
    const int tid = threadIdx.x, lane = lane_id();
    if (G != 1) lanes = nullptr;
    {
        // two windows per thread: their approximate start values -> binades
        const int w0 = 2 * tid;
        const float a0 = w0 < nW ? f.winA[w0] : 0.0f, a1 = w0 + 1 < nW ? f.winA[w0 + 1] : 0.0f;
        float tot;
        const float pre = fblock_excl_scan_f(a0 + a1, &tot, st);
        const int E0 = w0 == 0 ? -126 : xs_binade(pre), E1 = xs_binade(pre + a0);
        const bool l0 = lanes != nullptr && w0 > 0 && xs_binade((pre + a0) * 1.001f) != E0;
        const bool l1 = lanes != nullptr && xs_binade((pre + a0 + a1) * 1.001f) != E1;
        if (w0 < nW) f.winEF[w0] = gpack(E0, l0 ? kGLanes : 0u);
        if (w0 + 1 < nW) f.winEF[w0 + 1] = gpack(E1, l1 ? kGLanes : 0u);
    }
    __syncthreads();
    {
        XPair wp{0u, 0u};
        bool nz = false;
        wpass(x, nW, G, [&](int w, int g, const float (&u)[8]) {
            const uint32_t ef = f.winEF[w];
            const int E = (int)(ef & 0xFFFFu) - 256;
            const int i0 = w * kFWin * G + g * kFWin + lane * 8;
            // increments by float arithmetic; plain (saturating) sums while no
            // value is half-way, the parity pairs in order otherwise
            float v[8];
            bool tie = false;
            uint32_t ls = 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                bool t;
                v[j] = keep(u[j], i0 + j);
                ls += xinc1f(v[j], E, t);
                tie |= t;
                nz |= v[j] != 0.0f;
            }
            ls = min(ls, 1u << 25);
            XPair lp{ls, ls};
            if (__ballot(tie) != 0ull) {
                lp = XPair{0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    bool t;
                    lp = xcomp(lp, xinc2f(v[j], E, t));
                }
            }
            const bool lon = ((ef >> 16) & kGLanes) != 0u;
            if (lon) {
                XPair l1{0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    bool t;
                    l1 = xcomp(l1, xinc2f(v[j], E + 1, t));
                }
                lanes[(size_t)w * 64 + lane] = make_uint4(lp.d0, lp.d1, l1.d0, l1.d1);
            }
            const XPair sp = wave_scan_pair_any(lp);
            wp = xcomp(wp, XPair{(uint32_t)__builtin_amdgcn_readlane((int)sp.d0, 63),
                                 (uint32_t)__builtin_amdgcn_readlane((int)sp.d1, 63)});
            if (g == G - 1) {
                const bool empty = __ballot(nz) == 0ull;
                if (lane == 0) {
                    f.winD0[w] = wp.d0;
                    f.winD1[w] = wp.d1;
                    f.winEF[w] = gpack(E, (empty ? kGEmpty : 0u) | (lon ? kGLanes : 0u));
                }
                wp = XPair{0u, 0u};
                nz = false;
            }
        });
    }
    __syncthreads();
    return exact_index_compose(x, nW, G, f, st, lanes, keep);
}

// Segmented inclusive scan of pairs over the wave in lane order: a lane with
// head set starts a segment (its prefix begins with its own pair). The pair
// operator extended by a head flag, (ha, a) then (hb, b) = (ha | hb, hb ? b :
// a then b), is associative, so the DPP steps of wave_scan_pair apply.
template <int CTRL, int ROWM>
__device__ __forceinline__ void seg_scan_step(XPair& x, uint32_t& h) {
    const XPair o{dpp_u32<CTRL, ROWM>(0u, x.d0), dpp_u32<CTRL, ROWM>(0u, x.d1)};
    const uint32_t oh = dpp_u32<CTRL, ROWM>(0u, h);
    const XPair c = xcomp(o, x);
    x = h ? x : c;
    h |= oh;
}
__device__ __forceinline__ XPair wave_seg_scan_pair(XPair x, bool head) {
    uint32_t h = head ? 1u : 0u;
    seg_scan_step<0x111, 0xF>(x, h);
    seg_scan_step<0x112, 0xF>(x, h);
    seg_scan_step<0x114, 0xF>(x, h);
    seg_scan_step<0x118, 0xF>(x, h);
    seg_scan_step<0x142, 0xA>(x, h);
    seg_scan_step<0x143, 0xC>(x, h);
    return x;
}


// The same scans for pairs without half-way values (d0 == d1 in every lane):
// plain sums, at most 64 x 2^25 < 2^32.
template <int CTRL, int ROWM>
__device__ __forceinline__ void seg_sum_step(uint32_t& x, uint32_t& h) {
    const uint32_t o = dpp_u32<CTRL, ROWM>(0u, x);
    const uint32_t oh = dpp_u32<CTRL, ROWM>(0u, h);
    x = h ? x : o + x;
    h |= oh;
}
__device__ __forceinline__ uint32_t wave_seg_sum_u32(uint32_t x, bool head) {
    uint32_t h = head ? 1u : 0u;
    seg_sum_step<0x111, 0xF>(x, h);
    seg_sum_step<0x112, 0xF>(x, h);
    seg_sum_step<0x114, 0xF>(x, h);
    seg_sum_step<0x118, 0xF>(x, h);
    seg_sum_step<0x142, 0xA>(x, h);
    seg_sum_step<0x143, 0xC>(x, h);
    return x;
}

// Windows the index-order compose stages in LDS (window 0 and the windows
// with lane tables, in index order): 64 lane entries and 512 values each.
constexpr int kStage = 24;
static_assert(kStage * (64 * 16 + 512 * 4) + kStage * 4 <= 4 * (6 * kFNB + 1), "staging fits the bucket tables");

// The exact sum from the windows' tables in LDS (f.winEF / winD0 / winD1:
// each window's predicted binade and its integer increments there), composed
// in index order by wave 0. The windows of each batch of 64 are split into
// runs of one predicted binade; a segmented scan gives every window its
// run's prefix, so a run is taken at once while the state is in its binade
// and below 2^24. The window where the sum leaves the binade is resolved
// exactly: with lane tables (lanes: each lane's pair at E and E + 1, windows
// of one 512-step) the pairs at E find the lane whose values cross, that
// lane's eight values are added as floats and the lanes after it compose at
// E + 1 by their pairs; otherwise, or where the sum lands elsewhere or
// crosses again, the window's values are chained as float adds. The next run
// then starts at its own binade; a run whose binade the state is not in is
// replayed from its first window. With lane tables the other waves stage the
// windows to be resolved (window 0, the lane-table windows) in LDS while
// wave 0 composes, each marked ready once written.
__device__ __forceinline__ XState exact_index_compose(const float* x, int nW, int G, FullLds f, FullShared& st,
                                                      const uint4* lanes, Keep keep) {
    const int lane = lane_id(), wid = wave_id();
    const int WS = kFWin * G;
    const bool staged = lanes != nullptr && G == 1;
    const lds_u32* EF = (const lds_u32*)f.winEF;
    const lds_u32* D0 = (const lds_u32*)f.winD0;
    const lds_u32* D1 = (const lds_u32*)f.winD1;
    lds_u4* s_lt = (lds_u4*)f.bcnt;
    lds_f32* s_val = (lds_f32*)(f.bcnt + kStage * 64 * 4);
    volatile lds_u32* s_rdy = (volatile lds_u32*)(f.bcnt + kStage * 64 * 4 + kStage * 512);
    if (staged) {
        if ((int)threadIdx.x < kStage) s_rdy[threadIdx.x] = 0u;
        __syncthreads();
    }
    auto is_staged = [&](int g) -> bool { return g == 0 || ((EF[g] >> 16) & kGLanes) != 0u; };
    if (wid != 0) {
        if (staged) {
            int q = 0;
            for (int c = 0; c < nW && q < kStage; c += 64) {
                const int g = c + lane;
                u64 m = __ballot(g < nW && is_staged(g));
                while (m != 0ull && q < kStage) {
                    const int w = c + __ffsll((long long)m) - 1;
                    m &= m - 1ull;
                    if (q % (kFW - 1) == wid - 1) {
                        if (w > 0) {
                            const uint4 t = lanes[(size_t)w * 64 + lane];
                            s_lt[q * 64 + lane] = u32x4{t.x, t.y, t.z, t.w};
                        }
                        const float* src = x + (size_t)w * WS + lane * 8;
                        const float4 q0 = gload4(src), q1 = gload4(src + 4);
                        lds_f32* dst = s_val + q * 512 + lane * 8;
                        const int i0 = w * WS + lane * 8;
                        dst[0] = keep(q0.x, i0); dst[1] = keep(q0.y, i0 + 1);
                        dst[2] = keep(q0.z, i0 + 2); dst[3] = keep(q0.w, i0 + 3);
                        dst[4] = keep(q1.x, i0 + 4); dst[5] = keep(q1.y, i0 + 5);
                        dst[6] = keep(q1.z, i0 + 6); dst[7] = keep(q1.w, i0 + 7);
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                        if (lane == 0) s_rdy[q] = (uint32_t)w + 1u;
                    }
                    ++q;
                }
            }
        }
    } else {
        XState s{-126, 0u};
        // the exact resolution of window w (rank q among the staged windows)
        auto resolve = [&](int w, int q) {
            const uint32_t ef = EF[w];
            uint4 t = make_uint4(0u, 0u, 0u, 0u);
            float v[8];
            bool have = false;
            if (staged && q < kStage && is_staged(w)) {
                uint32_t spin = 0u;
                while (s_rdy[q] != (uint32_t)w + 1u && ++spin < (1u << 20)) __builtin_amdgcn_s_sleep(1);
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                if (s_rdy[q] == (uint32_t)w + 1u) {
                    if (w > 0) {
                        const u32x4 l4 = s_lt[q * 64 + lane];
                        t = make_uint4(l4.x, l4.y, l4.z, l4.w);
                    }
                    const lds_f32* sv = s_val + q * 512 + lane * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = sv[j];
                    have = true;
                }
            }
            const bool by_lanes = lanes != nullptr && G == 1 && ((ef >> 16) & kGLanes) &&
                                  s.E == (int)(ef & 0xFFFFu) - 256;
            if (!have && G == 1) {
                if (by_lanes) t = lanes[(size_t)w * 64 + lane];
                const float* src = x + (size_t)w * WS + lane * 8;
                const float4 q0 = gload4(src), q1 = gload4(src + 4);
                const int i0 = w * WS + lane * 8;
                v[0] = keep(q0.x, i0); v[1] = keep(q0.y, i0 + 1); v[2] = keep(q0.z, i0 + 2); v[3] = keep(q0.w, i0 + 3);
                v[4] = keep(q1.x, i0 + 4); v[5] = keep(q1.y, i0 + 5); v[6] = keep(q1.z, i0 + 6); v[7] = keep(q1.w, i0 + 7);
            }
            if (G != 1) {
                for (int g = 0; g < G; ++g) {
                    const float* src = x + (size_t)w * WS + g * kFWin + lane * 8;
                    const float4 q0 = gload4(src), q1 = gload4(src + 4);
                    const int i0 = w * WS + g * kFWin + lane * 8;
                    const float u[8] = {keep(q0.x, i0), keep(q0.y, i0 + 1), keep(q0.z, i0 + 2), keep(q0.w, i0 + 3),
                                        keep(q1.x, i0 + 4), keep(q1.y, i0 + 5), keep(q1.z, i0 + 6),
                                        keep(q1.w, i0 + 7)};
                    xs_replay(s, u, 0, false, 0.0f);
                }
                return;
            }
            if (!by_lanes) {
                xs_replay(s, v, 0, false, 0.0f);
                return;
            }
            const int E = s.E;
            const uint32_t M = s.M;
            const XPair incl = wave_scan_pair_any(XPair{t.x, t.y});
            const uint32_t end = sat_add(M, xat(incl, M));   // M after this lane's values
            const u64 cm = __ballot(end >= (1u << 24));
            if (cm == 0ull) {
                s.M = (uint32_t)__builtin_amdgcn_readlane((int)end, 63);
                return;
            }
            const int L = __ffsll((long long)cm) - 1;
            const uint32_t ML = L == 0 ? M : (uint32_t)__builtin_amdgcn_readlane((int)end, L - 1);
            float acc = xs_value(XState{E, ML});
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + readlane_f(v[j], L);
            int ex;
            uint32_t X;
            fparts(acc, ex, X);
            s = XState{ex, X};
            if (L == 63) return;
            if (ex == E + 1) {
                const XPair rest = wave_scan_pair_any(lane > L ? XPair{t.z, t.w} : XPair{0u, 0u});
                const XPair tot{(uint32_t)__builtin_amdgcn_readlane((int)rest.d0, 63),
                                (uint32_t)__builtin_amdgcn_readlane((int)rest.d1, 63)};
                const uint32_t Me = sat_add(X, xat(tot, X));
                if (Me < (1u << 24)) {
                    s.M = Me;
                    return;
                }
            }
            xs_replay(s, v, (L + 1) * 8, false, 0.0f);
        };
        int c = 0, qc = 0;   // batch start, rank of the first staged window at or after it
        while (c < nW) {
            const int g = c + lane;
            const bool valid = g < nW;
            const uint32_t ef = valid ? EF[g] : 0u;
            const int Eg = (int)(ef & 0xFFFFu) - 256;
            const bool empty = valid && ((ef >> 16) & kGEmpty) != 0u;
            const XPair d = (valid && !empty) ? XPair{D0[g], D1[g]} : XPair{0u, 0u};
            const int Ep = __shfl_up(Eg, 1, 64);
            const bool head = lane == 0 || Eg != Ep;
            XPair sp;
            if (__ballot(d.d0 != d.d1) != 0ull) {
                sp = wave_seg_scan_pair(d, head);
            } else {
                const uint32_t u = wave_seg_sum_u32(d.d0, head);
                sp = XPair{u, u};
            }
            const u64 heads = __ballot(head && valid);
            const u64 smask = staged ? __ballot(valid && is_staged(g)) : 0ull;
            const u64 nonempty = __ballot(valid && !empty);
            const int nval = min(64, nW - c);
            auto rank = [&](int lo) { return qc + __popcll(smask & ((1ull << lo) - 1ull)); };
            int h = 0, next = c + 64;
            while (h < nval) {
                const u64 above = h < 63 ? heads & ~((2ull << h) - 1ull) : 0ull;
                const int e = above ? __ffsll((long long)above) - 2 : nval - 1;
                const u64 segm = (e < 63 ? (2ull << e) - 1ull : ~0ull) & ~((1ull << h) - 1ull);
                const int Eh = __builtin_amdgcn_readlane(Eg, h);
                if ((nonempty & segm) == 0ull) {
                    h = e + 1;
                    continue;
                }
                if (Eh != s.E) {
                    // the run was predicted at another binade: its first window exactly, then a new batch
                    resolve(c + h, rank(h));
                    next = c + h + 1;
                    break;
                }
                const uint32_t tot = sat_add(s.M, xat(sp, s.M));
                const u64 bm = __ballot(tot >= (1u << 24)) & segm;
                if (bm == 0ull) {
                    s.M = (uint32_t)__builtin_amdgcn_readlane((int)tot, e);
                    h = e + 1;
                    continue;
                }
                const int fb = __ffsll((long long)bm) - 1;
                if (fb > h) s.M = (uint32_t)__builtin_amdgcn_readlane((int)tot, fb - 1);
                resolve(c + fb, rank(fb));
                if (fb < e) {
                    // the sum left the binade before the run's end: the rest of the run from a new batch
                    next = c + fb + 1;
                    break;
                }
                h = e + 1;
            }
            qc += __popcll(smask & (next - c >= 64 ? ~0ull : (1ull << (next - c)) - 1ull));
            c = next;
        }
        if (lane == 0) st.xs = s;
    }
    __syncthreads();
    return st.xs;
}

// Bitonic sort, descending, of 64 Q keys held Q per lane (position t * 64 +
// lane in v[t]): a stage of distance J joins position e with e ^ J, across
// lanes for J < 64 (xor_lane_u32), inside a lane for J >= 64. In a run of
// size K that descends (e & K == 0) the lower position keeps the larger key.
template <int Q, int K, int J>
__device__ __forceinline__ void bsort_stage(uint32_t (&v)[Q]) {
    const int lane = lane_id();
    if constexpr (J >= 64) {
        constexpr int JJ = J / 64;
#pragma unroll
        for (int t = 0; t < Q; ++t) {
            if ((t & JJ) == 0) {
                const bool desc = ((t * 64) & K) == 0;
                const uint32_t a = v[t], b = v[t | JJ];
                v[t] = desc ? max(a, b) : min(a, b);
                v[t | JJ] = desc ? min(a, b) : max(a, b);
            }
        }
    } else {
        const bool lower = (lane & J) == 0;
#pragma unroll
        for (int t = 0; t < Q; ++t) {
            const bool desc = ((t * 64 + lane) & K) == 0;
            const uint32_t o = xor_lane_u32<J>(v[t]);
            v[t] = (lower == desc) ? max(v[t], o) : min(v[t], o);
        }
    }
}
template <int Q, int K, int J>
__device__ __forceinline__ void bsort_steps(uint32_t (&v)[Q]) {
    bsort_stage<Q, K, J>(v);
    if constexpr (J > 1) bsort_steps<Q, K, J / 2>(v);
}
template <int Q, int K = 2>
__device__ __forceinline__ void bsort_all(uint32_t (&v)[Q]) {
    bsort_steps<Q, K, K / 2>(v);
    if constexpr (K < 64 * Q) bsort_all<Q, 2 * K>(v);
}
// src[0, n) sorted descending into dst[0, n) by one wave (n <= 64 Q), in
// registers (padding 0, below every key).
template <int Q>
__device__ __forceinline__ void wave_bitonic_to(const lds_u32* src, int n, lds_u32* dst) {
    const int lane = lane_id();
    uint32_t v[Q];
#pragma unroll
    for (int t = 0; t < Q; ++t) v[t] = t * 64 + lane < n ? src[t * 64 + lane] : 0u;
    bsort_all<Q>(v);
#pragma unroll
    for (int t = 0; t < Q; ++t)
        if (t * 64 + lane < n) dst[t * 64 + lane] = v[t];
    wave_sync();
}
__device__ __forceinline__ void wave_sort_desc_to(const lds_u32* src, int n, lds_u32* dst) {
    if (n <= 64) wave_bitonic_to<1>(src, n, dst);
    else if (n <= 128) wave_bitonic_to<2>(src, n, dst);
    else if (n <= 256) wave_bitonic_to<4>(src, n, dst);
    else wave_bitonic_to<8>(src, n, dst);
}

// Replays keys[0, n) (floats as bits, in that order) onto s as float adds --
// the sum they define, whatever binades it crosses: the running sum handed
// from lane to lane (eight adds, then a readlane, per lane holding values).
// Stops at the first value after which the sum reaches thr: returns its
// position (s is the sum there), else -1 (s is the sum of all n).
__device__ int chain_replay(XState& s, const uint32_t* keys, int n, float thr) {
    const int lane = lane_id();
    const lds_u32* kl = (const lds_u32*)keys;
    for (int o = 0; o < n; o += 512) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int e = o + lane * 8 + j;
            v[j] = e < n ? __uint_as_float(kl[e]) : 0.0f;   // (+0 leaves a sum >= 0 as it is)
        }
        const int nl = min(64, (n - o + 7) >> 3);
        float acc = xs_value(s), start = 0.0f;
        for (int l = 0; l < nl; ++l) {
            float b = acc;
#pragma unroll
            for (int j = 0; j < 8; ++j) b = b + v[j];
            start = lane == l ? acc : start;
            acc = readlane_f(b, l);
        }
        // the first value whose sum reaches thr (the sums only grow: none
        // when the last does not): each lane's adds again from its start
        if (acc >= thr) {
            float c = start, cat = 0.0f;
            int first = 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                c = c + v[j];
                if (first == 8 && lane < nl && c >= thr) {
                    first = j;
                    cat = c;
                }
            }
            const u64 hm = __ballot(first < 8);
            if (hm != 0ull) {
                const int L = __ffsll((long long)hm) - 1;
                int ex;
                uint32_t X;
                fparts(readlane_f(cat, L), ex, X);
                s = XState{ex, X};
                return o + L * 8 + __builtin_amdgcn_readlane(first, L);
            }
        }
        int ex;
        uint32_t X;
        fparts(acc, ex, X);
        s = XState{ex, X};
    }
    return -1;
}

// A top-p bucket of n values (keys k0 .. k0 + 2^shift - 1: one exponent, eb;
// notes: bit t - 9 set when a value's mantissa has t >= 9 trailing zero
// bits) added onto sv at its binade E, where d = E - eb >= shift + 1 and
// >= 10 and no value has d - 1 or more trailing zero bits (none half-way at
// E or E + 1): every value adds the same increment at E, and the add that
// takes the sum out of E rounds alike for every value (by the parity of M
// plus the increment and the side of one half the value's fraction lies on,
// never on it), as do the increments at E + 1 after it. The order within the
// bucket then does not matter: the sum after it is arithmetic, across at
// most one crossing. False (sv unchanged) when this does not hold, the sum
// would leave E + 1 or it reaches thr.
__device__ __forceinline__ bool xs_uniform_bucket(XState& sv, uint32_t k0, uint32_t n, uint32_t notes, int shift,
                                                  float thr) {
    const int E = sv.E, d = E - ((int)max(k0 >> 23, 1u) - 127);
    if (sv.M == 0u || d < max(shift + 1, 10)) return false;
    if (d - 10 < 32 && (notes >> (d - 10)) != 0u) return false;
    const uint32_t X0 = (k0 & 0x7FFFFFu) | ((k0 >> 23) != 0u ? 0x800000u : 0u);
    const uint64_t inc = d >= 26 ? 0u : ((X0 >> (d - 1)) + 1u) >> 1;
    const uint64_t thrM = xs_thr(thr, E);
    const uint64_t end = (uint64_t)sv.M + (uint64_t)n * inc;
    if (end < (1u << 24)) {
        if (end >= thrM) return false;
        sv.M = (uint32_t)end;
        return true;
    }
    // the jc-th value's add leaves E (k0 | 1, which shares the values' bits
    // from shift up and has a nonzero fraction at E, gives that add's result)
    const uint64_t jc = ((1u << 24) - (uint64_t)sv.M + inc - 1u) / inc;
    const uint64_t Mb = (uint64_t)sv.M + (jc - 1u) * inc;
    if (Mb >= thrM) return false;
    const XState s1 = xs_add(XState{E, (uint32_t)Mb}, __uint_as_float(k0 | 1u));
    if (s1.E != E + 1) return false;
    const uint64_t inc1 = d + 1 >= 26 ? 0u : ((X0 >> d) + 1u) >> 1;
    const uint64_t end1 = (uint64_t)s1.M + (uint64_t)(n - jc) * inc1;
    if (end1 >= (1u << 24) || end1 >= xs_thr(thr, E + 1)) return false;
    sv = XState{E + 1, (uint32_t)end1};
    return true;
}

// The row's top-p cutoff (sampler.cpp:146-164) over the probabilities
// p = e * inv (e = pv, inv = fl(1 / softmax sum)): the cumulative float sum in
// (p desc, index asc) order, exactly. Keys (float bits of p > 0) in [lo, hi]
// go to kFNB buckets of equal key width in descending order. One pass counts
// them; a scan gives each bucket's place and, from counts times the bucket's
// middle value, its predicted binade; a second pass adds every value's
// increment at its bucket's binade (noting half-way values, whose order
// then matters) and copies into LDS the keys of the buckets that are likely
// to be replayed value by value -- those early in the order (half-way
// values are common while the sum is within 2^10 of them) or where the
// approximate sum changes binade or reaches top_p. One wave composes the
// buckets; a bucket of one increment that leaves its binade (or was
// predicted at another) is added by arithmetic (xs_uniform_bucket), one that
// must be replayed is sorted in registers (or taken as it is when all its
// keys are equal) -- the copied ones found to hold half-way values sorted
// beforehand by all the block's waves. Buckets flagged by the pass but not
// copied are copied by one more pass, any other bucket on demand; one too
// large to sort is refined (its key range becomes the next [lo, hi]), and a
// range that runs out continues below it. A bucket replayed value by value
// is sorted, then added as floats in that order. Returns whether the running sum reached top_p; then
// *cut_key is the key of the last kept value, *cut_count the number kept,
// *cut_gt the number with a larger key, *cut_eq the number with that key and
// st.dS the sum there. range_lo / range_hi: the smallest and largest keys
// above 0 when the caller knows them (range_hi 0: one more pass finds them).
__device__ bool full_top_p(const float* pv, int V, int Vp, float inv, float top_p, FullLds f, FullShared& st,
                           uint32_t range_lo, uint32_t range_hi, uint32_t* cut_key, int* cut_count, int* cut_gt,
                           int* cut_eq) {
    // the bucket tables as LDS pointers (through FullLds, plain pointers, the
    // compiler would reach them with flat instructions)
    lds_u32* const bcnt = (lds_u32*)f.bcnt;
    lds_u32* const bfill = (lds_u32*)f.bfill;
    lds_u32* const bD = (lds_u32*)f.bD;
    lds_u32* const bEF = (lds_u32*)f.bEF;
    lds_u32* const gst = (lds_u32*)f.gst;
    lds_u32* const gfill = (lds_u32*)f.gfill;
    lds_u32* const gath = (lds_u32*)f.gath;
    lds_u32* const sortb = (lds_u32*)f.sortb;
    const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
    uint32_t kmx = range_hi, kmn = range_lo;
    if (range_hi == 0u) {
        kmx = 0u;
        kmn = 0xFFFFFFFFu;
        fpass(pv, Vp, [&](int, float e) {
            const uint32_t key = __float_as_uint(e * inv);
            if (key != 0u) {
                kmx = max(kmx, key);
                kmn = min(kmn, key);
            }
        });
        kmx = fblock_max_u(kmx, st);
        kmn = fblock_min_u(kmn, st);
    }
    HSAMP_PHASE(13000 + blockIdx.x, 0);
    if (kmx == 0u) return false;
    XState s{-126, 0u};
    int counted = 0;
    uint32_t lo = kmn, hi = kmx;
    for (int level = 0; level < 1024; ++level) {
        // Buckets aligned to multiples of 2^shift in key space: bucket b holds
        // the keys k with k >> shift = (hi >> shift) - b, so its values share
        // their exponent (shift < 23) and their mantissa bits from shift up.
        const uint32_t span = hi - lo;
        int shift = span >= (uint32_t)kFNB ? (32 - __clz((int)span)) - 12 : 0;
        if ((int)((hi >> shift) - (lo >> shift)) + 1 > kFNB) ++shift;
        const int nb = (int)((hi >> shift) - (lo >> shift)) + 1;
        const uint32_t htop = hi >> shift;
        auto bucket_of = [&](uint32_t key) -> int { return (int)(htop - (key >> shift)); };
        auto in_range = [&](uint32_t key) -> bool { return key != 0u && key >= lo && key <= hi; };
        // bucket b's lowest key (below lo for the last bucket) and its values' biased exponent
        auto bkey = [&](int b) -> uint32_t { return (htop - (uint32_t)b) << shift; };
        auto bexp = [&](int b) -> int { return (int)(bkey(b) >> 23); };
        for (int b = tid; b < nb; b += kFT) {
            bcnt[b] = 0u;
            bD[b] = 0u;
            bfill[b] = 0u;
        }
        __syncthreads();
        // The counts; and where a value falls half-way: X * 2^(ex-23) is
        // half-way between two multiples of binade E's ulp exactly when
        // E = ex + tz + 1 (tz: X's trailing zeros). Far from the value's own
        // binade (tz >= 9) that is rare: such binades are noted per bucket
        // (bit tz - 9; the bucket's values share ex) for the scan below.
        fpass(pv, Vp, [&](int, float e) {
            const uint32_t key = __float_as_uint(e * inv);
            if (in_range(key)) {
                const int b = bucket_of(key);
                lds_add(bcnt + b, 1u);
                if ((key & 0x1FFu) == 0u) {   // (X's low nine bits are the key's)
                    const uint32_t bx = key >> 23;
                    const uint32_t X = (key & 0x7FFFFFu) | (bx != 0u ? 0x800000u : 0u);
                    const int tz = __builtin_ctz(X | 0x1000000u);
                    if (tz <= 23) lds_or(bfill + b, 1u << (tz - 9));
                }
            }
        });
        __syncthreads();
        if (level == 0) HSAMP_PHASE(13000 + blockIdx.x, 1);
        {
            // starts, predicted binades and the buckets to copy: 4 per thread, in order
            uint32_t c[4];
            float a4[4], mv[4];
            uint32_t cs = 0u;
            float as = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = 4 * tid + q;
                c[q] = b < nb ? bcnt[b] : 0u;
                // count times the bucket's middle value
                const int64_t mid = (int64_t)bkey(b) + (((int64_t)1 << shift) >> 1);
                mv[q] = __uint_as_float((uint32_t)min(max(mid, (int64_t)lo), (int64_t)hi));
                a4[q] = (float)c[q] * mv[q];
                cs += c[q];
                as += a4[q];
            }
            int ctot;
            uint32_t cpos = (uint32_t)fblock_excl_scan((int)cs, &ctot, st);
            float atot;
            float apos = xs_value(s) + fblock_excl_scan_f(as, &atot, st);
            bool gq[4];
            int gcnt = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = 4 * tid + q;
                gq[q] = false;
                if (b < nb) {
                    bcnt[b] = cpos;
                    const int E = xs_binade(apos);
                    // a value noted half-way at E (or the binade after, where a
                    // crossing may take the sum)
                    const int eb = max(bexp(b), 1) - 127;
                    const uint32_t tm = bfill[b];
                    const int t0 = E - eb - 10;
                    const bool tie_e = t0 >= 0 && t0 < 32 && ((tm >> t0) & 1u);
                    const bool tie_at = tie_e || (t0 + 1 >= 0 && t0 + 1 < 32 && ((tm >> (t0 + 1)) & 1u));
                    // At d = E - eb >= shift + 1 (and >= 10, where any half-way
                    // value is noted) every value's increment, (X >> d) rounded
                    // half up, depends on mantissa bits the bucket's values
                    // share: the bucket's sum is its count times that of its
                    // lowest key, exactly, unless a value is half-way at E.
                    // Otherwise (or more than 255 values: a sum of increments
                    // could wrap) the increments pass sums them value by value.
                    const int d = E - eb;
                    const bool uni = c[q] != 0u && d >= max(shift + 1, 10) && !tie_e;
                    uint32_t fl = c[q] == 0u ? kGEmpty : 0u;
                    if (uni) {
                        const uint32_t k0 = bkey(b);
                        const uint32_t X0 = (k0 & 0x7FFFFFu) | ((k0 >> 23) != 0u ? 0x800000u : 0u);
                        const uint32_t inc = d >= 26 ? 0u : ((X0 >> (d - 1)) + 1u) >> 1;
                        bD[b] = (uint32_t)min((uint64_t)c[q] * inc, (uint64_t)1 << 25);
                    } else if (c[q] != 0u) {
                        fl |= kGInc | (c[q] > 255u ? kGCare : 0u);
                    }
                    bEF[b] = gpack(E, fl);
                    if (c[q] != 0u && c[q] <= (uint32_t)kFSort) {
                        // (the approximate sums are within about 1e-4 of the true ones)
                        const float lo_e = apos * 0.998f, hi_e = (apos + a4[q]) * 1.002f;
                        const bool tie_prone = E - xs_binade(mv[q]) <= 10;
                        const bool cross = xs_binade(lo_e) != xs_binade(hi_e);
                        const bool at_thr = lo_e <= top_p && top_p <= hi_e;
                        gq[q] = tie_prone || cross || at_thr || tie_at;
                    }
                    gcnt += gq[q] ? (int)c[q] : 0;
                }
                cpos += c[q];
                apos += a4[q];
            }
            // places in the copy area, in bucket order, while it has room
            int gtot;
            int gpos = fblock_excl_scan(gcnt, &gtot, st);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = 4 * tid + q;
                if (b < nb) {
                    const bool g = gq[q] && gpos + (int)c[q] <= kFGather;
                    gst[b] = g ? (uint32_t)gpos : kNoGath;
                    if (g) bEF[b] = bEF[b] | (kGGath << 16);   // (this thread's entry)
                    gfill[b] = (uint32_t)gpos;
                    gpos += gq[q] ? (int)c[q] : 0;
                }
            }
            if (tid == 0) {
                bcnt[nb] = (uint32_t)ctot;
                st.sel_d = min(gtot, kFGather);   // the copy area in use (a bound)
            }
        }
        __syncthreads();
        if (level == 0) HSAMP_PHASE(13000 + blockIdx.x, 2);
        fpass(pv, Vp, [&](int, float e) {
            const float p = e * inv;
            const uint32_t key = __float_as_uint(p);
            if (in_range(key)) {
                const int b = bucket_of(key);
                const uint32_t ef = bEF[b];
                if ((ef >> 16) & kGInc) {
                    bool t, bg;
                    const uint32_t inc = xincf(p, (int)(ef & 0xFFFFu) - 256, t, bg);
                    if (inc) lds_add(bD + b, inc);
                    if ((t || bg) && !((ef >> 16) & kGCare)) lds_or(bEF + b, kGCare << 16);
                }
                if ((ef >> 16) & kGGath) gath[lds_add(gfill + b, 1u)] = key;
            }
        });
        __syncthreads();
        if (level == 0) HSAMP_PHASE(13000 + blockIdx.x, 3);
        // buckets flagged by the pass (half-way values) but not copied
        {
            int gcnt = 0;
            bool gq[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = 4 * tid + q;
                const uint32_t n = b < nb ? bcnt[b + 1] - bcnt[b] : 0u;
                gq[q] = b < nb && gst[b] == kNoGath && n != 0u && n <= (uint32_t)kFSort &&
                        ((bEF[b] >> 16) & kGCare) != 0u;
                gcnt += gq[q] ? (int)n : 0;
            }
            int gtot;
            int gpos = st.sel_d + fblock_excl_scan(gcnt, &gtot, st);
            const bool fits = st.sel_d + gtot <= kFGather;
            if (gtot > 0 && fits) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int b = 4 * tid + q;
                    if (gq[q]) {
                        gst[b] = kNoGath - 1u;   // being copied: marked, then given its place
                        gfill[b] = (uint32_t)gpos;
                        gpos += (int)(bcnt[b + 1] - bcnt[b]);
                    }
                }
                __syncthreads();
                fpass(pv, Vp, [&](int, float e) {
                    const uint32_t key = __float_as_uint(e * inv);
                    if (in_range(key)) {
                        const int b = bucket_of(key);
                        if (gst[b] == kNoGath - 1u) gath[lds_add(gfill + b, 1u)] = key;
                    }
                });
                __syncthreads();
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int b = 4 * tid + q;
                    if (gq[q]) gst[b] = gfill[b] - (bcnt[b + 1] - bcnt[b]);
                }
                if (tid == 0) st.sel_d += gtot;
            }
            __syncthreads();
        }
        // The copied buckets with half-way values (replayed value by value
        // when the compose gets there) sorted in place now, one per wave in
        // parallel, rather than each by the composing wave in turn.
        if (shift != 0) {
            int scnt = 0;
            bool sq[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = 4 * tid + q;
                const uint32_t n = b < nb ? bcnt[b + 1] - bcnt[b] : 0u;
                sq[q] = n > 1u && gst[b] != kNoGath && ((bEF[b] >> 16) & kGCare) != 0u;
                scnt += sq[q] ? 1 : 0;
            }
            int stot;
            int spos = fblock_excl_scan(scnt, &stot, st);
            if (stot > 0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (sq[q] && spos < kFSort) sortb[spos] = (uint32_t)(4 * tid + q);
                    spos += sq[q] ? 1 : 0;
                }
                __syncthreads();
                const int ns = min(stot, kFSort);
                for (int k = wid; k < ns; k += kFW) {
                    const int b = (int)sortb[k];
                    lds_u32* keys = gath + gst[b];
                    wave_sort_desc_to(keys, (int)(bcnt[b + 1] - bcnt[b]), keys);
                    if (lane == 0) bEF[b] |= kGSorted << 16;
                }
                __syncthreads();
            }
        }
        // compose (wave 0) from bucket c0; st.found: 1 = reached, 2 = refine
        // bucket st.fgroup, 3 = copy bucket st.fgroup first
        int c0 = 0;
        for (;;) {
            if (wid == 0) {
                if (lane == 0) st.found = 0;
                const int g = xs_compose(nb, bEF, bD, bD, true, top_p, s, [&](int b, XState& sv) -> bool {
                    const uint32_t b0 = bcnt[b], n = bcnt[b + 1] - b0;
                    if (n == 0u) return false;
                    const uint32_t gs = gst[b];
                    if (shift == 0) {
                        // a bucket of one key: n equal values, in any order
                        const float val = __uint_as_float(hi - (uint32_t)b);
                        for (uint32_t o = 0; o < n; o += 512) {
                            float v[8];
#pragma unroll
                            for (int j = 0; j < 8; ++j) v[j] = o + lane * 8 + j < n ? val : 0.0f;
                            const int pos = xs_replay(sv, v, 0, true, top_p);
                            if (pos >= 0) {
                                if (lane == 0) {
                                    st.found = 1;
                                    st.fpos = (int)(b0 + o) + pos;
                                    st.fkey = hi - (uint32_t)b;
                                    st.fgt = (int)b0;
                                    st.feq = (int)n;
                                    st.xs = sv;
                                }
                                return true;
                            }
                        }
                        return false;
                    }
                    if (!((bEF[b] >> 16) & (kGInc | kGCare)) &&
                        xs_uniform_bucket(sv, bkey(b), n, bfill[b], shift, top_p))
                        return false;
                    if (gs == kNoGath) {
                        if (n > (uint32_t)kFSort) {
                            if (lane == 0) {
                                st.found = 2;
                                st.fgroup = b;
                                st.xs = sv;
                                st.fpos = (int)b0;
                            }
                        } else if (lane == 0) {
                            st.found = 3;
                            st.fgroup = b;
                            st.xs = sv;
                        }
                        return true;
                    }
                    // the bucket's keys sorted (n <= kFSort), then added as floats in that order
                    const lds_u32* keys = gath + gs;
                    if (!((bEF[b] >> 16) & kGSorted)) {
                        wave_sort_desc_to(gath + gs, (int)n, sortb);
                        keys = sortb;
                    }
                    const int pos = chain_replay(sv, (const uint32_t*)keys, (int)n, top_p);
                    if (pos < 0) return false;
                    // the keys above the cut's and equal to it (all in this bucket)
                    const uint32_t ck = keys[pos];
                    int ngt = 0, neq = 0;
                    for (uint32_t e = lane; e < n; e += 64) {
                        const uint32_t y = keys[e];
                        ngt += y > ck;
                        neq += y == ck;
                    }
                    ngt = __builtin_amdgcn_readlane(wave_incl_sum_i(ngt), 63);
                    neq = __builtin_amdgcn_readlane(wave_incl_sum_i(neq), 63);
                    if (lane == 0) {
                        st.found = 1;
                        st.fpos = (int)b0 + pos;
                        st.fkey = ck;
                        st.fgt = (int)b0 + ngt;
                        st.feq = neq;
                        st.xs = sv;
                    }
                    return true;
                }, c0);
                if (g < 0 && lane == 0) st.xs = s;
            }
            __syncthreads();
            const int fd = st.found;
            s = st.xs;
            if (fd != 3) break;
            // copy bucket st.fgroup (into LDS when it fits, else refine it)
            const int b = st.fgroup;
            const uint32_t n = bcnt[b + 1] - bcnt[b];
            if (st.sel_d + (int)n <= kFGather) {
                if (tid == 0) {
                    gst[b] = kNoGath - 1u;
                    gfill[b] = (uint32_t)st.sel_d;
                }
                __syncthreads();
                fpass(pv, Vp, [&](int, float e) {
                    const uint32_t key = __float_as_uint(e * inv);
                    if (in_range(key) && bucket_of(key) == b) gath[lds_add(gfill + b, 1u)] = key;
                });
                __syncthreads();
                if (tid == 0) {
                    gst[b] = (uint32_t)st.sel_d;
                    st.sel_d += (int)n;
                }
                __syncthreads();
                c0 = b;
                continue;
            }
            if (tid == 0) {
                st.found = 2;
                st.fpos = (int)bcnt[b];
            }
            __syncthreads();
            break;
        }
        if (level == 0) HSAMP_PHASE(13000 + blockIdx.x, 4);
        if (threadIdx.x == 0 && level < 8) g_phase_lv(blockIdx.x, level);
        const int fd = st.found;
        if (fd == 1) {
            *cut_key = st.fkey;
            *cut_count = counted + st.fpos + 1;
            *cut_gt = counted + st.fgt;
            *cut_eq = st.feq;
            st.dS = (double)xs_value(s);
            return true;
        }
        if (fd == 2) {
            // refine: the bucket's key range, from the state before it
            const int b = st.fgroup;
            counted += st.fpos;
            const uint64_t k0 = (uint64_t)bkey(b);
            const uint64_t top = min(k0 + ((uint64_t)1 << shift) - 1u, (uint64_t)hi);
            const uint64_t bot = max(k0, (uint64_t)lo);
            hi = (uint32_t)top;
            lo = (uint32_t)bot;
            __syncthreads();
            continue;
        }
        // the range ran out: continue below it
        counted += (int)bcnt[nb];
        __syncthreads();
        if (lo <= kmn) return false;
        hi = lo - 1u;
        lo = kmn;
    }
    return false;
}

}  // namespace hsamp
