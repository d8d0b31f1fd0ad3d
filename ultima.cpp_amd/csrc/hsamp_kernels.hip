// HIP kernels of the gfx950 token sampler (reference src/sampler/sampler.cpp).
//
// Top-k rows (k <= the candidate limit) stream the [B, V] logits once:
// k_stream takes one workgroup per (row, slice), applies mask -> bias ->
// repetition -> DRY -> frequency/presence -> temperature to each logit in
// registers (sampler.cpp:235-264) and leaves the slice's candidates in
// global scratch:
//   - exact lists (sampling rows with k <= 1024 and greedy rows, penalties
//     that only lower logits -- repetition, frequency/presence, DRY sharing
//     their count window -- and up to 256 logit-bias ids, each evaluated on
//     its own): every id whose final key can still be in the row's top k,
//     filtered by a bound from the slice's own top keys;
//     k_pick (every k <= 64) or k_pick_l, one block per row on the XCD that
//     streamed it, merges the row's lists;
//   - general path (more bias entries, DRY shorter than the repetition
//     window, write-back, longer histories, ...): a candidate buffer in LDS under a
//     rising threshold (or the slice's argmax for a greedy row), merged by
//     k_merge.
// The merge gives the exact top-k (value desc, index asc) and runs the rest
// of the ladder over the <= k kept logits: softmax with glibc-exact expf and
// index-order float sums, top-p over the (p desc, index asc) order, min-p,
// the double-precision CDF and the draw against the row's u.
//
// k_full: one 1024-thread block per row that samples the whole vocabulary
//   (top-k off or above the candidate limit): the same ladder over all V
//   values, with the reference's sequential float sums reproduced exactly in
//   parallel (integer increments per binade, half-way ties as parity pairs).
//
// k_writeback: optional pass leaving the logits exactly as the reference's
//   sample() leaves them (kept logits post-temperature, the rest -inf;
//   post-penalty logits for greedy rows).
//
// No MFMA: nothing here is a contraction. The stream phase is HBM-bound.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "hsamp_plan.h"
#include "hsamp_wave.h"
#include "hsamp_xsum.h"
#include "libm_expf.h"

#pragma clang fp contract(off)

namespace hsamp {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// LDS-qualified views (see lds_u32): 64-bit keys and doubles, ids, flags
typedef __attribute__((address_space(3))) u64 lds_u64;
typedef __attribute__((address_space(3))) double lds_f64;
typedef __attribute__((address_space(3))) int32_t lds_i32;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr uint32_t kKeyNegInf = 0x007FFFFFu;        // key32(-inf)
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
// Key of a flagged candidate (a penalised id whose true value k_merge finds):
// the key of the NaN bit pattern 0x7FFFFFFF, which no stored key can take
// (NaNs are stored as kKeyNegInf or left out).
constexpr uint32_t kKeyFlag = 0xFFFFFFFFu;
constexpr u64 kThetaFloor = (u64)(kKeyNegInf + 1) << 32;  // smallest finite composite

// Order-preserving key of a float: larger float -> larger key; -0 == +0.
__device__ __forceinline__ uint32_t key32(float x) {
    uint32_t b = __float_as_uint(x);
    if ((b << 1) == 0u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// Composite: value desc, then index asc, as one unsigned order.
__device__ __forceinline__ u64 comp(uint32_t key, int32_t idx) {
    return ((u64)key << 32) | (u64)(~(uint32_t)idx);
}
__device__ __forceinline__ int32_t comp_idx(u64 c) { return (int32_t)(~(uint32_t)c); }

// Row r's plan. A row whose history length is read on the device (a history
// kept on the GPU, grown and compacted there: RF_DEVWIN) takes its windows
// from that length, as window_slice does (sampler.cpp:19-24): each stage's
// window is min(cap, length), DRY's only when it holds two ids or more
// (sampler.cpp:69), so that one plan serves every step from the first token
// on.
__device__ __forceinline__ RowPlan plan_of(const StreamArgs& a, int r) {
    RowPlan P = a.plans[r];
    if (P.flags & RF_DEVWIN) {
        const int L = min(max(a.hist_len_dev[r], 0), (int)a.hist_stride);
        const int rc = (int)(P.win_caps[0] & 0xFFFFu), dc = (int)(P.win_caps[0] >> 16);
        const int fc = (int)(P.win_caps[1] & 0xFFFFu);
        P.hist_len = L;
        P.rep_win = min(rc, L);
        P.dry_win = min(dc, L) >= 2 ? min(dc, L) : 0;
        P.fp_win = min(fc, L);
        P.scan_len = max(max(P.rep_win, P.dry_win), P.fp_win);
    }
    return P;
}

// Ids in row r's history (its plan from plan_of).
__device__ __forceinline__ int hist_len_of(const StreamArgs&, const RowPlan& P, int) { return P.hist_len; }

struct Shared {
    u64 theta;          // current survival threshold (composite)
    u64 minv;
    int n;              // entries in the candidate buffer
    int nst;            // exact lists: staged chunks
    int last;           // this block merges its row
    int sel_d, sel_need, sel_cnt;
    int scan[8];
    uint32_t twave[4];
    float fred[4];
    int ired[4];
    u64 ured[4];
    u64 minv_w[4];
    int fw[4];          // per-wave flags (k_pick)
    uint32_t hist[256];
    int soff[257];      // slice offsets during the merge
    int flags;
    int nan0;
    uint32_t thmax;     // largest survival bound of the row's sampling slices
    alignas(16) u64 wv[64];  // the finishing wave's cross-lane scratch
    double u;           // the row's uniform
    uint64_t expT[32];  // expf's table (libm_expf.h), copied to LDS
    float sm_m, sm_inv;
    int cutoff;
    double dS;
    double dred[4];
    double hat, hbefore;   // general finalize: the draw's hit (tree sums) and the sum before it
    int tok;
};

// Exclusive block scan of one int per thread; *total gets the block sum.
__device__ __forceinline__ int block_excl_scan(int v, int* total, Shared& st) {
    const int lane = lane_id(), w = wave_id();
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) st.scan[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kBlock / 64; ++i) {
        const int s = st.scan[i];
        base += (i < w) ? s : 0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

__device__ __forceinline__ float block_max_f(float v, Shared& st) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    if (lane_id() == 0) st.fred[wave_id()] = v;
    __syncthreads();
    float r = st.fred[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) r = fmaxf(r, st.fred[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ u64 block_max_u64(u64 v, Shared& st) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const u64 o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    if (lane_id() == 0) st.ured[wave_id()] = v;
    __syncthreads();
    u64 r = st.ured[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) r = st.ured[i] > r ? st.ured[i] : r;
    __syncthreads();
    return r;
}

// kw-th largest of the 64*G keys a wave holds (G per lane), by a bitwise
// radix select over ballots. Keys of 0 stand for "no value".
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t (&g)[4], int G, int kw) {
    uint32_t prefix = 0u, known = 0u;
    int need = kw;
    for (int b = 31; b >= 0; --b) {
        const uint32_t bit = 1u << b;
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < G) {
                const bool m = ((g[i] & known) == prefix) && (g[i] & bit);
                cnt += __popcll(__ballot(m));
            }
        }
        if (cnt >= need) prefix |= bit;
        else need -= cnt;
        known |= bit;
    }
    return prefix;
}

__device__ __forceinline__ u64 shfl_xor_u64(u64 v, int m) {
    return (u64)__shfl_xor((long long)v, m, 64);
}

// Keep the k largest of the buffer's n = st.n distinct composites (exactly
// k), and raise the threshold to the k-th. The entries are held in registers
// (n <= 16 * 256); the k-th is found by 8-bit radix passes that start below
// the bits all entries share, and stop as soon as the digit's bucket is
// exactly what is still needed.
__device__ __attribute__((noinline)) void buf_compact(u64* buf_, int k, Shared& st) {
    lds_u64* buf = (lds_u64*)buf_;   // (always a block's LDS buffer)
    const int n = st.n;
    if (n <= k) return;
    constexpr int MAXE = 16;
    const int tid = threadIdx.x, lane = lane_id();
    u64 v[MAXE];
    u64 lo = ~0ull, hi = 0ull;
#pragma unroll
    for (int m = 0; m < MAXE; ++m) {
        const int i = tid + m * kBlock;
        v[m] = (i < n) ? buf[i] : 0ull;
        if (i < n) {
            lo = v[m] < lo ? v[m] : lo;
            hi = v[m] > hi ? v[m] : hi;
        }
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const u64 a2 = shfl_xor_u64(lo, d), b2 = shfl_xor_u64(hi, d);
        lo = a2 < lo ? a2 : lo;
        hi = b2 > hi ? b2 : hi;
    }
    if (lane == 0) {
        st.ured[wave_id()] = lo;
        st.minv_w[wave_id()] = hi;
    }
    __syncthreads();
    lo = st.ured[0];
    hi = st.minv_w[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) {
        lo = st.ured[i] < lo ? st.ured[i] : lo;
        hi = st.minv_w[i] > hi ? st.minv_w[i] : hi;
    }
    const int hb = 63 - __clzll((long long)(lo ^ hi));   // highest differing bit (n >= 2)
    u64 pmask = (hb >= 63) ? 0ull : ~((2ull << hb) - 1ull);
    u64 prefix = hi & pmask;
    int need = k;
    u64 kth = 0ull;
    bool done = false;
    for (int shift = hb >= 7 ? hb - 7 : 0;; ) {
        st.hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MAXE; ++m)
            if (tid + m * kBlock < n && (v[m] & pmask) == prefix)
                atomicAdd(&st.hist[(uint32_t)(v[m] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 64) {
            const int c0 = st.hist[255 - 4 * lane], c1 = st.hist[254 - 4 * lane];
            const int c2 = st.hist[253 - 4 * lane], c3 = st.hist[252 - 4 * lane];
            const int s4 = c0 + c1 + c2 + c3;
            int incl = s4;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(incl, d, 64);
                if (lane >= d) incl += y;
            }
            const int excl = incl - s4;
            const bool mine = excl < need && need <= incl;
            const u64 bal = __ballot(mine);
            if (mine && (int)(__ffsll((long long)bal) - 1) == lane) {
                int q, cnt, before;
                if (excl + c0 >= need) { q = 0; cnt = c0; before = excl; }
                else if (excl + c0 + c1 >= need) { q = 1; cnt = c1; before = excl + c0; }
                else if (excl + c0 + c1 + c2 >= need) { q = 2; cnt = c2; before = excl + c0 + c1; }
                else { q = 3; cnt = c3; before = excl + c0 + c1 + c2; }
                st.sel_d = 255 - 4 * lane - q;
                st.sel_need = need - before;
                st.sel_cnt = cnt;
            }
        }
        __syncthreads();
        const int dgt = st.sel_d, cnt = st.sel_cnt;
        need = st.sel_need;
        prefix = (prefix & ~((u64)0xFF << shift)) | ((u64)dgt << shift);
        pmask |= (u64)0xFF << shift;
        if (cnt == need || shift == 0) {
            // every entry under this prefix is in: the k-th is their minimum
            u64 mn = ~0ull;
#pragma unroll
            for (int m = 0; m < MAXE; ++m)
                if (tid + m * kBlock < n && (v[m] & pmask) == prefix && v[m] < mn) mn = v[m];
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) {
                const u64 o = shfl_xor_u64(mn, d);
                mn = o < mn ? o : mn;
            }
            if (lane == 0) st.ured[wave_id()] = mn;
            __syncthreads();
            kth = st.ured[0];
#pragma unroll
            for (int i = 1; i < kBlock / 64; ++i) kth = st.ured[i] < kth ? st.ured[i] : kth;
            done = true;
        }
        __syncthreads();
        if (done) break;
        shift = shift >= 8 ? shift - 8 : 0;
    }
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < MAXE; ++m) cnt += (tid + m * kBlock < n && v[m] >= kth) ? 1 : 0;
    int total;
    int pos = block_excl_scan(cnt, &total, st);
#pragma unroll
    for (int m = 0; m < MAXE; ++m)
        if (tid + m * kBlock < n && v[m] >= kth) buf[pos++] = v[m];
    __syncthreads();
    if (tid == 0) {
        st.n = total;
        st.theta = kth;
    }
    __syncthreads();
}

// Offer register-held candidates to the LDS buffer. Slot i of every thread
// holds an order key kv[i] (0 = empty) of id idx(i); it survives when its
// composite is >= the threshold. Each lane counts its survivors, the wave
// reserves one contiguous range with a single LDS atomic, and each lane writes
// its survivors in slot order; entries past the buffer's capacity go to the
// block's global overflow area `ovf` (drained by drain_overflow).
template <int NE, typename Idx>
__device__ __forceinline__ void append_regs(u64* buf, int cap, const uint32_t (&kv)[NE], Idx idx,
                                            u64* ovf, Shared& st) {
    static_assert(NE <= 32, "survivor mask is 32 bits");
    const int lane = lane_id();
    const u64 th = st.theta;
    const uint32_t thk = (uint32_t)(th >> 32);
    const uint32_t thi = ~(uint32_t)th;   // largest index that survives a tie on thk
    uint32_t sv = 0u;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const uint32_t key = kv[i];
        const bool ok = key > thk || (key == thk && (uint32_t)idx(i) <= thi);
        sv |= ok ? (1u << i) : 0u;
    }
    const int cnt = __popc(sv);
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
    }
    const int wtot = __shfl(incl, 63, 64);
    if (wtot == 0) return;
    int base = 0;
    if (lane == 63) base = atomicAdd(&st.n, wtot);
    base = __shfl(base, 63, 64);
    int pos = base + incl - cnt;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        if ((sv >> i) & 1u) {
            const u64 c = comp(kv[i], idx(i));
            if (pos < cap) buf[pos] = c;
            else ovf[pos - cap] = c;
            ++pos;
        }
    }
}

// Append m candidates fetched by get(j), j < m, in rounds that always fit:
// before each round the buffer is compacted to at most k entries and the
// round adds at most cap - k.
template <typename Get>
__device__ void append_fetch(u64* buf, int cap, int k, int m, Get get, Shared& st) {
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int room = cap - k;
    for (int base = 0; base < m; base += room) {
        buf_compact(buf, k, st);
        const u64 th = st.theta;
        const int chunk = min(room, m - base);
        for (int q = 0; q < chunk; q += kBlock) {
            const int j = q + tid;
            u64 c = 0ull;
            if (j < chunk) c = get(base + j);
            const bool sv = j < chunk && c >= th;
            const u64 bal = __ballot(sv);
            if (bal == 0ull) continue;
            const int leader = __ffsll((long long)bal) - 1;
            int b0 = 0;
            if (lane == leader) b0 = atomicAdd(&st.n, __popcll(bal));
            b0 = __shfl(b0, leader, 64);
            if (sv) buf[b0 + __popcll(bal & ((1ull << lane) - 1ull))] = c;
        }
        __syncthreads();
    }
}

// After append_regs: if the buffer overflowed, keep its k best and re-offer
// the overflow entries.
__device__ void drain_overflow(u64* buf, int cap, int k, const u64* ovf, Shared& st) {
    __syncthreads();
    const int n = st.n;
    if (n <= cap) return;
    __syncthreads();
    if (threadIdx.x == 0) st.n = cap;
    __syncthreads();
    __threadfence_block();
    append_fetch(buf, cap, k, n - cap, [&](int j) { return ovf[j]; }, st);
}

// Bitonic sort of 1024 keys held four per thread in registers (thread t:
// entries 4t .. 4t+3). A stage of distance J joins entry i with i ^ J: J <= 2
// inside a thread, 4 <= J <= 128 between the lanes of a wave (lane distance
// J / 4), J = 256, 512 between waves through x[0 .. 1024) in LDS with block
// barriers. Of each pair the lower entry keeps the minimum when the bitonic
// run of size K containing it ascends (DESC flips every run).
template <bool DESC, int K, int J, class P>
__device__ __forceinline__ void rsort_stage(u64 (&v)[4], P x) {
    const int t = threadIdx.x;
    if constexpr (J <= 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if ((q & J) == 0) {
                const bool up = (((4 * t + q) & K) == 0) != DESC;
                const u64 a = v[q], b = v[q | J];
                const bool sw = (a > b) == up;
                v[q] = sw ? b : a;
                v[q | J] = sw ? a : b;
            }
        }
    } else {
        constexpr int M = J / 4;   // partner thread t ^ M
        u64 o[4];
        if constexpr (M < 64) {
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = xor_lane_u64<M>(v[q]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) x[4 * t + q] = v[q];
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = x[4 * (t ^ M) + q];
            __syncthreads();
        }
        const bool lower = (t & M) == 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool up = (((4 * t + q) & K) == 0) != DESC;
            const bool lt = o[q] < v[q];
            v[q] = (lt == (lower == up)) ? o[q] : v[q];
        }
    }
}
template <bool DESC, int K, int J, class P>
__device__ __forceinline__ void rsort_steps(u64 (&v)[4], P x) {
    rsort_stage<DESC, K, J>(v, x);
    if constexpr (J > 1) rsort_steps<DESC, K, J / 2>(v, x);
}
template <bool DESC, int K = 2, class P>
__device__ __forceinline__ void rsort1024(u64 (&v)[4], P x) {
    rsort_steps<DESC, K, K / 2>(v, x);
    if constexpr (K < 1024) rsort1024<DESC, 2 * K>(v, x);
}

__device__ __forceinline__ uint32_t align16u(uint32_t x) { return (x + 15u) & ~15u; }

__device__ __forceinline__ int next_pow2(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// ---- penalty bookkeeping -----------------------------------------------------

// The row's penalty table, open addressing over mhash_slots keys and values,
// in LDS or (for windows too large for LDS) in the row's global area. Reads go
// through agent-scope atomic loads, which are plain LDS reads for LDS and bypass
// the vector L1 for global memory, where the table was filled by atomics.
struct PenaltyLds {
    uint32_t* hkey;
    uint32_t* hval;
    uint32_t hmask;
    uint32_t hshift;
};

__device__ __forceinline__ uint32_t tab_ld(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// GT: the table lives in the row's global area (windows too large for LDS).
template <bool GT>
__device__ __forceinline__ PenaltyLds pen_table(const StreamArgs& a, int r, unsigned char* smem) {
    PenaltyLds pl;
    if (GT) pl.hkey = a.gtab + (int64_t)r * 2 * a.mhash_slots;
    else pl.hkey = reinterpret_cast<uint32_t*>(smem);
    pl.hval = pl.hkey + a.mhash_slots;
    pl.hmask = (uint32_t)a.mhash_slots - 1u;
    pl.hshift = 32u - (uint32_t)__popc(pl.hmask);
    return pl;
}

__device__ __forceinline__ uint32_t hslot(int32_t t, PenaltyLds pl) {
    return ((uint32_t)t * 0x9E3779B1u) >> pl.hshift;
}

__device__ uint32_t pen_insert(int32_t t, PenaltyLds pl) {
    uint32_t s = hslot(t, pl);
    for (;;) {
        const uint32_t old = atomicCAS(&pl.hkey[s], kEmpty, (uint32_t)t);
        if (old == kEmpty || old == (uint32_t)t) return s;
        s = (s + 1) & pl.hmask;
    }
}

// Stages 1-4 of the ladder for id t whose table value is v (sampler.cpp:28-99).
__device__ __forceinline__ float pen_value(float x, int32_t t, uint32_t v, const StreamArgs& a, const RowPlan& P) {
    if (v & HV_BIAS) {
        int lo = 0, hi = P.bias_cnt;
        const int32_t* ids = a.bias_ids + P.bias_off;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (ids[mid] < t) lo = mid + 1;
            else hi = mid;
        }
        x = x + a.bias_vals[P.bias_off + lo];
    }
    if (v & HV_REP) x = (x > 0.0f) ? (x / P.rep) : (x * P.rep);
    const int dc = (int)((v >> HV_DRY_SHIFT) & HV_DRY_MASK);
    if (dc > P.dry_allowed) x = x - a.dry_tab[P.dry_tab + dc];
    const int fc = (int)(v & HV_FP_MASK);
    if (fc > 0) {
        x = x - (float)fc * P.freq;
        x = x - P.pres;
    }
    return x;
}

// The same for an id with a table entry, found by probing.
__device__ __forceinline__ float pen_apply(float x, int32_t t, const StreamArgs& a, const RowPlan& P,
                                           PenaltyLds pl) {
    uint32_t s = hslot(t, pl);
    while (tab_ld(&pl.hkey[s]) != (uint32_t)t) s = (s + 1) & pl.hmask;
    return pen_value(x, t, tab_ld(&pl.hval[s]), a, P);
}

// ---- tile loading --------------------------------------------------------------

template <int DT>
struct Tile {
    static constexpr int VW = DT == 0 ? 4 : 8;    // elements per 16-byte chunk
    static constexpr int NCH = DT == 0 ? 8 : 4;   // chunks per thread per tile
    static constexpr int NE = VW * NCH;           // 32 elements per thread
    static constexpr int ES = DT == 0 ? 4 : 2;    // bytes per element
    static constexpr int ELEMS = kBlock * NE;     // 8192 per tile
};

// Buffer resource over one row's first `elems` elements: loads past them
// return 0 (the hardware's range check), so tile loads need no bounds.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const char* rowp, int elems, int es) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(rowp), (short)0, elems * es, 0x00020000);
}

// One tile of this thread's chunks from [tb, hi) through the row's buffer
// resource (range hi): every chunk is one 16-byte non-temporal load (VEC:
// aligned rows, slices ending on a whole chunk; the row's last V % VW ids are
// left to k_merge), or its elements one by one (unaligned rows). Chunks past
// hi read as zeros; tile_keys counts them absent.
template <int DT, bool VEC, int NC = Tile<DT>::NCH>
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t rs, int tb, uint4 (&raw)[NC]) {
    using T = Tile<DT>;
    const int e0 = tb + (int)threadIdx.x * T::VW;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if (VEC) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, e0 * T::ES, j * kBlock * 16, 2);
            raw[j] = make_uint4(v.x, v.y, v.z, v.w);
        } else {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            const int ej = e0 + j * kBlock * T::VW;
#pragma unroll
            for (int c = 0; c < T::VW; ++c) {
                if (DT == 0) w[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, (ej + c) * 4, 0, 0);
                else w[c >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (ej + c) * 2, 0, 0) << ((c & 1) * 16);
            }
            raw[j] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

template <int DT>
__device__ __forceinline__ float elem(const uint4& r, int c) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if (DT == 0) return __uint_as_float(w[c]);
    const uint32_t x = w[c >> 1];
    return __uint_as_float((c & 1) ? (x & 0xFFFF0000u) : (x << 16));
}

// ---- the token ---------------------------------------------------------------------

// Row r's token (lane 0's tok), written by the wave that decided it, with
// ultima_hsamp_run_commit's rules when the launch carries them (the server
// loop's per token, src/server/http_server.cpp:174-201): an ended row
// (active 0) gets -1; -1 or a stop id ends the row without being pushed;
// any other token is appended to the row's device history (a full row first
// keeps its last c_keep ids at its front, copied by the whole wave) and
// counted against the row's budget, which ends the row at 0. Called by all 64
// lanes of one wave.
__device__ __forceinline__ void emit_token_wave(const StreamArgs& a, int r, int32_t tok) {
    const int lane = lane_id();
    tok = __builtin_amdgcn_readlane(tok, 0);
    if (a.c_hist == nullptr) {
        if (lane == 0) a.token[r] = tok;
        return;
    }
    // an ended slot, or one whose budget is spent (max_tokens 0: the
    // reference's loop body never runs), emits nothing
    if (a.c_active[r] == 0 || (a.c_budget != nullptr && a.c_budget[r] <= 0)) {
        if (lane == 0) {
            a.token[r] = -1;
            a.c_active[r] = 0;
        }
        return;
    }
    bool end = tok < 0;
    for (int i = 0; i < a.c_nstop; ++i) end = end || tok == a.c_stop[i];
    if (end) {
        if (lane == 0) {
            a.token[r] = tok;
            a.c_active[r] = 0;
        }
        return;
    }
    int32_t* h = a.c_hist + (int64_t)r * a.c_stride;
    int L = max(a.c_len[r], 0);
    if (L >= a.c_stride) {
        // [stride - keep, stride) -> [0, keep) (keep <= stride / 2: the
        // ranges do not overlap), eight ids per lane in flight at a time
        const int keep = a.c_keep;
        const int64_t from = a.c_stride - keep;
        for (int i0 = 0; i0 < keep; i0 += 8 * 64) {
            int32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = h[from + min(i0 + j * 64 + lane, keep - 1)];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (i0 + j * 64 + lane < keep) h[i0 + j * 64 + lane] = v[j];
        }
        L = keep;
    }
    if (lane == 0) {
        a.token[r] = tok;
        h[L] = tok;
        a.c_len[r] = L + 1;
        if (a.c_budget != nullptr) {
            const int32_t b = a.c_budget[r] - 1;
            a.c_budget[r] = b;
            if (b <= 0) a.c_active[r] = 0;
        }
    }
}

// ---- finalize over the kept set ------------------------------------------------

struct FinLds {
    u64* sortk;     // [1024] sort keys, then the double q_i (the candidate buffer itself)
    int32_t* fidx;  // [kmax] kept ids, index order
    float* fv;      // values (post-temperature)
    float* fe;      // expf(v - m), replaced in place by the probabilities
    float* fp;      // probabilities (the same storage as fe)
    uint8_t* keep;  // still kept
};

// FinLds's arrays (and the candidate buffers, all in LDS) as LDS pointers:
// the noinline functions that receive them as plain pointers would otherwise
// reach them with flat instructions.
struct FinView {
    lds_u64* sortk;
    lds_i32* fidx;
    lds_f32* fv;
    lds_f32* fe;
    lds_f32* fp;
    lds_u8* keep;
};
__device__ __forceinline__ FinView fin_view(const FinLds& f) {
    return FinView{(lds_u64*)f.sortk, (lds_i32*)f.fidx, (lds_f32*)f.fv,
                   (lds_f32*)f.fe,    (lds_f32*)f.fp,   (lds_u8*)f.keep};
}

// Exclusive block scan of one double per thread (tree association: only for
// decisions taken with a margin); *total gets the block sum.
__device__ __forceinline__ double block_excl_scan_d(double v, double* total, Shared& st) {
    const double incl = wave_tree_prefix_d(v);
    if (lane_id() == 63) st.dred[wave_id()] = incl;
    __syncthreads();
    double base = 0.0, tot = 0.0;
#pragma unroll
    for (int i = 0; i < kBlock / 64; ++i) {
        const double x = st.dred[i];
        base += (i < wave_id()) ? x : 0.0;
        tot += x;
    }
    __syncthreads();
    *total = tot;
    return base + incl - v;
}

// The reference's sequential float sum of v(i) over i < n, the same additions
// in the same order, by one wave: lane l holds entries [16 l, 16 l + 16) of
// each 1024-entry round, loaded together; every lane adds its sixteen to the
// running sum and a readlane hands lane l's result on (sixteen additions and
// one readlane per lane, the additions of lane l the only ones kept). With
// thr_on, stops at the first entry after which the sum reaches thr and
// returns its position (else -1); *sum gets the sum there (or the whole sum).
template <class Val>
__device__ int wave_seq_sum_f(int n, Val v, bool thr_on, float thr, float* sum) {
    const int lane = lane_id();
    float s = 0.0f;
    for (int c = 0; c < n; c += 1024) {
        float x[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = c + lane * 16 + j;
            x[j] = i < n ? v(i) : 0.0f;
        }
        const int lanes = min(64, (n - c + 15) >> 4);
        for (int l = 0; l < lanes; ++l) {
            float b = s;
#pragma unroll
            for (int j = 0; j < 16; ++j) b = b + x[j];
            const float s1 = readlane_f(b, l);
            if (thr_on && s1 >= thr) {
                // the first entry of lane l's sixteen after which the sum reaches thr
                float s2 = s;
                int hit = 16;
                float at = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    s2 = s2 + x[j];
                    if (hit == 16 && s2 >= thr) {
                        hit = j;
                        at = s2;
                    }
                }
                *sum = readlane_f(at, l);
                return c + l * 16 + __builtin_amdgcn_readlane(hit, l);
            }
            s = s1;
        }
    }
    *sum = s;
    return -1;
}

// softmax_probs over the kept entries (sampler.cpp:124-142): m, e, float
// index-order sum (exact, on wave 0), p = e * fl(1/sum). Returns false when
// nothing is kept.
__device__ __attribute__((noinline)) bool fin_softmax(FinLds f_, int nk, Shared& st) {
    const FinView f = fin_view(f_);
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (int j = tid; j < nk; j += kBlock)
        if (f.keep[j]) m = fmaxf(m, f.fv[j]);
    m = block_max_f(m, st);
    if (m == -__builtin_inff()) return false;
    for (int j = tid; j < nk; j += kBlock) f.fe[j] = f.keep[j] ? libm_expf_t(f.fv[j] - m, st.expT) : 0.0f;
    __syncthreads();
    if (tid < 64) {
        // (entries not kept hold +0, which leaves a sum of values >= 0 unchanged)
        float s;
        wave_seq_sum_f(nk, [&](int i) { return f.fe[i]; }, false, 0.0f, &s);
        if (tid == 0) {
            st.sm_inv = (s <= 0.0f) ? __builtin_nanf("") : 1.0f / s;
            st.sm_m = s;
        }
    }
    __syncthreads();
    const float s = st.sm_m, inv = st.sm_inv;
    for (int j = tid; j < nk; j += kBlock)
        f.fp[j] = f.keep[j] ? ((s <= 0.0f) ? f.fe[j] : f.fe[j] * inv) : 0.0f;
    __syncthreads();
    return true;
}

// Uniform draw over all V ids when no finite logit is left (sampler.cpp:127-130
// feeding the CDF of 178-182). Sequential on one lane; a degenerate path.
__device__ __attribute__((noinline)) int32_t uniform_draw(int V, double u) {
    const float pu = 1.0f / (float)V;
    if (!(u > 0.0)) return 0;
    double S = 0.0;
    for (int i = 0; i < V; ++i) S = S + (double)pu;
    const double q = (double)pu / S;
    double cp = 0.0;
    for (int i = 0; i < V; ++i) {
        cp = cp + q;
        const double c = (i == V - 1) ? 1.0 : cp;
        if (c >= u) return i;
    }
    return V - 1;
}

// The ladder after top-k for one row whose top-k set is buf[0..nk).
__device__ __attribute__((noinline)) void finalize_row(const StreamArgs& a, const RowPlan& P, int r,
                                                       const u64* buf_, int nk, FinLds f_, Shared& st,
                                                       uint32_t rflags) {
    const FinView f = fin_view(f_);
    const lds_u64* buf = (const lds_u64*)buf_;
    const int tid = threadIdx.x;
    const int V = a.vocab;
    const double u = st.u;
    const bool single = (P.flags & RF_SINGLE) != 0;
    if (!single) rflags |= ROWF_U_USED;
    int32_t tok = 0;
    int nkept = nk;
    if (nk > 0) {
        // index order: (id, key) pairs sorted in registers (nk <= 1024; the
        // sort's LDS exchange reuses the first 1024 entries of the buffer)
        {
            u64 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = 4 * tid + q;
                const u64 c = buf[min(i, nk - 1)];
                v[q] = (i < nk) ? (((u64)(uint32_t)comp_idx(c) << 32) | (c >> 32)) : ~0ull;
            }
            __syncthreads();
            rsort1024<false>(v, f.sortk);
            HSAMP_PHASE(9500 + r, 6);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = 4 * tid + q;
                if (j < nk) {
                    f.fidx[j] = (int32_t)(v[q] >> 32);
                    f.fv[j] = key_to_float((uint32_t)v[q]);
                    f.keep[j] = 1;
                }
            }
        }
        __syncthreads();
        if (a.topk_idx != nullptr) {
            for (int j = tid; j < nk && j < a.set_cap; j += kBlock)
                a.topk_idx[(int64_t)r * a.set_cap + j] = f.fidx[j];
        }
        if (a.topk_count != nullptr && tid == 0) a.topk_count[r] = single ? -1 : nk;

        bool have = fin_softmax(f_, nk, st);
        HSAMP_PHASE(9500 + r, 7);
        bool fresh = true;  // fp matches the current kept set
        if (have && (P.flags & RF_TOPP)) {
            // sampler.cpp:146-164: (probability, -position) descending
            {
                u64 v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = 4 * tid + q;
                    const int ic = min(i, nk - 1);
                    v[q] = (i < nk && f.keep[ic])
                               ? (((u64)key32(f.fp[ic]) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)i))
                               : 0ull;
                }
                rsort1024<true>(v, f.sortk);
#pragma unroll
                for (int q = 0; q < 4; ++q) f.sortk[4 * tid + q] = v[q];
            }
            __syncthreads();
            if (tid < 64) {
                // the running float sum in that order (entries not kept sort
                // last as 0 and add +0)
                float c;
                const int hit = wave_seq_sum_f(
                    nk,
                    [&](int i) {
                        const u64 e = f.sortk[i];
                        return e == 0ull ? 0.0f : f.fp[(int)(0xFFFFFFFFu - (uint32_t)e)];
                    },
                    true, P.top_p, &c);
                const int cutoff = hit >= 0 ? hit + 1 : -1;
                if (tid == 0) {
                    if (cutoff > 0 && fabsf(c - P.top_p) <= 1e-6f) rflags |= ROWF_TOPP_NEAR;
                    st.cutoff = cutoff;
                    st.flags = (int)rflags;
                }
            }
            __syncthreads();
            rflags = (uint32_t)st.flags;
            const int cutoff = st.cutoff;
            if (cutoff > 0) {
                for (int i = tid; i < nk; i += kBlock) {
                    const u64 e = f.sortk[i];
                    if (e != 0ull && i >= cutoff) f.keep[(int)(0xFFFFFFFFu - (uint32_t)e)] = 0;
                }
                __syncthreads();
                fresh = false;
            }
        }
        HSAMP_PHASE(9500 + r, 8);
        if (have && (P.flags & RF_MINP)) {
            // sampler.cpp:167-176
            if (!fresh) have = fin_softmax(f_, nk, st);
            fresh = true;
            if (have) {
                float mp = 0.0f;
                for (int j = tid; j < nk; j += kBlock)
                    if (f.keep[j]) mp = fmaxf(mp, f.fp[j]);
                mp = block_max_f(mp, st);
                const float thr = P.min_p * mp;
                int dropped = 0;
                for (int j = tid; j < nk; j += kBlock)
                    if (f.keep[j] && f.fp[j] < thr) {
                        f.keep[j] = 0;
                        dropped = 1;
                    }
                int any;
                block_excl_scan(dropped, &any, st);
                if (any) fresh = false;
            }
        }
        if (have && !fresh) have = fin_softmax(f_, nk, st);
        HSAMP_PHASE(9500 + r, 9);
        if (have) {
            // sampler.cpp:178-182 / discrete_distribution: double sum S, q = p / S,
            // partial sums of q (cp[V-1] = 1), the first cp >= u. A tree prefix
            // of p over its tree total decides when every comparison that
            // decides the token and the CDF_NEAR flag is clear of u by 2e-6
            // (for <= 1024 terms the tree and the sequential sums, quotients
            // and partial sums differ by < 1e-12); otherwise the reference's
            // sequential sums on one thread.
            bool decided = false;
            if (single || !(u > 0.0)) {
                if (tid == 0) {
                    st.tok = 0;
                    st.flags = (int)rflags;
                }
                decided = true;
            } else if (nk <= 4 * kBlock) {
                double pd[4], c4[4], run = 0.0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = 4 * tid + q;
                    pd[q] = (j < nk && f.keep[j]) ? (double)f.fp[j] : 0.0;
                    run = run + pd[q];
                    c4[q] = run;
                }
                if (tid == 0) st.tok = INT32_MAX;
                double tot;
                const double base = block_excl_scan_d(run, &tot, st);   // (its barriers publish st.tok)
                int hit = INT32_MAX;
                double at = 0.0, before = 0.0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = 4 * tid + q;
                    if (hit == INT32_MAX && j < nk && f.keep[j]) {
                        const double cp = (base + c4[q]) / tot;
                        const double cj = (f.fidx[j] == V - 1) ? 1.0 : cp;
                        if (cj >= u) {
                            hit = j;
                            at = cj;
                            before = (base + c4[q] - pd[q]) / tot;
                        }
                    }
                }
                if (hit != INT32_MAX) atomicMin(&st.tok, hit);
                __syncthreads();
                const int h0 = st.tok;
                if (hit != INT32_MAX && hit == h0) {
                    st.hat = at;
                    st.hbefore = before;
                }
                __syncthreads();
                const bool clear = (h0 != INT32_MAX) ? (fabs(st.hat - u) > 2e-6 && fabs(st.hbefore - u) > 2e-6)
                                                     : fabs(1.0 - u) > 2e-6;
                if (clear) {
                    decided = true;
                    __syncthreads();   // every thread has read st.tok / st.hat
                    if (tid == 0) {
                        st.tok = (h0 != INT32_MAX) ? f.fidx[h0] : V - 1;
                        st.flags = (int)rflags;
                    }
                }
            }
            if (!decided) {
                lds_f64* fq = (lds_f64*)f.sortk;
                if (tid == 0) {
                    double S = 0.0;
                    for (int j = 0; j < nk; ++j)
                        if (f.keep[j]) S = S + (double)f.fp[j];
                    st.dS = S;
                }
                __syncthreads();
                const double S = st.dS;
                for (int j = tid; j < nk; j += kBlock) fq[j] = f.keep[j] ? (double)f.fp[j] / S : 0.0;
                __syncthreads();
                if (tid == 0) {
                    int32_t t = V - 1;
                    double near = 1.0;
                    double cp = 0.0, prev = 0.0;
                    bool found = false;
                    for (int j = 0; j < nk; ++j) {
                        if (!f.keep[j]) continue;
                        prev = cp;
                        cp = cp + fq[j];
                        const double c = (f.fidx[j] == V - 1) ? 1.0 : cp;
                        if (c >= u) {
                            t = f.fidx[j];
                            near = fmin(fabs(c - u), fabs(prev - u));
                            found = true;
                            break;
                        }
                    }
                    if (!found) near = fmin(fabs(1.0 - u), fabs(cp - u));
                    if (near <= 1e-6) rflags |= ROWF_CDF_NEAR;
                    st.tok = t;
                    st.flags = (int)rflags;
                }
            }
            __syncthreads();
            tok = st.tok;
            rflags = (uint32_t)st.flags;
        } else {
            nkept = 0;
        }
        HSAMP_PHASE(9500 + r, 10);
        if (have) {
            // kept ids in index order: one scan per 256 positions
            int running = 0;
            for (int base = 0; base < nk; base += kBlock) {
                const int j = base + tid;
                const int kj = (j < nk && f.keep[j]) ? 1 : 0;
                int total;
                const int pos = running + block_excl_scan(kj, &total, st);
                if (kj) {
                    if (a.kept_idx != nullptr && pos < a.set_cap) {
                        a.kept_idx[(int64_t)r * a.set_cap + pos] = f.fidx[j];
                        a.kept_prob[(int64_t)r * a.set_cap + pos] = f.fp[j];
                    }
                    if (a.fin_idx != nullptr && pos < a.fin_cap)
                        a.fin_idx[(int64_t)r * a.fin_cap + pos] = f.fidx[j];
                }
                running += total;
            }
            nkept = running;
        }
    } else {
        nkept = 0;
        if (a.topk_count != nullptr && tid == 0) a.topk_count[r] = single ? -1 : 0;
    }
    if (nkept == 0) {
        rflags |= ROWF_UNIFORM;
        if (tid == 0) tok = uniform_draw(V, u);
    }
    if (wave_id() == 0) emit_token_wave(a, r, tok);
    if (tid == 0) {
        if (a.row_flags != nullptr) a.row_flags[r] = rflags;
        if (a.kept_count != nullptr) a.kept_count[r] = nkept;
        if (a.fin_n != nullptr) a.fin_n[r] = nkept;
    }
    HSAMP_PHASE(9500 + r, 11);
}


// ---- wave-level finalize (k <= 64) -----------------------------------------------
// One wave finishes a row whose top-k set fits its 64 lanes. Cross-lane work
// goes through the wave's 512-byte LDS scratch (Shared::wv): a lane writes its
// value and every lane then reads all 64 with broadcast loads, so sorts are
// rank placements and the reference's sequential sums are one unrolled chain
// of adds per lane, in lane order, with no shuffles or readlanes.

// Ascending sort of 64 distinct keys across the lanes (payload travels along).
// All 64 keys are read before any is compared, so the LDS latency is paid once.
__device__ __forceinline__ void wave_sort_asc(uint32_t& key, uint32_t& pay, u64* wv) {
    const int lane = lane_id();
    uint32_t* w = reinterpret_cast<uint32_t*>(wv);
    w[lane] = key;
    wave_sync();
    const uint4* w4 = reinterpret_cast<const uint4*>(w);
    uint4 x[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) x[q] = w4[q];
    int rank = 0;
#pragma unroll
    for (int q = 0; q < 16; ++q) rank += (x[q].x < key) + (x[q].y < key) + (x[q].z < key) + (x[q].w < key);
    wave_sync();
    w[rank] = key;
    w[64 + rank] = pay;
    wave_sync();
    key = w[lane];
    pay = w[64 + lane];
    wave_sync();
}

// Descending sort of 64 distinct 64-bit keys across the lanes.
__device__ __forceinline__ u64 wave_sort_desc(u64 key, u64* wv) {
    const int lane = lane_id();
    wv[lane] = key;
    wave_sync();
    const ulonglong2* w2 = reinterpret_cast<const ulonglong2*>(wv);
    ulonglong2 x[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) x[q] = w2[q];
    int rank = 0;
#pragma unroll
    for (int q = 0; q < 32; ++q) rank += (x[q].x > key) + (x[q].y > key);
    wave_sync();
    wv[rank] = key;
    wave_sync();
    key = wv[lane];
    wave_sync();
    return key;
}

// Lane-order float sum of x over the 64 lanes, starting from +0.0f. Every
// value must be >= +0 (absent lanes pass +0.0f): the extra +0 terms then leave
// the index-order sum of the present ones bit for bit. Every lane reads all 64
// values up front and runs the same chain of adds.
__device__ __forceinline__ float wave_seq_sum_f(float x, u64* wv) {
    float* w = reinterpret_cast<float*>(wv);
    w[lane_id()] = x;
    wave_sync();
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = w4[q];
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        s = s + v[q].x;
        s = s + v[q].y;
        s = s + v[q].z;
        s = s + v[q].w;
    }
    wave_sync();
    return s;
}

// Inclusive lane-order prefix of the same sequential float sum: lane l gets
// the running sum after adding lane l's value.
__device__ __forceinline__ float wave_seq_prefix_f(float x, u64* wv) {
    const int lane = lane_id();
    float* w = reinterpret_cast<float*>(wv);
    w[lane] = x;
    wave_sync();
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = w4[q];
    float s = 0.0f, mine = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        s = s + v[q].x;
        mine = (lane == 4 * q) ? s : mine;
        s = s + v[q].y;
        mine = (lane == 4 * q + 1) ? s : mine;
        s = s + v[q].z;
        mine = (lane == 4 * q + 2) ? s : mine;
        s = s + v[q].w;
        mine = (lane == 4 * q + 3) ? s : mine;
    }
    wave_sync();
    return mine;
}

// The double versions (values >= +0.0).
__device__ __forceinline__ double wave_seq_sum_d(double x, u64* wv) {
    double* w = reinterpret_cast<double*>(wv);
    w[lane_id()] = x;
    wave_sync();
    const double2* w2 = reinterpret_cast<const double2*>(w);
    double2 v[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) v[q] = w2[q];
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        s = s + v[q].x;
        s = s + v[q].y;
    }
    wave_sync();
    return s;
}

__device__ __forceinline__ double wave_seq_prefix_d(double x, u64* wv) {
    const int lane = lane_id();
    double* w = reinterpret_cast<double*>(wv);
    w[lane] = x;
    wave_sync();
    const double2* w2 = reinterpret_cast<const double2*>(w);
    double2 v[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) v[q] = w2[q];
    double s = 0.0, mine = 0.0;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        s = s + v[q].x;
        mine = (lane == 2 * q) ? s : mine;
        s = s + v[q].y;
        mine = (lane == 2 * q + 1) ? s : mine;
    }
    wave_sync();
    return mine;
}


// softmax_probs (sampler.cpp:124-142) over the kept lanes of one wave; lanes
// are in index order. The float denominator is the index-order sequential sum.
// Returns false when nothing is kept.
__device__ __forceinline__ bool wave_softmax(float v, bool keep, float& p, u64* wv, const uint64_t* expT) {
    if (__ballot(keep) == 0ull) return false;
    const float m = wave_max_f(keep ? v : -__builtin_inff());
    const float e = keep ? libm_expf_t(v - m, expT) : 0.0f;
    const float s = wave_seq_sum_f(e, wv);
    p = keep ? ((s <= 0.0f) ? e : e * (1.0f / s)) : 0.0f;
    return true;
}

// Exact top-k (k <= 64) of the n <= 256 distinct nonzero composites buf[0..n)
// by one wave: the k-th largest composite by an MSB-first bitwise select over
// ballots (4 entries per lane), starting at the highest bit the entries do not
// share and stopping once the entries under the prefix are exactly the ones
// still needed. Lane l < min(k, n) returns one member of the set, any order.
__device__ __forceinline__ u64 wave_topk(const u64* buf, int n, int k, u64* wv) {
    const int lane = lane_id();
    u64 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (lane + 64 * i < n) ? buf[lane + 64 * i] : 0ull;
    if (n <= k) return v[0];
    u64 lo = ~0ull, hi = 0ull;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (v[i] != 0ull) lo = v[i] < lo ? v[i] : lo;
        hi = v[i] > hi ? v[i] : hi;
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const u64 a2 = shfl_xor_u64(lo, d), b2 = shfl_xor_u64(hi, d);
        lo = a2 < lo ? a2 : lo;
        hi = b2 > hi ? b2 : hi;
    }
    const int hb = 63 - __clzll((long long)(lo ^ hi));   // n >= 2 distinct: lo != hi
    u64 known = (hb >= 63) ? 0ull : ~((2ull << hb) - 1ull);
    u64 prefix = hi & known;
    int need = k, match = n;
    u64 kth = 0ull;
    bool found = false;
    for (int b = hb; b >= 0; --b) {
        const u64 bit = 1ull << b;
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            cnt += __popcll(__ballot(v[i] != 0ull && (v[i] & known) == prefix && (v[i] & bit) != 0ull));
        if (cnt >= need) {
            prefix |= bit;
            match = cnt;
        } else {
            need -= cnt;
            match -= cnt;
        }
        known |= bit;
        if (match == need) {
            // every entry under the prefix is in: the k-th is their minimum
            u64 mn = ~0ull;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (v[i] != 0ull && (v[i] & known) == prefix && v[i] < mn) mn = v[i];
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) {
                const u64 o = shfl_xor_u64(mn, d);
                mn = o < mn ? o : mn;
            }
            kth = mn;
            found = true;
            break;
        }
    }
    if (!found) kth = prefix;
    // the k members, packed into lanes 0..k-1
    int base = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool in = v[i] != 0ull && v[i] >= kth;
        const u64 bal = __ballot(in);
        if (in) wv[base + __popcll(bal & ((1ull << lane) - 1ull))] = v[i];
        base += __popcll(bal);
    }
    wave_sync();
    const u64 c = (lane < k) ? wv[lane] : 0ull;
    wave_sync();
    return c;
}

// The ladder after top-k for one row, by one wave: lane l < nk holds a
// composite of the row's top-k set (any order), nk <= 64. Same semantics as
// finalize_row.
__device__ __forceinline__ void wave_finalize(const StreamArgs& a, const RowPlan& P, int r, u64 c, int nk,
                                                        uint32_t rflags, Shared& st) {
    const int lane = lane_id();
    const int V = a.vocab;
    const double u = st.u;
    const bool single = (P.flags & RF_SINGLE) != 0;
    u64* wv = st.wv;
    if (!single) rflags |= ROWF_U_USED;
    // index order; absent lanes carry distinct ids above every token id
    uint32_t id = (lane < nk) ? (uint32_t)comp_idx(c) : (0x80000000u | (uint32_t)lane);
    uint32_t vk = (lane < nk) ? (uint32_t)(c >> 32) : 0u;
    wave_sort_asc(id, vk, wv);
    HSAMP_PHASE(8192 + r, 6);
    const bool has = lane < nk;
    const float v = key_to_float(vk);
    if (a.topk_idx != nullptr && has && lane < a.set_cap) a.topk_idx[(int64_t)r * a.set_cap + lane] = (int32_t)id;
    if (a.topk_count != nullptr && lane == 0) a.topk_count[r] = single ? -1 : nk;
    bool keep = has;
    float p = 0.0f;
    bool have = nk > 0 && wave_softmax(v, keep, p, wv, st.expT);
    HSAMP_PHASE(8192 + r, 7);
    bool fresh = true;
    if (have && (P.flags & RF_TOPP)) {
        // sampler.cpp:146-164: order by (p desc, index asc), float running sum;
        // absent lanes sort last with keys below 2^32
        const u64 key = keep ? (((u64)key32(p) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)lane)) : (u64)lane;
        const u64 srt = wave_sort_desc(key, wv);
        const bool real = srt > 0xFFFFFFFFull;
        const float ps = real ? key_to_float((uint32_t)(srt >> 32)) : 0.0f;
        // the first sorted entry whose running float sum reaches top_p: from
        // a tree prefix (within 5e-6 of the sequential sums of <= 64 values
        // up to 1) when the decision and the TOPP_NEAR flag are clear of it
        // by 1e-5 on both sides, else from the reference's sequential sums
        float cum = wave_tree_prefix_f(ps);
        {
            const u64 h0 = __ballot(real && cum >= P.top_p);
            const int c0 = (h0 != 0ull) ? __ffsll((long long)h0) - 1 : 64;
            const float at = (c0 < 64) ? readlane_f(cum, c0) : 0.0f;
            const float before = (c0 > 0) ? readlane_f(cum, min(c0, 64) - 1) : -1.0f;
            const bool clear = (c0 < 64 ? fabsf(at - P.top_p) > 1e-5f : true) &&
                               (c0 > 0 ? fabsf(before - P.top_p) > 1e-5f : true);
            if (!clear) cum = wave_seq_prefix_f(ps, wv);
        }
        const u64 hit = __ballot(real && cum >= P.top_p);
        if (hit != 0ull) {
            const int cutoff = __ffsll((long long)hit);   // entries kept in sorted order
            if (fabsf(readlane_f(cum, cutoff - 1) - P.top_p) <= 1e-6f) rflags |= ROWF_TOPP_NEAR;
            // sorted lane i tells index-order lane pos_i whether it stays
            uint32_t* w = reinterpret_cast<uint32_t*>(wv);
            w[lane] = 0u;
            wave_sync();
            if (real && lane < cutoff) w[(int)(0xFFFFFFFFu - (uint32_t)srt)] = 1u;
            wave_sync();
            keep = keep && w[lane] != 0u;
            wave_sync();
            fresh = false;
        }
    }
    if (have && (P.flags & RF_MINP)) {
        // sampler.cpp:167-176
        if (!fresh) have = wave_softmax(v, keep, p, wv, st.expT);
        fresh = true;
        if (have) {
            const float mp = wave_max_f(keep ? p : 0.0f);
            const float thr = P.min_p * mp;
            const bool drop = keep && p < thr;
            if (__ballot(drop) != 0ull) fresh = false;
            keep = keep && !drop;
        }
    }
    if (have && !fresh) have = wave_softmax(v, keep, p, wv, st.expT);
    int32_t tok = 0;
    const u64 km = have ? __ballot(keep) : 0ull;
    if (have) {
        // the kept set and its probabilities go out ahead of the draw
        const int pos = __popcll(km & ((1ull << lane) - 1ull));
        if (keep) {
            if (a.kept_idx != nullptr && pos < a.set_cap) {
                a.kept_idx[(int64_t)r * a.set_cap + pos] = (int32_t)id;
                a.kept_prob[(int64_t)r * a.set_cap + pos] = p;
            }
            if (a.fin_idx != nullptr && pos < a.fin_cap) a.fin_idx[(int64_t)r * a.fin_cap + pos] = (int32_t)id;
        }
        // sampler.cpp:178-182 / discrete_distribution: double sum, q, partial sums
        HSAMP_PHASE(8192 + r, 8);
        const double pd = keep ? (double)p : 0.0;
        HSAMP_PHASE(8192 + r, 9);
        int32_t t = V - 1;
        double near = 1.0;
        if (single) {
            t = 0;
        } else if (!(u > 0.0)) {
            t = 0;
        } else {
            // the partial sums as a tree prefix of p over its tree total
            // (within 1e-13 of the reference's sequential q = p / S and
            // partial sums of q) when every comparison that decides the token
            // and the CDF_NEAR flag is clear of u by 2e-6, else the
            // reference's sequential sum, quotients and partial sums
            const double pp = wave_tree_prefix_d(pd);
            double cp = pp / readlane_d(pp, 63);
            {
                const double cja = (keep && (int32_t)id == V - 1) ? 1.0 : cp;
                const u64 h0 = __ballot(keep && cja >= u);
                const int j0 = (h0 != 0ull) ? __ffsll((long long)h0) - 1 : 64;
                const double at = (j0 < 64) ? readlane_d(cja, j0) : readlane_d(cp, 63);
                const double before = (j0 > 0) ? readlane_d(cp, min(j0, 64) - 1) : -1.0;
                const bool clear = fabs(at - u) > 2e-6 && (j0 > 0 ? fabs(before - u) > 2e-6 : true) &&
                                   (j0 < 64 ? true : fabs(1.0 - u) > 2e-6);
                if (!clear) {
                    const double S = wave_seq_sum_d(pd, wv);
                    cp = wave_seq_prefix_d(keep ? pd / S : 0.0, wv);
                }
            }
            const double cj = (keep && (int32_t)id == V - 1) ? 1.0 : cp;
            const u64 hit = __ballot(keep && cj >= u);
            if (hit != 0ull) {
                const int j = __ffsll((long long)hit) - 1;
                t = __builtin_amdgcn_readlane((int)id, j);
                const double prev = (j > 0) ? readlane_d(cp, j - 1) : 0.0;
                near = fmin(fabs(readlane_d(cj, j) - u), fabs(prev - u));
            } else {
                near = fmin(fabs(1.0 - u), fabs(readlane_d(cp, 63) - u));
            }
        }
        if (near <= 1e-6) rflags |= ROWF_CDF_NEAR;
        HSAMP_PHASE(8192 + r, 10);
        tok = t;
    }
    const int nkept = __popcll(km);
    if (nkept == 0) {
        rflags |= ROWF_UNIFORM;
        if (lane == 0) tok = uniform_draw(V, u);
    }
    emit_token_wave(a, r, tok);
    if (lane == 0) {
        if (a.row_flags != nullptr) a.row_flags[r] = rflags;
        if (a.kept_count != nullptr) a.kept_count[r] = nkept;
        if (a.fin_n != nullptr) a.fin_n[r] = nkept;
    }
}

// The k largest of the n <= 256 distinct nonzero composites buf[0..n), in
// descending order, into st.wv[0..min(k, n)) (k <= 64): entry i's rank is the
// number of entries above it, counted against broadcast reads of the buffer.
__device__ __forceinline__ void block_rank_topk(u64* buf, int n, int k, Shared& st) {
    const int tid = threadIdx.x;
    if (tid == 0) buf[n] = 0ull;   // pad to pairs; 0 is below every composite
    __syncthreads();
    if (tid < n) {
        const u64 me = buf[tid];
        const ulonglong2* b2 = reinterpret_cast<const ulonglong2*>(buf);
        int rank = 0;
        for (int j = 0; j < (n + 1) >> 1; ++j) {
            const ulonglong2 x = b2[j];
            rank += (x.x > me) + (x.y > me);
        }
        if (rank < k) st.wv[rank] = me;
    }
    __syncthreads();
}

// The exact top-k of the buffer's n candidates, then the rest of the row.
// For k <= 64 the block ranks up to 256 candidates (more are first compacted)
// and wave 0 finishes alone; larger k finish with finalize_row.
__device__ __attribute__((noinline)) void select_and_finalize(const StreamArgs& a, const RowPlan& P, int r, u64* buf,
                                                              FinLds f, Shared& st, uint32_t rflags) {
    int n = st.n;
    const int k = P.top_k;
    if (k <= 64) {
        if (n > 256) {
            buf_compact(buf, k, st);
            n = st.n;
        }
        block_rank_topk(buf, n, k, st);
        if (threadIdx.x >= 64) return;
        const u64 c = (lane_id() < min(k, n)) ? st.wv[lane_id()] : 0ull;
        wave_finalize(a, P, r, c, min(k, n), rflags, st);
        return;
    }
    buf_compact(buf, k, st);
    HSAMP_PHASE(9500 + r, 5);
    finalize_row(a, P, r, buf, st.n, f, st, rflags);
}

// ---- the stream kernel ---------------------------------------------------------

// Append the register-held keys kv[i] of ids idx(i) selected by bit i of sv
// to the slice's list in global memory: each lane counts its selections, the
// wave reserves one range with a single LDS atomic, and each lane writes its
// entries in slot order. The list holds a whole slice, so it cannot overflow.
template <int NE, typename Idx>
__device__ __forceinline__ void append_sel(u64* out, const uint32_t (&kv)[NE], Idx idx, uint32_t sv, Shared& st) {
    const int lane = lane_id();
    const int cnt = __popc(sv);
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
    }
    const int wtot = __shfl(incl, 63, 64);
    if (wtot == 0) return;
    int base = 0;
    if (lane == 63) base = atomicAdd(&st.n, wtot);
    int pos = __shfl(base, 63, 64) + incl - cnt;
#pragma unroll
    for (int i = 0; i < NE; ++i)
        if ((sv >> i) & 1u) out[pos++] = comp(kv[i], idx(i));
}

// A lower bound on the kw-th largest of the 64 * G keys a wave holds (G per
// lane): the kw-th largest with its low 16 bits cleared, by a bitwise radix
// select of the high 16 bits over ballots. Keys of 0 stand for "no value".
__device__ __forceinline__ uint32_t wave_kth_bound16(const uint32_t (&g)[4], int G, int kw) {
    uint32_t prefix = 0u, known = 0u;
    int need = kw;
#pragma unroll
    for (int b = 31; b >= 16; --b) {
        const uint32_t bit = 1u << b;
        int cnt = 0;
        // under the prefix with this bit set: one AND and one compare
        const uint32_t kb = known | bit, pb = prefix | bit;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < G) cnt += __popcll(__ballot((g[i] & kb) == pb));
        }
        if (cnt >= need) prefix |= bit;
        else need -= cnt;
        known |= bit;
    }
    return prefix;
}

// One logit of a row, by id.
template <int DT>
__device__ __forceinline__ float load_logit(const char* rowp, int t) {
    if (DT == 0) return reinterpret_cast<const float*>(rowp)[t];
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(rowp)[t] << 16);
}

// One logit of a row, by id, the element type chosen at run time.
__device__ __forceinline__ float load_logit_dt(const char* rowp, int dtype, int t) {
    return dtype == 0 ? load_logit<0>(rowp, t) : load_logit<1>(rowp, t);
}

// N logits by id (t < 0: none, 0.0f), the element type chosen once for the
// batch so that all N loads are in flight together.
template <int N>
__device__ __forceinline__ void load_logits(const char* rowp, int dtype, const int32_t (&t)[N], float (&x)[N]) {
    if (dtype == 0) {
#pragma unroll
        for (int q = 0; q < N; ++q) x[q] = (t[q] >= 0) ? load_logit<0>(rowp, t[q]) : 0.0f;
    } else {
#pragma unroll
        for (int q = 0; q < N; ++q) x[q] = (t[q] >= 0) ? load_logit<1>(rowp, t[q]) : 0.0f;
    }
}

// Order keys of one tile's elements held by this thread. kv[i] = 0 marks
// "absent": past the slice end, or penalised (finished by k_merge).
//  - greedy (GR): mask, then key32; a NaN never wins (key 0) but is noted.
//  - sampling: mask, x * fl(1/T) (1.0f without temperature), NaN -> -inf
//    (noted), key32.
// x + 0.0f turns -0 into +0 and leaves every other value as it is, so ties
// between zeros of either sign go to the lower index as in the reference.
// With `flag` set, penalised ids keep their (pre-penalty) key and come back
// as bits of `pm` instead of being left out.
template <int DT, bool PEN, bool MASK, bool GR>
__device__ __forceinline__ void tile_keys(const uint4 (&raw)[Tile<DT>::NCH], int tb, int lo, int hi,
                                          const uint32_t* pbm, const uint32_t* mbm, float inv_t, bool flag,
                                          uint32_t (&kv)[Tile<DT>::NE], uint32_t& pm, bool& nanseen) {
    using T = Tile<DT>;
    const int tid = threadIdx.x;
    bool nanv = false;
    pm = 0u;
#pragma unroll
    for (int j = 0; j < T::NCH; ++j) {
        const int e0 = tb + (j * kBlock + tid) * T::VW;
        const int o = e0 - lo;
        const bool in = e0 < hi;   // whole chunks (VEC) or per element below
        // branch-free: the word index is clamped into the slice's words
        const int wi = min(o, hi - lo - 1) >> 5;
        uint32_t mb = 0xFFFFFFFFu, pb = 0u;
        if (MASK) {
            const uint32_t w = mbm[wi];
            mb = in ? (w >> (o & 31)) : 0u;
        }
        if (PEN) {
            const uint32_t w = pbm[wi];
            pb = in ? (w >> (o & 31)) : 0u;
        }
#pragma unroll
        for (int c = 0; c < T::VW; ++c) {
            float x = elem<DT>(raw[j], c);
            if (MASK) x = ((mb >> c) & 1u) ? x : -__builtin_inff();
            if (!GR) x = x * inv_t;                          // sampler.cpp:101-106
            x = x + 0.0f;
            const bool nan = x != x;
            const uint32_t b = __float_as_uint(x);
            uint32_t key = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
            key = nan ? (GR ? 0u : kKeyNegInf) : key;
            bool here = e0 + c < hi;
            if (PEN) {
                const bool pe = here && ((pb >> c) & 1u);
                pm |= pe ? (1u << (j * T::VW + c)) : 0u;
                here = here && (flag || !pe);
            }
            nanv |= nan && here;
            kv[j * T::VW + c] = here ? key : 0u;
        }
        // chunks are consumed in load order, each after its own load
        // (the loads complete in order), not all after the last
        __builtin_amdgcn_sched_barrier(0);
    }
    nanseen |= nanv;
}

// Marks id t in the slice's penalised-id bitmap: the ids the penalty stages
// touch (sampler.cpp:236-258), which k_merge finishes from the row's counts.
__device__ __forceinline__ void stream_mark(int t, int lo, int hi, uint32_t* pbm) {
    if (t >= lo && t < hi) atomicOr(&pbm[(t - lo) >> 5], 1u << ((t - lo) & 31));
}

// Per-block set-up of k_stream, before the first tiles are requested: the
// block's counters, the slice's allowed-id mask words and the penalised-id
// bitmap (one bit per slice id, in LDS), cleared, with the ids whose loads
// wait here (logit-bias ids, history positions past the first 8 * kBlock)
// already marked. Their waits thus never cover tile loads.
template <bool PEN, bool MASK>
__device__ __forceinline__ void stream_setup(const StreamArgs& a, const RowPlan& P, int r, int lo, int hi,
                                             bool greedy, bool pen, bool masked, int p0, int L,
                                             const int32_t* hrow, uint32_t* pbm, uint32_t* mbm, Shared& st) {
    const int tid = threadIdx.x;
    const int words = a.bitmap_words;
    if (tid == 0) {
        st.theta = kThetaFloor;
        st.n = greedy ? 1 : 0;   // a greedy row's argmax goes to out[0]
        st.flags = 0;
    }
    for (int i = tid; i < words; i += kBlock) {
        if (PEN) pbm[i] = 0u;
        if (masked) mbm[i] = (lo + 32 * i < hi) ? a.mask[(int64_t)r * a.mask_stride + (lo >> 5) + i] : 0u;
        else if (MASK) mbm[i] = 0xFFFFFFFFu;
    }
    __syncthreads();
    if (PEN && pen) {
        for (int p = p0 + 8 * kBlock + tid; p < L; p += kBlock) stream_mark(hrow[p], lo, hi, pbm);
        if (P.flags & RF_BIAS)
            for (int j = tid; j < P.bias_cnt; j += kBlock) stream_mark(a.bias_ids[P.bias_off + j], lo, hi, pbm);
    }
}

// The greedy row's slice (argmax of sampler.cpp:220-228): the first id of the
// largest key goes to out[0]; k_merge settles id 0 holding a NaN. In flag
// mode the penalised ids that can still win are appended too (flagged), for
// k_merge to find their true values.
template <int DT, bool VEC, bool PEN, bool MASK>
__device__ __forceinline__ void stream_greedy(const StreamArgs& a, const RowPlan& P, int r, int lo, int hi,
                                              __amdgpu_buffer_rsrc_t rs, uint4 (&raw)[Tile<DT>::NCH],
                                              u64* out, int64_t slot,
                                              const unsigned char* smem, Shared& st) {
    using T = Tile<DT>;
    const int tid = threadIdx.x;
    const uint32_t* pbm = reinterpret_cast<const uint32_t*>(smem);
    const uint32_t* mbm = pbm + a.bitmap_words;
    const bool pflag = a.pen_flag != 0;
    bool nanseen = false;
    uint32_t bk = 0u;          // best key and its first id so far
    int32_t bi = 0x7FFFFFFF;
    auto process = [&](const uint4 (&raw)[T::NCH], int tb) {
        uint32_t kv[T::NE];
        uint32_t pm;
        tile_keys<DT, PEN, MASK, true>(raw, tb, lo, hi, pbm, mbm, 1.0f, pflag, kv, pm, nanseen);
        const int bt = tb + tid * T::VW;
        uint32_t m = 0u;
#pragma unroll
        for (int i = 0; i < T::NE; ++i) m = max(m, ((pm >> i) & 1u) ? 0u : kv[i]);
        int32_t mi = 0x7FFFFFFF;
#pragma unroll
        for (int i = T::NE - 1; i >= 0; --i)
            mi = (kv[i] == m && !((pm >> i) & 1u)) ? (bt + (i / T::VW) * (kBlock * T::VW) + (i % T::VW)) : mi;
        if (m > bk || (m == bk && mi < bi)) {
            bk = m;
            bi = mi;
        }
        if (PEN && pflag && __ballot(pm != 0u) != 0ull) {
            // A penalised id's true value is at most its key here (penalties
            // only lower it), so only those reaching the wave's best key so
            // far can be the argmax; they go with the flag key kKeyFlag.
            uint32_t wb = bk;
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) wb = max(wb, (uint32_t)__shfl_xor((int)wb, d, 64));
            uint32_t sel = 0u;
#pragma unroll
            for (int i = 0; i < T::NE; ++i) sel |= (((pm >> i) & 1u) && kv[i] >= wb) ? (1u << i) : 0u;
            if (__ballot(sel != 0u) != 0ull) {
#pragma unroll
                for (int i = 0; i < T::NE; ++i) kv[i] = kKeyFlag;
                auto idx = [&](int i) -> int32_t { return bt + (i / T::VW) * (kBlock * T::VW) + (i % T::VW); };
                append_sel<T::NE>(out, kv, idx, sel, st);
            }
        }
    };
    for (int tb = lo;;) {
        process(raw, tb);
        tb += T::ELEMS;
        if (tb >= hi) break;
        load_tile<DT, VEC>(rs, tb, raw);
    }
    if (nanseen) atomicOr(&st.flags, 1);
    const u64 best = block_max_u64(bk != 0u ? comp(bk, bi) : 0ull, st);   // has the barrier the flag needs
    if (tid == 0) {
        out[0] = best;
        a.cand_n[slot] = st.n | ((st.flags & 1) ? (1 << 30) : 0);
    }
}

// A sampling row's slice: every id whose key can still be among the row's top
// k is appended (composite form). The bound: each wave's kw-th largest group
// maximum (kw = ceil(k/4)), low 16 bits cleared, minimum over the 4 waves;
// the block keeps the highest bound seen so far, and keys at or above it
// survive. In flag mode penalised ids keep their pre-penalty key (an upper
// bound of the true one), take no part in the bound and are appended flagged.
template <int DT, bool VEC, bool PEN, bool MASK>
__device__ __forceinline__ void stream_sample(const StreamArgs& a, const RowPlan& P, int r, int lo, int hi,
                                              __amdgpu_buffer_rsrc_t rs, uint4 (&raw)[Tile<DT>::NCH],
                                              u64* out, int64_t slot,
                                              const unsigned char* smem, Shared& st) {
    using T = Tile<DT>;
    const int tid = threadIdx.x;
    const uint32_t* pbm = reinterpret_cast<const uint32_t*>(smem);
    const uint32_t* mbm = pbm + a.bitmap_words;
    const int k = P.top_k;
    const int kw = (k + 3) >> 2;
    const int G = min(4, max(1, (kw + 63) >> 6));
    // flag mode: keys of the raw logits (x * 1.0f is x); k_merge applies the
    // penalties and the temperature to the candidates
    const bool pflag = a.pen_flag != 0;
    const float inv_t = pflag ? 1.0f : P.inv_temp;
    bool nanseen = false;
    // Group maxima over every tile so far: each group's maximum is a distinct
    // id of the slice, so the kw-th largest of them bounds the slice's k-th
    // key from below, and the bound tightens as tiles go by (a bound from the
    // current tile alone would let each tile add about k candidates).
    uint32_t gk[4] = {0u, 0u, 0u, 0u};
    auto process = [&](const uint4 (&raw)[T::NCH], int tb) {
        uint32_t kv[T::NE];
        uint32_t pm;
        tile_keys<DT, PEN, MASK, false>(raw, tb, lo, hi, pbm, mbm, inv_t, pflag, kv, pm, nanseen);
        uint32_t lm = 0u;
#pragma unroll
        for (int j = 0; j < T::NCH; ++j) {
#pragma unroll
            for (int c = 0; c < T::VW; ++c) {
                const int i = j * T::VW + c;
                gk[i / (T::NE / 4)] = max(gk[i / (T::NE / 4)], ((pm >> i) & 1u) ? 0u : kv[i]);
                lm = max(lm, kv[i]);
            }
        }
        uint32_t gb[4] = {gk[0], gk[1], gk[2], gk[3]};
        if (G == 2) {
            gb[0] = max(gk[0], gk[1]);
            gb[1] = max(gk[2], gk[3]);
        } else if (G == 1) {
            gb[0] = max(max(gk[0], gk[1]), max(gk[2], gk[3]));
        }
        const uint32_t tw = (kw <= 64 * G) ? wave_kth_bound16(gb, G, kw) : 0u;
        if (lane_id() == 0) st.twave[wave_id()] = tw;
        __syncthreads();
        uint32_t tt = st.twave[0];
#pragma unroll
        for (int i = 1; i < kBlock / 64; ++i) tt = min(tt, st.twave[i]);
        const uint32_t th0 = (uint32_t)(st.theta >> 32);
        __syncthreads();
        const uint32_t thk = max(max(tt, th0), (uint32_t)(kThetaFloor >> 32));
        if (tid == 0) st.theta = (u64)thk << 32;
        if (__ballot(lm >= thk) != 0ull) {
            uint32_t sv = 0u;
#pragma unroll
            for (int i = 0; i < T::NE; ++i) sv |= (kv[i] >= thk) ? (1u << i) : 0u;
            // penalised survivors go with the flag key kKeyFlag
            if (PEN) {
#pragma unroll
                for (int i = 0; i < T::NE; ++i) kv[i] = ((pm >> i) & 1u) ? kKeyFlag : kv[i];
            }
            const int bt = tb + tid * T::VW;
            auto idx = [&](int i) -> int32_t { return bt + (i / T::VW) * (kBlock * T::VW) + (i % T::VW); };
            append_sel<T::NE>(out, kv, idx, sv, st);
        }
    };
    for (int tb = lo;;) {
        process(raw, tb);
        tb += T::ELEMS;
        if (tb >= hi) break;
        load_tile<DT, VEC>(rs, tb, raw);
    }
    if (nanseen) atomicOr(&st.flags, 1);
    __syncthreads();
    if (tid == 0) {
        a.cand_n[slot] = st.n | ((st.flags & 1) ? (1 << 30) : 0);
        a.cand_th[slot] = (int32_t)(uint32_t)(st.theta >> 32);   // every id left out has a key below it
    }
}

// ---- exact lists ------------------------------------------------------------------
// Batches whose rows all sample with top-k <= 64 and whose penalties can only
// lower a logit (rep >= 1, freq/pres >= 0, no DRY, no bias) leave lists in
// which every candidate carries its final logit before temperature (the raw
// key below); k_pick applies the temperature. Every instruction a stream
// thread runs costs about 8 ns of its CU (some 19 waves share it), so the
// pass over the tile is lean:
//  A. as each 16-byte chunk arrives: the chunk's float maximum (v_max ignores
//     NaN) and one NaN test per two elements; nothing per element else.
//  B. the bound: each wave's kw-th largest lane maximum (kw = ceil((k+4)/4),
//     low 16 bits cleared), minimum over the waves: B, with at least k + 4
//     ids of the slice at or above it. ths = B's scaled key; every id whose
//     final key is below ths is beaten by them (if at least k of them keep a
//     final key >= ths, checked at the end) and left out. R = raw_edge(ths)
//     is the smallest raw key whose scaled key reaches ths, so the kept ids
//     are exactly those whose final raw key reaches R.
//  C. chunks whose maximum reaches R are staged in LDS (one wave-level prefix
//     and one LDS atomic per wave); D. one thread per staged chunk finds its
//     elements' final raw keys (penalised ids, nonzero count entry, take
//     stages 1-4 from the slice's history counts; a penalty only lowers the
//     key, so only ids at or above R before it can qualify) and appends those
//     that reach R.
//  E. when penalties took so many of them below R that fewer than k remain,
//     the block goes over the slice again down to the floor (rare).
// The slice's history counts sit in LDS, one 16-bit entry per slice id (XC_*).

constexpr int kStageCap = kBlock;          // staged chunks per round
constexpr uint32_t kKeyPosInf = 0xFF800000u;  // key32(+inf)

// Raw key of a logit: key32 without merging -0 into +0 (so that key_to_float
// gives x back), NaN as -inf. Non-decreasing in x.
__device__ __forceinline__ uint32_t raw_key(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
    return (x != x) ? kKeyNegInf : k;
}

// Final key of a raw key: temperature (sampler.cpp:101-106), -0 -> +0.
// Non-decreasing in the raw key; exact lists need 0 < inv_t < inf, so no NaN
// arises from a finite or infinite logit.
__device__ __forceinline__ uint32_t scaled_key(uint32_t kr, float inv_t) {
    float y = key_to_float(kr) * inv_t;
    y = y + 0.0f;
    return key32(y);
}

// The smallest raw key in [key(-FLT_MAX), key(+inf)] whose scaled key reaches
// ths (scaled_key(key(+inf)) = key(+inf) >= ths): from a first guess (ths's
// float times T) a few unit steps, else a binary search.
__device__ uint32_t raw_edge(uint32_t ths, float inv_t, float temp) {
    constexpr uint32_t lo0 = kKeyNegInf + 1u;
    const float g = key_to_float(ths) * temp;
    uint32_t r = raw_key(g);
    r = min(max(r, lo0), kKeyPosInf);
    for (int it = 0; it < 4 && r < kKeyPosInf && scaled_key(r, inv_t) < ths; ++it) ++r;
    for (int it = 0; it < 4 && r > lo0 && scaled_key(r - 1u, inv_t) >= ths; ++it) --r;
    if (scaled_key(r, inv_t) >= ths && (r == lo0 || scaled_key(r - 1u, inv_t) < ths)) return r;
    uint32_t lo = lo0, hi = kKeyPosInf;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (scaled_key(mid, inv_t) >= ths) hi = mid;
        else lo = mid + 1u;
    }
    return lo;
}

// Final raw key of slice id t (raw logit x, after the mask) with count entry
// h: stages 1-4 (sampler.cpp:28-99, those a count entry calls for), NaN ->
// -inf (noted). The entry's count is over the count window (the DRY window
// when DRY is on -- then also the frequency/presence window, or that stage is
// off -- else the frequency/presence window), which the DRY and
// frequency/presence stages take; one: the entry is a plain count over the
// whole scanned window (the repetition and count windows are equal, or one of
// them is off): the id repeats when it counts at all; else its repetition
// bit says so.
__device__ __forceinline__ float final_value(float x, int32_t t, uint32_t h, bool one, const StreamArgs& a,
                                             const RowPlan& P) {
    if (h == 0u) return x;
    const uint32_t c = h & XC_CNT_MASK;
    const uint32_t v = (one ? (P.rep_win > 0 && c > 0u ? HV_REP : 0u) : ((h & XC_REP) ? HV_REP : 0u)) |
                       ((h & XC_BIAS) ? HV_BIAS : 0u) | (P.fp_win > 0 ? c : 0u) |
                       (P.dry_win > 0 ? (c << HV_DRY_SHIFT) : 0u);
    return pen_value(x, t, v, a, P);
}
__device__ __forceinline__ uint32_t final_raw_key(float x, int32_t t, uint32_t h, bool one, const StreamArgs& a,
                                                  const RowPlan& P, bool& nan) {
    if (h == 0u) return raw_key(x);
    const float y = final_value(x, t, h, one, a, P);
    if (y != y) {
        nan = true;
        return kKeyNegInf;
    }
    return raw_key(y);
}

// A lower bound on the need-th largest of the block's chunk maxima (raw
// keys): at least `need` chunks of the slice, so at least `need` ids, have a
// maximum at or above it. Two levels of a 256-bin LDS histogram over the bits
// below those all finite maxima share (the block's key range), the second
// within the first's chosen bin; the bound keeps those 16 bits (or all, when
// the range is narrower). Binning by the varying bits keeps the bins' LDS
// atomics apart: the top byte alone (sign and high exponent bits) puts nearly
// every maximum in one or two bins, whose atomics then serialise. The
// large-k form of the waves' own bound (their kw-th largest lane maximum
// needs kw <= 64).
template <int NC>
__device__ uint32_t block_kth_bound16(const float (&cm)[NC], int need, Shared& st) {
    const int tid = threadIdx.x, lane = lane_id();
    uint32_t key[NC];
    uint32_t lmx = 0u, lmn = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        key[j] = raw_key(cm[j]);
        if (key[j] > kKeyNegInf) {
            lmx = max(lmx, key[j]);
            lmn = min(lmn, key[j]);
        }
    }
    lmx = wave_max_u32(lmx);
    lmn = wave_min_u32(lmn);
    if (lane == 0) {
        st.twave[wave_id()] = lmn;
        st.minv_w[wave_id()] = lmx;
    }
    __syncthreads();
    uint32_t kmn = st.twave[0], kmx = (uint32_t)st.minv_w[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) {
        kmn = min(kmn, st.twave[i]);
        kmx = max(kmx, (uint32_t)st.minv_w[i]);
    }
    if (kmx < kmn) return 0u;   // no finite maximum: every chunk qualifies
    const int hb = (kmx > kmn) ? 31 - __clz((int)(kmn ^ kmx)) : 0;
    const int sh1 = max(0, hb - 7), sh2 = max(0, sh1 - 8);
    const uint32_t top = hb >= 31 ? 0u : (kmx >> (hb + 1)) << (hb + 1);   // the shared bits
    uint32_t prefix = top;
    const int levels = sh1 > 0 ? 2 : 1;
    for (int level = 0; level < levels; ++level) {
        const int sh = level == 0 ? sh1 : sh2;
        const uint32_t b1 = level == 0 ? 0u : (prefix >> sh1) & 255u;
        st.hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const bool in = key[j] >= kmn && (level == 0 || ((key[j] >> sh1) & 255u) == b1);
            if (in) atomicAdd(&st.hist[(key[j] >> sh) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            // bins from the top: lane l holds 255 - 4l .. 252 - 4l
            const int c0 = st.hist[255 - 4 * lane], c1 = st.hist[254 - 4 * lane];
            const int c2 = st.hist[253 - 4 * lane], c3 = st.hist[252 - 4 * lane];
            const int s4 = c0 + c1 + c2 + c3;
            const int incl = wave_incl_sum_i(s4);
            const int excl = incl - s4;
            if (lane == 0) st.sel_d = -1;   // fewer than need at or above kmn
            if (excl < need && need <= incl) {
                int q, before;
                if (excl + c0 >= need) { q = 0; before = excl; }
                else if (excl + c0 + c1 >= need) { q = 1; before = excl + c0; }
                else if (excl + c0 + c1 + c2 >= need) { q = 2; before = excl + c0 + c1; }
                else { q = 3; before = excl + c0 + c1 + c2; }
                st.sel_d = 255 - 4 * lane - q;
                st.sel_need = need - before;
            }
        }
        __syncthreads();
        const int d = st.sel_d;
        need = st.sel_need;
        __syncthreads();   // sel_d and the bins are read before the next level
        if (d < 0) return 0u;   // too few finite maxima: every chunk qualifies
        prefix |= (uint32_t)d << sh;
    }
    return prefix;
}

// A sampling or greedy row's slice [lo, hi) with exact lists (one, two or
// four tiles, raw[] holds them); the row's last slice (last_slice) also takes
// the ragged end that whole-chunk loads leave out.
// LEAN: no row of the launch is greedy or has a logit bias, and every
// penalty row counts over one window (a count entry is a plain count): those
// paths are compiled out.
template <int DT, bool VEC, bool PEN, bool MASK, int NC, bool LEAN>
__device__ __forceinline__ void stream_exact(const StreamArgs& a, const RowPlan& P, int r, int lo, int hi,
                                             const uint4 (&raw)[NC], u64* out, int64_t slot,
                                             bool last_slice, bool pen, bool mk, const int32_t (&pre)[8],
                                             int pbase, unsigned char* smem, Shared& st) {
    using T = Tile<DT>;
    constexpr int NT = NC / T::NCH;   // tiles per slice
    const int tid = threadIdx.x, lane = lane_id();
    // History counts, 16-bit entries: one per slice id (dense), or (ranked:
    // four-tile slices, whose dense table would take 64 KB of LDS and hold
    // the blocks per CU to two) a bitmap over the slice's ids marks those in
    // the scanned window and each marked id's entry sits at its rank among
    // them (the word's rank prefix plus the bits below it in the word).
    constexpr bool ranked = NT == 4;
    const int bw = a.bitmap_words;
    uint32_t* hbm = reinterpret_cast<uint32_t*>(smem);
    uint16_t* hwr = reinterpret_cast<uint16_t*>(smem + align16u(4u * (uint32_t)bw));
    uint32_t* hcw = ranked ? reinterpret_cast<uint32_t*>(smem + align16u(4u * (uint32_t)bw) + align16u(2u * (uint32_t)bw))
                           : reinterpret_cast<uint32_t*>(smem);
    auto hrank = [&](uint32_t o) -> uint32_t {
        return (uint32_t)hwr[o >> 5] + (uint32_t)__popc(hbm[o >> 5] & ((1u << (o & 31)) - 1u));
    };
    // nonzero when slice offset o (< slice_len) has a count entry
    auto hmark = [&](uint32_t o) -> uint32_t {
        return ranked ? (hbm[o >> 5] >> (o & 31)) & 1u : (hcw[o >> 1] >> ((o & 1u) << 4)) & 0xFFFFu;
    };
    auto hentry = [&](uint32_t o, uint32_t mark) -> uint32_t {
        if (!ranked || mark == 0u) return mark;
        const uint32_t rk = hrank(o);
        return (hcw[rk >> 1] >> ((rk & 1u) << 4)) & 0xFFFFu;
    };
    const uint32_t* mbm = reinterpret_cast<const uint32_t*>(smem) + a.mbm_off;
    // staged chunks: 32-byte slots, 16 bytes of logits then the chunk's first id
    unsigned char* stg = smem + a.stage_off;
    constexpr uint32_t kFloor = (uint32_t)(kThetaFloor >> 32);

    // A. the slice's history counts, while the tile is still on its way (the
    // history row and the plan were asked for first). Exact lists take DRY
    // only where its window is also the frequency/presence window (or that
    // stage is off), so one count serves both: the count window cw is the DRY
    // window when DRY is on, else the frequency/presence window; the scanned
    // window is the larger of it and the repetition window. When those two
    // are equal (or one is off) a count entry is a plain count over it (one
    // atomic per id); else a count over cw and a repetition bit.
    const int cw = P.dry_win > 0 ? P.dry_win : P.fp_win;
    const bool one = LEAN || P.rep_win == 0 || cw == 0 || P.rep_win == cw;
    // The row's logit-bias ids (at most kBlock): each marks its entry, and
    // each is evaluated on its own (bias_pass below: a bias can raise a logit
    // above the bound, so the chunk maxima cannot stand for it); the element
    // passes leave them out. (Their ids and logits are read again there:
    // values held from here to there would cost every row registers.)
    const bool bias = !LEAN && PEN && pen && (P.flags & RF_BIAS) != 0;
    const uint32_t bsl = (uint32_t)(min(a.vocab, lo + a.slice_len) - lo);
    auto bias_off = [&]() -> uint32_t {   // this thread's bias id, as a slice offset (>= bsl: none)
        return tid < P.bias_cnt ? (uint32_t)(a.bias_ids[P.bias_off + tid] - lo) : 0xFFFFFFFFu;
    };
    if (PEN && pen) {
        const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
        const uint32_t wl = (uint32_t)(L - p0), sl = bsl;
        const uint32_t ob = bias ? bias_off() : 0xFFFFFFFFu;
        uint32_t inw = 0u;   // bit q: pre[q] is a window id of this slice
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int p = pbase + q * kBlock + tid;   // pre[q]'s history position
            const uint32_t o = (uint32_t)(pre[q] - lo);
            if ((uint32_t)(p - p0) < wl && o < sl) {
                inw |= 1u << q;
                if constexpr (ranked) atomicOr(&hbm[o >> 5], 1u << (o & 31));
            }
        }
        if (ranked && bias && ob < sl) atomicOr(&hbm[ob >> 5], 1u << (ob & 31));
        if constexpr (ranked) {
            __syncthreads();
            // rank prefixes of the bitmap words: thread t takes words NT t .. NT t + NT - 1
            int c = 0;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const int w = tid * NT + i;
                c += w < bw ? __popc(hbm[w]) : 0;
            }
            int tot;
            int base = block_excl_scan(c, &tot, st);
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const int w = tid * NT + i;
                if (w < bw) {
                    hwr[w] = (uint16_t)base;
                    base += __popc(hbm[w]);
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if ((inw >> q) & 1u) {
                const int p = pbase + q * kBlock + tid;
                const uint32_t o = (uint32_t)(pre[q] - lo);
                const uint32_t e = ranked ? hrank(o) : o;
                const uint32_t sh = (e & 1u) << 4;
                if (one) {
                    atomicAdd(&hcw[e >> 1], 1u << sh);
                } else {
                    if (p >= L - cw) atomicAdd(&hcw[e >> 1], 1u << sh);
                    if (p >= L - P.rep_win) atomicOr(&hcw[e >> 1], XC_REP << sh);
                }
            }
        }
        if (bias && ob < sl) {
            const uint32_t e = ranked ? hrank(ob) : ob;
            atomicOr(&hcw[e >> 1], XC_BIAS << ((e & 1u) << 4));
        }
    }
    // B. chunk maxima, as the chunks arrive: IEEE maximum (NaN-propagating,
    // -0 < +0 as raw keys order them), so that a NaN shows in its chunk's
    // maximum; such chunks then take the NaN-ignoring maximum of their other
    // ids (NaN ids count as -inf), after the loop
    // (opaque: the chunk's words pass through an empty asm statement first, so
    // that the elements are unpacked anew there instead of being kept, and
    // spilled to scratch memory, from the maxima's pass for the NaN fix-up)
    auto chunk_v = [&](uint4 rv, int j, bool opaque, float (&x)[T::VW]) {
        if (opaque) __asm__("" : "+v"(rv.x), "+v"(rv.y), "+v"(rv.z), "+v"(rv.w));
        const int e0 = lo + (j * kBlock + tid) * T::VW;
#pragma unroll
        for (int c = 0; c < T::VW; ++c) x[c] = elem<DT>(rv, c);
        if (MASK) {
            const int o = e0 - lo;
            const uint32_t mb = mbm[max(0, min(o, hi - lo - 1)) >> 5] >> (o & 31);
#pragma unroll
            for (int c = 0; c < T::VW; ++c) x[c] = ((mb >> c) & 1u) ? x[c] : -__builtin_inff();
        }
        if (!VEC) {
            // element loads: the slice's last chunk may end inside (past hi reads 0)
#pragma unroll
            for (int c = 0; c < T::VW; ++c) x[c] = (e0 + c < hi) ? x[c] : -__builtin_inff();
        }
    };
    auto chunk = [&](int j, float (&x)[T::VW]) { chunk_v(raw[j], j, false, x); };
    float cm[NC];
    bool nanv = false;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        float x[T::VW];
        chunk(j, x);
        float m = x[0];
#pragma unroll
        for (int c = 1; c < T::VW; ++c) m = __builtin_elementwise_maximum(m, x[c]);
        nanv |= m != m;
        cm[j] = m;
        __builtin_amdgcn_sched_barrier(0);
    }
    if (nanv) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (cm[j] != cm[j]) {
                float x[T::VW];
                chunk_v(raw[j], j, true, x);
                float m = -__builtin_inff();
#pragma unroll
                for (int c = 0; c < T::VW; ++c) m = (x[c] == x[c]) ? __builtin_elementwise_maximum(m, x[c]) : m;
                cm[j] = m;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j)
        if (lo + (j * kBlock + tid) * T::VW >= hi) cm[j] = -__builtin_inff();
    HSAMP_PHASE(slot, 3);

    HSAMP_PHASE(slot, 10);
    // the lane's largest chunk maximum as a raw key (cm is never NaN)
    float lmf = cm[0];
#pragma unroll
    for (int j = 1; j < NC; ++j) lmf = __builtin_elementwise_maximum(lmf, cm[j]);
    const uint32_t lk = raw_key(lmf);
    // a greedy row (argmax, sampler.cpp:220-228) keeps the ids that can be its
    // largest final logit: the lists of top-k 1, no temperature
    const bool greedy = !LEAN && (P.flags & RF_GREEDY) != 0;
    const int k = greedy ? 1 : P.top_k;
    uint32_t tw;
    if (k <= 64) {
        const int kw = (k + 4 + 3) >> 2;   // <= 17
        const uint32_t g4[4] = {lk, 0u, 0u, 0u};
        tw = wave_kth_bound16(g4, 1, kw);
    } else {
        tw = block_kth_bound16(cm, k + 4, st);   // (the same for every wave)
    }
    if (lane == 0) st.twave[wave_id()] = tw;
    HSAMP_PHASE(slot, 11);
    // the ragged end (the row's last slice): read while the bound settles
    float xt = 0.0f;
    const bool tl = VEC && last_slice && tid < a.vec_tail;
    const int32_t tt_id = a.vocab - a.vec_tail + tid;
    if (tl) {
        const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * T::ES;
        xt = load_logit<DT>(rowp, tt_id);
        if (mk && !((a.mask[(int64_t)r * a.mask_stride + (tt_id >> 5)] >> (tt_id & 31)) & 1u)) xt = -__builtin_inff();
    }
    __syncthreads();   // also publishes the history counts
    HSAMP_PHASE(slot, 4);
    uint32_t thr = st.twave[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) thr = min(thr, st.twave[i]);
    thr = max(thr, kFloor);
    const float inv_t = P.inv_temp;
    // R: thr itself when the raw key below it scales below ths (the usual
    // case; a greedy row's keys are not scaled), else the search
    const uint32_t sthr = scaled_key(thr, inv_t);
    uint32_t R = thr;
    if (!greedy && !(sthr >= kFloor && (thr == kFloor || scaled_key(thr - 1u, inv_t) < sthr)))
        R = raw_edge(max(sthr, kFloor), inv_t, P.temp);
    // a greedy row whose id 0 ends NaN (after its mask and penalties) samples
    // id 0: no later logit compares greater (sampler.cpp:220-228)
    if (greedy && lo == 0 && tid == 0) {
        float x[T::VW];
        chunk(0, x);
        const float y = PEN ? final_value(x[0], 0, hentry(0u, hmark(0u)), one, a, P) : x[0];
        if (y != y) atomicOr(&st.flags, 2);
    }
    HSAMP_PHASE(slot, 7);

    // C, D. the ids whose final raw key lies in [Rlo, Rhi). Each wave stages
    // its own chunks whose maximum reaches Rlo (as floats: a superset of the
    // raw-key test, which orders -0 below +0) into its own LDS slots, in
    // (lane, chunk) order from one wave scan of the lanes' counts, and runs
    // them one element per lane: no block barrier between staging and the
    // pass.
    constexpr int kCapW = kStageCap / (kBlock / 64);   // slots per wave and round
    unsigned char* wst = stg + (uint32_t)wave_id() * (uint32_t)kCapW * 32u;
    auto pass = [&](uint32_t Rlo, uint32_t Rhi) {
        const float Rf = key_to_float(Rlo);
        // the wave's chunks at positions [rb, rb + kCapW) of its order (lane,
        // then chunk): each lane counts its own, one wave scan places them
        auto stage = [&](int rb) -> int {
            int c = 0;
#pragma unroll
            for (int j = 0; j < NC; ++j) c += cm[j] >= Rf ? 1 : 0;
            const int incl = wave_incl_sum_i(c);
            const int tot = __builtin_amdgcn_readlane(incl, 63);
            uint32_t p = (uint32_t)(incl - c - rb);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const bool in = cm[j] >= Rf;
                if (in && p < (uint32_t)kCapW) {
                    unsigned char* sp = wst + p * 32u;
                    *reinterpret_cast<uint4*>(sp) = raw[j];
                    *reinterpret_cast<int32_t*>(sp + 16) = lo + (j * kBlock + tid) * T::VW;
                }
                p += in ? 1u : 0u;
            }
            return tot;
        };
        HSAMP_PHASE(slot, 12);
        bool nanp = false;
        const int wtot = stage(0);
        for (int rb = 0; rb < wtot; rb += kCapW) {
            if (rb > 0) stage(rb);
            wave_sync();
            HSAMP_PHASE(slot, 8);
            // VW lanes per staged chunk, one element each; every lane runs
            // every step, so each step appends with one ballot and one atomic
            const int ne = min(kCapW, wtot - rb) * T::VW;
            for (int e1 = 0; e1 < ne; e1 += 64) {
                const int e = e1 + lane;
                const int ci = e / T::VW, c = e % T::VW;
                const unsigned char* sp = wst + (uint32_t)min(ci, kCapW - 1) * 32u;
                const int t = *reinterpret_cast<const int32_t*>(sp + 16) + c;
                const int o = t - lo;
                const uint32_t wsel = reinterpret_cast<const uint32_t*>(sp)[DT == 0 ? c : (c >> 1)];
                float x = (DT == 0) ? __uint_as_float(wsel)
                                    : __uint_as_float((c & 1) ? (wsel & 0xFFFF0000u) : (wsel << 16));
                // one branch, for the penalised ids; the rest is straight-line
                const bool live = e < ne && (VEC || t < hi);
                const uint32_t oc = min((uint32_t)o, (uint32_t)(a.slice_len - 1));
                if (MASK && !((mbm[oc >> 5] >> (oc & 31)) & 1u)) x = -__builtin_inff();
                uint32_t kf = raw_key(x);
                const uint32_t hm = PEN ? hmark(oc) : 0u;
                uint32_t hv = 0u;
                if (PEN && live && hm != 0u && kf >= Rlo) {
                    hv = hentry(oc, hm);
                    kf = final_raw_key(x, t, hv, one, a, P, nanp);
                }
                const bool keep = live && kf >= Rlo && kf < Rhi && !(hv & XC_BIAS);
                const u64 mk2 = __ballot(keep);
                if (mk2 != 0ull) {
                    int ob = 0;
                    if (lane == 0) ob = atomicAdd(&st.n, __popcll(mk2));
                    ob = __builtin_amdgcn_readfirstlane(ob);
                    if (keep)
                        out[ob + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk2 >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)mk2, 0u))] =
                            comp(kf, t);
                }
            }
            wave_sync();   // the slots are read before the next round writes them
        }
        if (tl) {
            const uint32_t ht = PEN ? hentry((uint32_t)(tt_id - lo), hmark((uint32_t)(tt_id - lo))) : 0u;
            const uint32_t kf = final_raw_key(xt, tt_id, ht, one, a, P, nanp);
            if (kf >= Rlo && kf < Rhi && !(ht & XC_BIAS)) out[atomicAdd(&st.n, 1)] = comp(kf, tt_id);
        }
        if (nanp) atomicOr(&st.flags, 1);
        HSAMP_PHASE(slot, 9);
        __syncthreads();
    };
    // The bias ids of the slice whose final raw key lies in [Rlo, Rhi).
    auto bias_pass = [&](uint32_t Rlo, uint32_t Rhi) {
        if (!bias) return;
        bool nanb = false;
        const uint32_t ob = bias_off();
        const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * T::ES;
        const float xb = load_logit<DT>(rowp, lo + (int)min(ob, bsl - 1u));   // (clamped: no branch)
        if (ob < bsl) {
            float x = xb;
            if (MASK && !((mbm[ob >> 5] >> (ob & 31)) & 1u)) x = -__builtin_inff();
            const int t = lo + (int)ob;
            const uint32_t kf = final_raw_key(x, t, hentry(ob, hmark(ob)), one, a, P, nanb);
            if (kf >= Rlo && kf < Rhi) out[atomicAdd(&st.n, 1)] = comp(kf, t);
        }
        if (nanb) atomicOr(&st.flags, 1);
        __syncthreads();
    };
    pass(R, 0xFFFFFFFFu);
    bias_pass(R, 0xFFFFFFFFu);
    HSAMP_PHASE(slot, 5);
    // E. fewer than k ids kept above a raised bound (penalties took the rest
    // below it): every id down to the floor
    if (PEN && st.n < k) {
        const uint32_t Rf = greedy ? kFloor : raw_edge(max(scaled_key(kFloor, inv_t), kFloor), inv_t, P.temp);
        if (R > Rf) {
            pass(Rf, R);
            bias_pass(Rf, R);
        }
    }
    if (nanv) atomicOr(&st.flags, 1);
    __syncthreads();
    // bit 30: a NaN logit in the slice; bit 29: a greedy row's id 0 is NaN
    if (tid == 0) a.cand_n[slot] = st.n | ((st.flags & 1) ? (1 << 30) : 0) | ((st.flags & 2) ? (1 << 29) : 0);
    // the rest of k_pick's window reads as empty (it then needs no lengths)
    for (int i = st.n + tid; i < a.win; i += kBlock) out[i] = 0ull;
    HSAMP_PHASE(slot, 6);
}

// One block per (row, slice): stream the slice once and leave for k_merge the
// ids whose key can still be among the row's top k (all of them, in composite
// form), or the slice's argmax for a greedy row. Penalised ids (history window
// or logit bias) are left out, or in flag mode appended with a flag: k_merge
// finishes them from the row's counts.
// PEN / MASK: some row of the launch has penalties / an allowed-token mask.
// LDS: [penalised-id bitmap][allowed-id mask words], one bit per slice id.
// GR: the launch's greedy rows (true) or sampling rows (false); a batch with
// both takes one launch of each, so that each loop has the whole register
// budget of five blocks per CU.
// EX: exact lists (sampling and greedy rows, see stream_exact); LDS then
// [history counts (PEN): 2 B per slice id, or (four-tile slices) a bitmap
// over the slice's ids, 2 B rank prefix per bitmap word, 2 B entries for up
// to 2048 distinct ids][allowed-id mask words][staged chunks].
// g / nslices for block and row indices (a 32-bit reciprocal; one slice per
// row divides by 1, which the reciprocal cannot express)
__device__ __forceinline__ int div_slices(int g, const StreamArgs& a) {
    return a.nslices == 1 ? g : (int)__umulhi((uint32_t)g, a.ns_magic);
}

template <int DT, bool VEC, bool PEN, bool MASK, bool GR, int EX = 0, bool LEAN = false>
__global__ __launch_bounds__(kBlock, EX >= 2 ? 4 : 5) void k_stream(StreamArgs a) {
    using T = Tile<DT>;
    constexpr int NT = EX > 1 ? EX : 1;        // tiles per slice (exact lists: 1 or 2)
    constexpr int NC = T::NCH * NT;            // chunks per thread
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Shared st;
    const int tid = threadIdx.x;
    uint32_t bid = blockIdx.x;
    if constexpr (EX) {
        // the launch arguments the first loads need, in registers together:
        // one round of scalar loads instead of one per branch that uses them
        // (an asm statement that reads them; it touches no memory)
        __asm__("" : "+s"(bid)
                : "s"(a.logits), "s"(a.logits_stride), "s"(a.hist), "s"(a.hist_stride), "s"(a.mask),
                  "s"(a.mask_stride), "s"(a.plans), "s"(a.rows), "s"(a.vocab), "s"(a.nslices), "s"(a.slice_len),
                  "s"(a.bitmap_words), "s"(a.blocks_per_xcd), "s"(a.ns_magic), "s"(a.vec_tail), "s"(a.hist_direct));
    }
    const int logical = (int)(bid % kXcds) * a.blocks_per_xcd + (int)(bid / kXcds);
    const int r = div_slices(logical, a), s = logical - r * a.nslices;
    if (r >= a.rows) return;
    const int lo = s * a.slice_len;
    const int hi = min(a.vocab - (VEC ? a.vec_tail : 0), lo + a.slice_len);   // k_merge takes the ragged end
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * T::ES;
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(rowp, hi, T::ES);
    // When every row of the launch is this kernel's, the first tile goes out
    // before the plan is read (it is processed chunk by chunk as its loads
    // complete in order); otherwise after the plan has said the row is ours.
    const bool early = EX || ((a.uniform >> (GR ? 0 : 1)) & 1) != 0;
    uint4 raw[NC];
    // Exact lists: the history row, the slice's mask words and the tile go out
    // first (their addresses come from the launch arguments alone) and the
    // plan's scalar load after them: a wait for the plan placed ahead of the
    // tile's loads would hold the whole slice back by one memory round trip.
    RowPlan P;
    // exact lists with short history rows: the whole row goes out first
    int32_t pre[8];
    const bool hd = EX && PEN && a.hist_direct != 0;
    if (hd) {
        // one buffer resource over the row: positions past hist_stride read 0
        const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(a.hist + (int64_t)r * a.hist_stride), (short)0, (int)a.hist_stride * 4, 0x00020000);
#pragma unroll
        for (int q = 0; q < 8; ++q) pre[q] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(hr, tid * 4, q * kBlock * 4, 0);
    }
    if constexpr (EX && PEN) {
        if (!hd) {
            // longer history rows: the window's place comes from the plan,
            // which then goes first (the tile waits one round trip); the
            // window still goes out ahead of the tile, as the short rows do
            P = plan_of(a, r);
            const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
            const int32_t* hrow = a.hist + (int64_t)r * a.hist_stride;
#pragma unroll
            for (int q = 0; q < 8; ++q) pre[q] = -1;
            if ((P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0 && L > 0) {
#pragma unroll
                for (int q = 0; q < 8; ++q) pre[q] = hrow[max(0, min(p0 + q * kBlock + tid, L - 1))];
            }
        }
    }
    // (MASK launches may carry no mask: the general instantiations for
    // unaligned rows take MASK = true; the mask words are then all ones)
    const bool mk = MASK && a.mask != nullptr;
    uint32_t mw_pre[NT];
#pragma unroll
    for (int q = 0; q < NT; ++q) {
        const int w = tid + q * kBlock;
        mw_pre[q] = 0xFFFFFFFFu;
        if (EX && mk && w < a.bitmap_words)
            mw_pre[q] = (lo + 32 * w < hi) ? a.mask[(int64_t)r * a.mask_stride + (lo >> 5) + w] : 0u;
    }
    if (early) load_tile<DT, VEC, NC>(rs, lo, raw);
    if (EX) __builtin_amdgcn_sched_barrier(0);
    if (!(EX && PEN) || hd) P = plan_of(a, r);
    if (!early) {
        if (P.flags & RF_FULL) return;                     // k_full's row
        if (((P.flags & RF_GREEDY) != 0) != GR) return;    // the other kernel's row
    }
    // (flag mode: sampling rows stream without penalty marks -- k_merge finds
    // their penalised ids -- also in the instantiations for unaligned rows,
    // which take PEN = true for every batch)
    const bool pen = PEN && (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0 && (GR || EX || !a.pen_flag);
    const bool masked = MASK && (P.flags & RF_MASK) != 0;

    // The history window goes out next (before the first tile when that has
    // not gone yet). Branch-free: clamped loads (pre[q] holds position
    // p0 + q * kBlock + tid, used only below L), so nothing here waits.
    const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
    const int32_t* hrow = a.hist + (int64_t)r * a.hist_stride;
    if (!EX) {
#pragma unroll
        for (int q = 0; q < 8; ++q) pre[q] = -1;
    }
    if (!EX && PEN && pen && L > 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) pre[q] = hrow[max(0, min(p0 + q * kBlock + tid, L - 1))];
    }
    uint32_t* pbm = reinterpret_cast<uint32_t*>(smem);
    if constexpr (EX) {
        HSAMP_PHASE(logical, 0);
        if (PEN) {
            for (int i = tid; i < (a.mbm_off >> 2); i += kBlock) reinterpret_cast<uint4*>(smem)[i] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int q = 0; q < NT; ++q)
            if (MASK && tid + q * kBlock < a.bitmap_words) pbm[a.mbm_off + tid + q * kBlock] = mw_pre[q];
        if (tid == 0) {
            st.n = 0;
            st.nst = 0;
            st.flags = 0;
        }
        __syncthreads();
        HSAMP_PHASE(logical, 1);
        const int64_t slot = (int64_t)r * a.nslices + s;
        u64* out = a.cand + slot * a.cand_cap;
        stream_exact<DT, VEC, PEN, MASK, NC, LEAN>(a, P, r, lo, hi, raw, out, slot, VEC && s == a.nslices - 1, pen,
                                                   mk, pre, hd ? 0 : p0, smem, st);
    } else {
        stream_setup<PEN, MASK>(a, P, r, lo, hi, GR, pen, masked, p0, L, hrow, pbm, pbm + a.bitmap_words, st);
        if (!early) load_tile<DT, VEC>(rs, lo, raw);
        if (PEN) {
            // the history window (waits for pre[] only when the tile was requested after)
            if (pen) {
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (p0 + q * kBlock + tid < L) stream_mark(pre[q], lo, hi, pbm);
            }
            __syncthreads();
        }
        const int64_t slot = (int64_t)r * a.nslices + s;
        u64* out = a.cand + slot * a.cand_cap;
        if constexpr (GR) stream_greedy<DT, VEC, PEN, MASK>(a, P, r, lo, hi, rs, raw, out, slot, smem, st);
        else stream_sample<DT, VEC, PEN, MASK>(a, P, r, lo, hi, rs, raw, out, slot, smem, st);
    }
}

// ---- the merge kernel ------------------------------------------------------------

// The row's penalty table: every id of the history window with its counts
// (repetition flag, DRY count, frequency/presence count) and its bias flag.
// The first 8 * 256 history entries are loaded before the table is cleared.
__device__ __forceinline__ void pen_add(const StreamArgs& a, const RowPlan& P, int L, int p, int32_t t,
                                        PenaltyLds pl) {
    if (t < 0 || t >= a.vocab) return;
    uint32_t add = 0u, orv = 0u;
    if (p >= L - P.rep_win) orv |= HV_REP;
    if (p >= L - P.dry_win) add += 1u << HV_DRY_SHIFT;
    if (p >= L - P.fp_win) add += 1u;
    const uint32_t sl = pen_insert(t, pl);
    if (add) atomicAdd(&pl.hval[sl], add);
    if (orv) atomicOr(&pl.hval[sl], orv);
}

// The first 8 * 256 entries of the row's history window, loaded early.
__device__ __forceinline__ void hist_prefetch(const StreamArgs& a, const RowPlan& P, int r, bool pen,
                                              int32_t (&pre)[8]) {
    const int L = hist_len_of(a, P, r);
    const int p0 = L - P.scan_len;
    const int32_t* h = a.hist + (int64_t)r * a.hist_stride;
    // (clamped positions, no branch around a load: the eight stay in flight)
#pragma unroll
    for (int q = 0; q < 8; ++q) pre[q] = -1;
    if (pen && L > 0) {
        int32_t v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = h[max(0, min(p0 + q * kBlock + (int)threadIdx.x, L - 1))];
#pragma unroll
        for (int q = 0; q < 8; ++q) pre[q] = (p0 + q * kBlock + (int)threadIdx.x < L) ? v[q] : -1;
    }
}

__device__ __forceinline__ void pen_build_row(const StreamArgs& a, const RowPlan& P, int r, PenaltyLds pl,
                                              const int32_t (&pre)[8]) {
    const int tid = threadIdx.x;
    const int L = hist_len_of(a, P, r);
    const int p0 = L - P.scan_len;
    const int32_t* h = a.hist + (int64_t)r * a.hist_stride;
    for (int i = tid; i < a.mhash_slots; i += kBlock) {
        pl.hkey[i] = kEmpty;
        pl.hval[i] = 0u;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) pen_add(a, P, L, p0 + q * kBlock + tid, pre[q], pl);
    for (int p = p0 + 8 * kBlock + tid; p < L; p += kBlock) pen_add(a, P, L, p, h[p], pl);
    if (P.flags & RF_BIAS) {
        for (int j = tid; j < P.bias_cnt; j += kBlock) {
            const uint32_t sl = pen_insert(a.bias_ids[P.bias_off + j], pl);
            atomicOr(&pl.hval[sl], HV_BIAS);
        }
    }
    __syncthreads();
}

// Offer NM register-held composites c[i] (0 = none) to the buffer: the
// batch bounds the row's k-th largest from below (each wave's kw-th largest
// lane maximum, kw = ceil(k/4), minimum over the waves), the bound raises the
// threshold, and the survivors are appended.
template <int NM>
__device__ __forceinline__ void offer_regs(u64* buf, u64* ovf, int cap, int k, const u64 (&c)[NM], Shared& st) {
    const int tid = threadIdx.x;
    const int kw = (k + 3) >> 2;
    uint32_t kv[NM];
    int32_t id[NM];
    uint32_t g = 0u;
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        kv[i] = (uint32_t)(c[i] >> 32);
        id[i] = comp_idx(c[i]);
        g = max(g, kv[i]);
    }
    const uint32_t gk[4] = {g, 0u, 0u, 0u};
    const uint32_t tw = (kw <= 64) ? wave_kth_largest(gk, 1, kw) : 0u;
    if (lane_id() == 0) st.twave[wave_id()] = tw;
    __syncthreads();
    {
        uint32_t tt = st.twave[0];
#pragma unroll
        for (int i = 1; i < kBlock / 64; ++i) tt = min(tt, st.twave[i]);
        const u64 tl = (u64)tt << 32;
        __syncthreads();
        if (tid == 0 && tl > st.theta) st.theta = tl;
        __syncthreads();
    }
    append_regs<NM>(buf, cap, kv, [&](int i) { return id[i]; }, ovf, st);
    drain_overflow(buf, cap, k, ovf, st);
}

// A row's last ids that the stream's whole-chunk loads leave out, and that
// are not penalised: mask, (temperature), NaN handling and key as in
// tile_keys; 0 = no candidate (greedy NaN).
__device__ __forceinline__ u64 tail_candidate(float x, bool allowed, int32_t t, bool greedy, float inv_t,
                                              Shared& st) {
    if (!allowed) x = -__builtin_inff();
    if (!greedy) x = x * inv_t;
    if (x != x) {
        atomicOr(&st.flags, 4);
        if (greedy) return 0ull;
        x = -__builtin_inff();
    }
    return comp(key32(x), t);
}

// The merge of one row when k <= 64, the history window holds at most 8 * 256
// ids, at most 256 bias entries, and the penalty table fits LDS next to a
// 2048-bin histogram. LDS: [bins 8 KB][list 1 KB][table: keys, 64-bit counts].
//  - Penalty table: each thread inserts its (up to) 8 history ids and 1 bias
//    id with all first probes in flight together; the thread whose insert
//    claims a slot owns the id, reads its logit at once and, after one
//    64-bit add per history entry (frequency/presence, DRY and repetition
//    counts in 16-bit fields), runs stages 1-6 for it.
//  - Selection over the 9 + NW register candidates per thread: a lower bound
//    L on the k-th largest key (each wave's kw-th largest lane maximum, low
//    16 bits cleared, minimum over waves) and the maximum M fix the bits all
//    top-k keys share; a 2048-bin histogram of the next 11 bits finds the bin
//    holding the k-th; entries at or above it (< 128) are ranked exactly by
//    wave 0. More entries (massive ties) or list entries beyond the windows
//    take the buffer path.
template <int NW, bool LM>
__device__ __forceinline__ void merge_fast(const StreamArgs& a, const RowPlan& P, int r, const int32_t (&pre)[8],
                                           int32_t bias_t, int32_t bias_h, bool nan_at0, int32_t tail_t, float tail_x,
                                           bool tail_ok, double ur,
                                           u64 (&win)[NW], unsigned char* smem, Shared& st, const StreamArgs& sa,
                                           const RowPlan& sP) {
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const bool greedy = (P.flags & RF_GREEDY) != 0;
    const bool pen = (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;
    const bool masked = (P.flags & RF_MASK) != 0;
    const int k = P.top_k;
    const int S = a.nslices, W = a.win;
    const int fs = a.mhash_slots;
    uint32_t* bins = reinterpret_cast<uint32_t*>(smem);
    u64* list = reinterpret_cast<u64*>(smem + 8192);
    uint32_t* tkey = reinterpret_cast<uint32_t*>(smem + 9216);
    u64* tval = reinterpret_cast<u64*>(smem + 9216 + 4 * fs);
    const uint32_t hmask = (uint32_t)fs - 1u, hshift = 32u - (uint32_t)__popc(hmask);
    // flag mode (penalties only lower logits): the stream handed penalised ids
    // over flagged; their true values are found for just those ids, from
    // counters of the history's ids, without a table.
    // LDS there: [bins][list][counters: 64 bits per distinct history id]
    // [vocabulary bitmap: 16 B per 128 ids][rank prefixes: 2 B per 128 ids],
    // all after the list replaced by the buffer once the values are found
    constexpr bool lmode = LM;   // flag mode (a launch-level choice: its own instantiation)
    u64* cnt = reinterpret_cast<u64*>(smem + 9216);
    uint4* vb4 = reinterpret_cast<uint4*>(smem + 9216 + 8 * kCntCap);
    if (pen && !lmode) {
        for (int i = tid; i < fs; i += kBlock) {
            tkey[i] = kEmpty;
            tval[i] = 0ull;
        }
    }
    if (lmode && pen) {
        for (int i = tid; i < kCntCap; i += kBlock) cnt[i] = 0ull;
        for (int i = tid; i < ((a.vocab + 127) >> 7); i += kBlock) vb4[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    for (int i = tid; i < 2048; i += kBlock) bins[i] = 0u;
    __syncthreads();   // also publishes the slice counts

    // Flag mode, before anything waits for the lists: counters of the
    // history's ids. A bitmap over the vocabulary marks the ids, and an id's
    // rank among them (prefix popcounts per 128 ids) indexes its counters.
    const int ng = (a.vocab + 127) >> 7;
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(vb4 + ng);
    if (lmode && pen) {
        uint32_t* vb = reinterpret_cast<uint32_t*>(vb4);
        uint16_t* vpw = reinterpret_cast<uint16_t*>(vb4 + ng);
        const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int p = p0 + q * kBlock + tid;
            if (p >= 0 && p < L && pre[q] >= 0 && pre[q] < a.vocab) atomicOr(&vb[pre[q] >> 5], 1u << (pre[q] & 31));
        }
        if (bias_h >= 0 && bias_h < a.vocab) atomicOr(&vb[bias_h >> 5], 1u << (bias_h & 31));   // zero counts
        __syncthreads();
        {
            const int per = (ng + kBlock - 1) / kBlock;
            const int g0 = min(ng, tid * per), g1 = min(ng, g0 + per);
            constexpr int GM = 8;   // groups per thread read at once (V <= 262144)
            if (per <= GM) {
                int pc[GM], sum = 0;
#pragma unroll
                for (int i = 0; i < GM; ++i) {
                    const uint4 w = vb4[min(g0 + i, ng - 1)];
                    pc[i] = (g0 + i < g1) ? __popc(w.x) + __popc(w.y) + __popc(w.z) + __popc(w.w) : 0;
                    sum += pc[i];
                }
                int tot;
                int run = block_excl_scan(sum, &tot, st);
#pragma unroll
                for (int i = 0; i < GM; ++i) {
                    if (g0 + i < g1) vpw[g0 + i] = (uint16_t)run;
                    run += pc[i];
                }
            } else {
                int sum = 0;
                for (int g = g0; g < g1; ++g) {
                    const uint4 w = vb4[g];
                    sum += __popc(w.x) + __popc(w.y) + __popc(w.z) + __popc(w.w);
                }
                int tot;
                int run = block_excl_scan(sum, &tot, st);
                for (int g = g0; g < g1; ++g) {
                    const uint4 w = vb4[g];
                    vpw[g] = (uint16_t)run;
                    run += __popc(w.x) + __popc(w.y) + __popc(w.z) + __popc(w.w);
                }
            }
        }
        __syncthreads();
    }
    // rank of id t among the marked ids, or -1 when t is not marked; every
    // word of the 16-byte group enters arithmetically, so the read stays one
    // unconditional 16-byte load
    auto rank = [&](int t) -> int {
        const uint4 w = vb4[t >> 7];
        const int wi = (t >> 5) & 3;
        const uint32_t s0 = 0u - (uint32_t)(wi == 0), s1 = 0u - (uint32_t)(wi == 1);
        const uint32_t s2 = 0u - (uint32_t)(wi == 2), s3 = 0u - (uint32_t)(wi == 3);
        const uint32_t wt = (w.x & s0) | (w.y & s1) | (w.z & s2) | (w.w & s3);
        const uint32_t b1 = 0u - (uint32_t)(wi > 0), b2 = 0u - (uint32_t)(wi > 1), b3 = 0u - (uint32_t)(wi > 2);
        const int rk = (int)vp[t >> 7] + __popc(w.x & b1) + __popc(w.y & b2) + __popc(w.z & b3) +
                       __popc(wt & ((1u << (t & 31)) - 1u));
        return ((wt >> (t & 31)) & 1u) ? rk : -1;
    };
    if (lmode && pen) {
        // every rank read first, then the adds (no wait inside a branch)
        const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
        int rkq[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int p = p0 + q * kBlock + tid;
            const bool ok = p >= 0 && p < L && pre[q] >= 0 && pre[q] < a.vocab;
            const int rk = rank(ok ? pre[q] : 0);
            rkq[q] = ok ? rk : -1;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int p = p0 + q * kBlock + tid;
            const u64 add = ((p >= L - P.fp_win) ? 1ull : 0ull) | ((p >= L - P.dry_win) ? (1ull << 16) : 0ull) |
                            ((p >= L - P.rep_win) ? (1ull << 32) : 0ull);
            if (rkq[q] >= 0) atomicAdd(&cnt[rkq[q]], add);
        }
        __syncthreads();
    }

    // ---- penalised ids ------------------------------------------------------------
    u64 cp[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) cp[q] = 0ull;
    if (pen && !lmode) {
        const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
        int32_t t[9];
        uint32_t sl[9];
#pragma unroll
        for (int q = 0; q < 8; ++q) t[q] = (pre[q] >= 0 && pre[q] < a.vocab) ? pre[q] : -1;
        t[8] = bias_t;
        // every thread reads the logits of its ids at once (ownership is
        // settled below); the loads overlap the table work
        const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
        float x[9];
        uint32_t mw[9];
        load_logits<9>(rowp, a.dtype, t, x);
#pragma unroll
        for (int q = 0; q < 9; ++q)
            mw[q] = (masked && t[q] >= 0) ? a.mask[(int64_t)r * a.mask_stride + (t[q] >> 5)] : 0xFFFFFFFFu;
        // Insert: probing runs over groups of 4 slots from the group the hash
        // names; an id sits in the first group on its way that had room, so a
        // lookup scans groups until it finds the id or an empty slot. Each
        // round reads every pending entry's group with one 16-byte load and
        // claims an empty slot with one CAS; both sets of operations go out
        // together, and entries with nothing to do repeat a harmless read and
        // a CAS that cannot succeed instead of branching.
        uint32_t pend = 0u, own = 0u;
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            sl[q] = (((uint32_t)t[q] * 0x9E3779B1u) >> hshift) & ~3u;
            if (t[q] >= 0) pend |= 1u << q;
        }
        while (pend != 0u) {
            uint4 g[9];
#pragma unroll
            for (int q = 0; q < 9; ++q) g[q] = *reinterpret_cast<const uint4*>(&tkey[sl[q] & ~3u]);
            uint32_t tryc = 0u, cs[9];
#pragma unroll
            for (int q = 0; q < 9; ++q) {
                cs[q] = sl[q] & ~3u;
                if (!((pend >> q) & 1u)) continue;
                const uint32_t tk = (uint32_t)t[q];
                const uint32_t k4[4] = {g[q].x, g[q].y, g[q].z, g[q].w};
                // the empty slot is taken from a point that depends on the id,
                // so that ids meeting in one group seldom race for one slot
                const int rot = (int)((tk * 0x9E3779B1u) >> 8) & 3;
                int hit = -1, emp = -1;
#pragma unroll
                for (int c = 3; c >= 0; --c) {
                    const int cc = (c + rot) & 3;
                    hit = (k4[c] == tk) ? c : hit;
                    emp = (k4[cc] == kEmpty) ? cc : emp;
                }
                if (hit >= 0) {                  // already in: a count goes to its slot
                    sl[q] = cs[q] + (uint32_t)hit;
                    pend &= ~(1u << q);
                } else if (emp >= 0) {
                    cs[q] += (uint32_t)emp;
                    tryc |= 1u << q;
                } else {
                    sl[q] = (cs[q] + 4u) & hmask;  // group full: the next one
                }
            }
            // entries not trying a slot this round aim their CAS at this lane's
            // own word of the (still unused) histogram, which never holds kEmpty
            uint32_t old[9];
#pragma unroll
            for (int q = 0; q < 9; ++q) {
                uint32_t* at = ((tryc >> q) & 1u) ? &tkey[cs[q]] : &bins[tid];
                old[q] = atomicCAS(at, kEmpty, (uint32_t)t[q]);
            }
#pragma unroll
            for (int q = 0; q < 9; ++q) {
                if (!((tryc >> q) & 1u)) continue;
                if (old[q] == kEmpty) {
                    own |= 1u << q;
                    sl[q] = cs[q];
                    pend &= ~(1u << q);
                } else if (old[q] == (uint32_t)t[q]) {
                    sl[q] = cs[q];
                    pend &= ~(1u << q);
                }                                  // else: lost the slot, read the group again
            }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (t[q] < 0) continue;
            const int p = p0 + q * kBlock + tid;
            const u64 add = ((p >= L - P.fp_win) ? 1ull : 0ull) | ((p >= L - P.dry_win) ? (1ull << 16) : 0ull) |
                            ((p >= L - P.rep_win) ? (1ull << 32) : 0ull);
            if (add) atomicAdd(&tval[sl[q]], add);
        }
        if (t[8] >= 0) atomicAdd(&tval[sl[8]], 1ull << 63);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            if (!((own >> q) & 1u)) continue;
            const u64 c = tval[sl[q]];
            const uint32_t v = ((c >> 32) & 0xFFFFull ? HV_REP : 0u) | ((c >> 63) ? HV_BIAS : 0u) |
                               ((uint32_t)((c >> 16) & 0xFFFFull) << HV_DRY_SHIFT) | (uint32_t)(c & 0xFFFFull);
            float y = ((mw[q] >> (t[q] & 31)) & 1u) ? x[q] : -__builtin_inff();
            y = pen_value(y, t[q], v, a, P);
            if (greedy) {
                if (y != y) {
                    atomicOr(&st.flags, 4);
                    if (t[q] == 0) atomicOr(&st.nan0, 1);
                    continue;
                }
            } else {
                if (P.flags & RF_TEMP) y = y * P.inv_temp;
                if (y != y) {
                    atomicOr(&st.flags, 4);
                    y = -__builtin_inff();
                }
            }
            cp[q] = comp(key32(y), t[q]);
        }
    }

    // the ragged end, unless penalised
    auto in_table = [&](int32_t t) -> bool {
        uint32_t s0 = (((uint32_t)t * 0x9E3779B1u) >> hshift) & ~3u;
        for (;;) {
            const uint32_t kk = tkey[s0];
            if (kk == (uint32_t)t || kk == kEmpty) return kk == (uint32_t)t;
            s0 = (s0 + 1u) & hmask;
        }
    };
    u64 ct = 0ull;
    if (!lmode && tail_t >= 0 && !(pen && in_table(tail_t)))
        ct = tail_candidate(tail_x, tail_ok, tail_t, greedy, P.inv_temp, st);

    // ---- the slices' lists ----------------------------------------------------------
    int extra = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int g = tid + j * kBlock;
        const int s2 = (int)__umulhi((uint32_t)g, a.win_magic);   // g / W
        if (s2 >= S || g - s2 * W >= st.soff[s2]) win[j] = 0ull;
    }
    extra = (st.flags & 8) ? 1 : 0;   // some slice's list runs past the window

    // the true value of id t (raw logit x, allowed by the mask or not,
    // history counters c) as a composite; 0 (absent) for a greedy row's NaN
    auto value = [&](int32_t t, float x, bool allowed, u64 c) -> u64 {
        uint32_t v = ((c >> 32) & 0xFFFFull ? HV_REP : 0u) | ((uint32_t)((c >> 16) & 0xFFFFull) << HV_DRY_SHIFT) |
                     (uint32_t)(c & 0xFFFFull);
        if (P.flags & RF_BIAS) {
            int lo = 0, hi = P.bias_cnt;
            const int32_t* ids = a.bias_ids + P.bias_off;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (ids[mid] < t) lo = mid + 1;
                else hi = mid;
            }
            if (lo < P.bias_cnt && ids[lo] == t) v |= HV_BIAS;
        }
        float y = allowed ? x : -__builtin_inff();
        y = pen_value(y, t, v, a, P);
        if (!greedy) y = y * P.inv_temp;
        if (y != y) {
            atomicOr(&st.flags, 4);
            return greedy ? 0ull : comp(kKeyNegInf, t);
        }
        return comp(key32(y), t);
    };
    if (lmode && !greedy) {
        // Flag mode, sampling rows: the stream handed over raw keys (key32 of
        // the masked logit, NaN as -inf), so each candidate's logit is its
        // key's float, exactly. Penalised ids (in the history or the bias
        // list: rank >= 0) take stages 1-6 (sampler.cpp:235-264) with their
        // counters, then every candidate takes the temperature (sampler.cpp:
        // 101-106). Batched: every rank, then every counter, then the values.
        int rk[NW];
        u64 cj[NW];
        if (pen) {
#pragma unroll
            for (int j = 0; j < NW; ++j) {
                const int rj = rank(win[j] != 0ull ? (int)comp_idx(win[j]) : 0);
                rk[j] = win[j] != 0ull ? rj : -1;
            }
#pragma unroll
            for (int j = 0; j < NW; ++j) cj[j] = rk[j] >= 0 ? cnt[rk[j]] : 0ull;
        }
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            if (win[j] == 0ull) continue;
            const int32_t t = (int32_t)comp_idx(win[j]);
            float y = key_to_float((uint32_t)(win[j] >> 32));
            if (pen && rk[j] >= 0) {
                const u64 c = cj[j];
                uint32_t v = ((c >> 32) & 0xFFFFull ? HV_REP : 0u) |
                             ((uint32_t)((c >> 16) & 0xFFFFull) << HV_DRY_SHIFT) | (uint32_t)(c & 0xFFFFull);
                if (P.flags & RF_BIAS) {
                    int lo = 0, hi = P.bias_cnt;
                    const int32_t* ids = a.bias_ids + P.bias_off;
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (ids[mid] < t) lo = mid + 1;
                        else hi = mid;
                    }
                    if (lo < P.bias_cnt && ids[lo] == t) v |= HV_BIAS;
                }
                y = pen_value(y, t, v, a, P);
            }
            y = y * P.inv_temp;
            if (y != y) {
                atomicOr(&st.flags, 4);
                y = -__builtin_inff();
            }
            win[j] = comp(key32(y), t);
        }
        if (tail_t >= 0) {
            const int rk0 = pen ? rank(tail_t) : -1;
            ct = value(tail_t, tail_x, tail_ok, rk0 >= 0 ? cnt[rk0] : 0ull);
        }
    } else if (lmode) {
        // Flag mode, greedy rows: the flagged entries (key kKeyFlag) and the
        // ragged end get their true values in place, from the row's raw
        // logits and their ids' counters.
        const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
        int32_t ft[NW];
#pragma unroll
        for (int j = 0; j < NW; ++j) ft[j] = ((uint32_t)(win[j] >> 32) == kKeyFlag) ? (int32_t)comp_idx(win[j]) : -1;
        float xr[NW];
        load_logits<NW>(rowp, a.dtype, ft, xr);
        uint32_t mwf[NW];
#pragma unroll
        for (int j = 0; j < NW; ++j)
            mwf[j] = (masked && ft[j] >= 0) ? a.mask[(int64_t)r * a.mask_stride + (ft[j] >> 5)] : 0xFFFFFFFFu;
        u64 cj[NW];
        if (pen) {
            int rk[NW];
#pragma unroll
            for (int j = 0; j < NW; ++j) rk[j] = ft[j] >= 0 ? rank(ft[j]) : -1;
#pragma unroll
            for (int j = 0; j < NW; ++j) cj[j] = rk[j] >= 0 ? cnt[rk[j]] : 0ull;
        }
#pragma unroll
        for (int j = 0; j < NW; ++j)
            if (ft[j] >= 0) win[j] = value(ft[j], xr[j], (mwf[j] >> (ft[j] & 31)) & 1u, pen ? cj[j] : 0ull);
        if (tail_t >= 0) {
            const int rk = pen ? rank(tail_t) : -1;
            ct = value(tail_t, tail_x, tail_ok, rk >= 0 ? cnt[rk] : 0ull);
        }
    }

    if (tid == 0) st.u = ur;
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
    // flag mode: the true value of list entry c (flagged, or any entry of a
    // sampling row whose id is penalised), read from the row
    auto resolve = [&](u64 c) -> u64 {
        if (c == 0ull) return 0ull;
        const int32_t t = (int32_t)comp_idx(c);
        const bool flagged = (uint32_t)(c >> 32) == kKeyFlag;
        const int rk = pen ? rank(t) : -1;
        if (!flagged && rk < 0) return c;
        const float x = load_logit_dt(rowp, a.dtype, t);
        const bool allowed = !masked || ((a.mask[(int64_t)r * a.mask_stride + (t >> 5)] >> (t & 31)) & 1u);
        return value(t, x, allowed, rk >= 0 ? cnt[rk] : 0ull);
    };

    if (greedy) {
        u64 best = ct;
#pragma unroll
        for (int q = 0; q < 9; ++q) best = cp[q] > best ? cp[q] : best;
#pragma unroll
        for (int j = 0; j < NW; ++j) best = win[j] > best ? win[j] : best;
        if (lmode && extra != 0) {
            // flagged entries past a slice's window (rare)
            const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
            for (int s2 = 0; s2 < S; ++s2) {
                const int n = st.soff[s2];
                for (int e = W + tid; e < n; e += kBlock) {
                    const u64 c = resolve(cand[(int64_t)s2 * a.cand_cap + e]);
                    best = c > best ? c : best;
                }
            }
        }
        best = block_max_u64(best, st);
        __syncthreads();
        int32_t gtok = 0;
        if (tid == 0) {
            // argmax returns 0 when id 0 holds a NaN: a penalised id 0 was
            // settled with the table, any other by its logit
            const bool pen0 = pen && !lmode && in_table(0);
            const bool nan0 = pen0 ? st.nan0 != 0 : nan_at0;
            gtok = nan0 ? 0 : comp_idx(best);
            if (a.row_flags != nullptr) a.row_flags[r] = ROWF_GREEDY | ((st.flags & 4) ? ROWF_NAN : 0u);
            if (a.topk_count != nullptr) a.topk_count[r] = -1;
            if (a.kept_count != nullptr) a.kept_count[r] = 0;
        }
        if (wave_id() == 0) emit_token_wave(a, r, gtok);
        return;
    }

    // ---- exact top-k ----------------------------------------------------------------
    constexpr int NC = 10 + NW;
    const uint32_t floor_key = (uint32_t)(kThetaFloor >> 32);
    uint32_t lmax = (uint32_t)(ct >> 32);
#pragma unroll
    for (int q = 0; q < 9; ++q) lmax = max(lmax, (uint32_t)(cp[q] >> 32));
#pragma unroll
    for (int j = 0; j < NW; ++j) lmax = max(lmax, (uint32_t)(win[j] >> 32));
    const int kw = (k + 3) >> 2;
    const uint32_t g4[4] = {lmax, 0u, 0u, 0u};
    const uint32_t tw = wave_kth_bound16(g4, 1, kw);
    uint32_t wm = lmax;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) wm = max(wm, (uint32_t)__shfl_xor((int)wm, d, 64));
    if (lane == 0) {
        st.twave[wave_id()] = tw;
        st.minv_w[wave_id()] = wm;
    }
    __syncthreads();
    uint32_t Lk = st.twave[0], Mk = (uint32_t)st.minv_w[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) {
        Lk = min(Lk, st.twave[i]);
        Mk = max(Mk, (uint32_t)st.minv_w[i]);
    }
    Lk = max(Lk, floor_key);
    const int hb = (Mk > Lk) ? 31 - __clz((int)(Lk ^ Mk)) : 0;
    const int shift = max(0, hb - 10);
    auto binof = [&](uint32_t key) -> uint32_t { return (key >> shift) & 2047u; };
    const bool any = Mk >= Lk;
    if (any) {
        if ((uint32_t)(ct >> 32) >= Lk) atomicAdd(&bins[binof((uint32_t)(ct >> 32))], 1u);
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            const uint32_t key = (uint32_t)(cp[q] >> 32);
            if (key >= Lk) atomicAdd(&bins[binof(key)], 1u);
        }
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const uint32_t key = (uint32_t)(win[j] >> 32);
            if (key >= Lk) atomicAdd(&bins[binof(key)], 1u);
        }
    }
    __syncthreads();
    // the bin holding the k-th largest, counting down from the top bin
    {
        const uint4 lo4 = reinterpret_cast<const uint4*>(bins)[(2047 - 8 * tid - 7) >> 2];
        const uint4 hi4 = reinterpret_cast<const uint4*>(bins)[(2047 - 8 * tid - 3) >> 2];
        const uint32_t c8[8] = {hi4.w, hi4.z, hi4.y, hi4.x, lo4.w, lo4.z, lo4.y, lo4.x};   // bins 2047-8t downwards
        int sum8 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) sum8 += (int)c8[i];
        int total;
        const int excl = block_excl_scan(sum8, &total, st);
        if (tid == 0) {
            st.sel_d = -1;         // fewer than k entries: all of them
            st.sel_need = total;
        }
        __syncthreads();
        if (excl < k && excl + sum8 >= k) {
            int cum = excl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (cum + (int)c8[i] >= k) {
                    st.sel_d = 2047 - 8 * tid - i;
                    st.sel_need = cum + (int)c8[i];   // entries at or above the bin
                    break;
                }
                cum += (int)c8[i];
            }
        }
        __syncthreads();
    }
    const int bstar = st.sel_d;
    const int nlist = st.sel_need;
    if (lmode) {
        // Sampling rows streamed on raw keys without penalties: every id a
        // slice left out has a raw key below that slice's bound, so its true
        // key (penalties only lower a logit, the temperature keeps the order)
        // is at most the bound's scaled key. The candidates hold the exact
        // top-k when its k-th key lies above the largest scaled bound (checked
        // against the lower edge of the k-th's bin). Otherwise, or when lists
        // ran past their windows (entries not yet resolved), the whole row is
        // read again (rare).
        const uint32_t th = st.thmax;
        bool ok = th <= floor_key;
        if (!ok && any && bstar >= 0) {
            const uint32_t ths = key32(key_to_float(th) * P.inv_temp);
            const uint32_t top = (shift + 11 >= 32) ? 0u : (Mk & ~((1u << (shift + 11)) - 1u));
            ok = (top | ((uint32_t)bstar << shift)) > ths;
        }
        if (!ok || extra != 0) {
            u64* rbuf = reinterpret_cast<u64*>(smem + 9216 + 8 * kCntCap + ((18 * ng + 15) & ~15));
            u64* ovf = a.ovf + (int64_t)r * a.ovf_cap;
            __syncthreads();
            if (tid == 0) {
                st.n = 0;
                st.theta = kThetaFloor;
            }
            __syncthreads();
            for (int base = 0; base < a.vocab; base += 8 * kBlock) {
                int32_t t[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) t[q] = (base + q * kBlock + tid < a.vocab) ? base + q * kBlock + tid : -1;
                float x[8];
                load_logits<8>(rowp, a.dtype, t, x);
                u64 c[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    c[q] = 0ull;
                    if (t[q] < 0) continue;
                    const bool allowed =
                        !masked || ((a.mask[(int64_t)r * a.mask_stride + (t[q] >> 5)] >> (t[q] & 31)) & 1u);
                    const int rk = pen ? rank(t[q]) : -1;
                    c[q] = value(t[q], x[q], allowed, rk >= 0 ? cnt[rk] : 0ull);
                }
                offer_regs<8>(rbuf, ovf, a.buf_cap, k, c, st);
            }
            __syncthreads();
            const uint32_t rflags = ((st.flags & 4) ? ROWF_NAN : 0u) | ROWF_REREAD;
            FinLds f{};
            select_and_finalize(sa, sP, r, rbuf, f, st, rflags);
            return;
        }
    }
    if (nlist < 128 && extra == 0) {
        // entries at or above the k-th's bin, then an exact rank by wave 0
        uint32_t inm = 0u;   // which of this thread's NC candidates go to the list
#pragma unroll
        for (int q = 0; q < NC; ++q) {
            const u64 c = (q < 9) ? cp[q] : (q == 9 ? ct : win[q - 10 < 0 ? 0 : q - 10]);
            const uint32_t key = (uint32_t)(c >> 32);
            inm |= (any && key >= Lk && (int)binof(key) >= bstar) ? (1u << q) : 0u;
        }
        if (__ballot(inm != 0u) != 0ull) {
            const int cnt = __popc(inm);
            int incl = cnt;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(incl, d, 64);
                if (lane >= d) incl += y;
            }
            int base = 0;
            if (lane == 63) base = atomicAdd(&st.n, incl);
            int pos = __shfl(base, 63, 64) + incl - cnt;
#pragma unroll
            for (int q = 0; q < NC; ++q)
                if ((inm >> q) & 1u) list[pos++] = (q < 9) ? cp[q] : (q == 9 ? ct : win[q - 10 < 0 ? 0 : q - 10]);
        }
        __syncthreads();
        const uint32_t rflags = (st.flags & 4) ? ROWF_NAN : 0u;
        if (tid >= 64) return;
        const int n = st.n;
        if (lane == 0) list[n] = 0ull;   // pad to pairs
        wave_sync();
        const u64 m0 = (lane < n) ? list[lane] : 0ull;
        const u64 m1 = (lane + 64 < n) ? list[lane + 64] : 0ull;
        int r0 = 0, r1 = 0;
        const ulonglong2* l2 = reinterpret_cast<const ulonglong2*>(list);
#pragma unroll 4
        for (int j = 0; j < (n + 1) >> 1; ++j) {
            const ulonglong2 x2 = l2[j];
            r0 += (x2.x > m0) + (x2.y > m0);
            r1 += (x2.x > m1) + (x2.y > m1);
        }
        wave_sync();
        if (lane < n && r0 < k) st.wv[r0] = m0;
        if (lane + 64 < n && r1 < k) st.wv[r1] = m1;
        wave_sync();
        const int nk = min(k, n);
        const u64 c = (lane < nk) ? st.wv[lane] : 0ull;
        wave_sync();
        wave_finalize(sa, sP, r, c, nk, rflags, st);
        return;
    }
    // buffer path: the table (or the counters) are dead and the buffer takes
    // their place
    u64* buf = reinterpret_cast<u64*>(smem + 9216);
    u64* ovf = a.ovf + (int64_t)r * a.ovf_cap;
    if (tid == 0) st.theta = (u64)Lk << 32;
    __syncthreads();
    offer_regs<9>(buf, ovf, a.buf_cap, k, cp, st);
    {
        const u64 c1[1] = {ct};
        offer_regs<1>(buf, ovf, a.buf_cap, k, c1, st);
    }
    offer_regs<NW>(buf, ovf, a.buf_cap, k, win, st);
    const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
    if (extra > 0) {
        for (int s2 = 0; s2 < S; ++s2) {
            const int n = st.soff[s2];
            for (int e0 = W; e0 < n; e0 += 8 * kBlock) {
                u64 c[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int e = e0 + q * kBlock + tid;
                    c[q] = cand[(int64_t)s2 * a.cand_cap + min(e, n - 1)];   // (clamped: no branch)
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) c[q] = (e0 + q * kBlock + tid < n) ? c[q] : 0ull;
                offer_regs<8>(buf, ovf, a.buf_cap, k, c, st);
            }
        }
    }
    __syncthreads();
    const uint32_t rflags = (st.flags & 4) ? ROWF_NAN : 0u;
    FinLds f{};
    select_and_finalize(sa, sP, r, buf, f, st, rflags);
}

// One block per row: finish the penalised ids, merge everything into the
// row's exact top-k (or argmax) and run the rest of the ladder.
//  - All first loads go out together: the history window, the slice counts,
//    the first `win` entries of every slice's list (NW per thread, entry g
//    of the window is slice g / win, position g % win) and u.
//  - The penalty table is built from the history; every id in it is
//    penalised: its logit is read from the row, masked, and run through
//    stages 1-6 (sampler.cpp:235-264) with the table's counts.
//  - Entries beyond a slice's window (rare) are offered in a second pass.
// Three blocks per CU (at most 168 registers, a few spilled): at two, the
// 1024-row batches of configuration 5 need two rounds of blocks (measured:
// 293 us against 322 us per cfg5 merge; four per CU spill more, 317 us).
template <bool GT, bool FAST, bool LM>
__global__ __launch_bounds__(kBlock, 3) void k_merge(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Shared st;
    __shared__ StreamArgs sa;
    __shared__ RowPlan sP;
    constexpr int NW = 16;
    const int tid = threadIdx.x;
    // The row whose slices k_stream handed over on this block's XCD (blocks
    // go to the XCDs round robin; row r's lists sit in the L2 of XCD
    // r * nslices / blocks_per_xcd).
    const int S = a.nslices, W = a.win;
    const int x = (int)(blockIdx.x % kXcds);
    const int r0 = min(a.rows, div_slices(x * a.blocks_per_xcd + S - 1, a));
    const int r1 = min(a.rows, div_slices((x + 1) * a.blocks_per_xcd + S - 1, a));
    const int r = r0 + (int)(blockIdx.x / kXcds);
    if (r >= r1) return;
    // Flag-mode launches read the plan first and request the history window
    // ahead of the lists (loads complete in order), so that the counters are
    // built while the lists are in flight; other launches request what needs
    // no plan first: the slice counts, the window of the slices' lists, the
    // ragged end and id 0's logit.
    constexpr bool hist_first = FAST && LM;
    RowPlan P;
    int32_t pre[8];
    if (hist_first) {
        P = plan_of(a, r);
        if (P.flags & RF_FULL) return;   // k_full's row
        // branch-free: clamped positions, used only below hist_len
#pragma unroll
        for (int q = 0; q < 8; ++q) pre[q] = -1;
        const int L = hist_len_of(a, P, r);
        if ((P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) && L > 0) {
            const int32_t* h = a.hist + (int64_t)r * a.hist_stride;
            const int p0 = L - P.scan_len;
#pragma unroll
            for (int q = 0; q < 8; ++q) pre[q] = h[max(0, min(p0 + q * kBlock + tid, L - 1))];
        }
    }
    // (flag mode: the bias ids count as penalised; read with the history)
    const int32_t bias_h = (hist_first && (P.flags & RF_BIAS) && tid < P.bias_cnt) ? a.bias_ids[P.bias_off + tid] : -1;
    const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
    const int cnt_raw = (tid < S) ? a.cand_n[(int64_t)r * S + tid] : 0;
    const uint32_t th_raw = (hist_first && tid < S) ? (uint32_t)a.cand_th[(int64_t)r * S + tid] : 0u;
    // one buffer resource over the row's lists: branch-free loads, entries
    // past the last slice read as 0
    u64 win[NW];
    {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<u64*>(cand), (short)0, S * a.cand_cap * 8, 0x00020000);
        const uint32_t magic = a.win_magic;
        const int cap = a.cand_cap;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int g = tid + j * kBlock;
            const int sl = (int)__umulhi((uint32_t)g, magic);   // g / W
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (sl * cap + (g - sl * W)) * 8, 0, 0);
            win[j] = ((u64)v[1] << 32) | v[0];
        }
    }
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
    // greedy: whether id 0 holds an allowed NaN; the row's ragged end (ids the
    // stream's whole-chunk loads leave out)
    const int32_t tail_t = (tid < a.vec_tail) ? a.vocab - a.vec_tail + tid : -1;
    // raw bits, converted where used (no wait here); absent ids read past the
    // row's buffer range and come back 0
    uint32_t xb0, xb1;
    {
        const int es = a.dtype == 0 ? 4 : 2;
        const __amdgpu_buffer_rsrc_t lr = row_rsrc(rowp, a.vocab, es);
        const int o0 = tid == 0 ? 0 : a.vocab * es, o1 = (tail_t >= 0 ? tail_t : a.vocab) * es;
        if (a.dtype == 0) {
            xb0 = __builtin_amdgcn_raw_buffer_load_b32(lr, o0, 0, 0);
            xb1 = __builtin_amdgcn_raw_buffer_load_b32(lr, o1, 0, 0);
        } else {
            xb0 = __builtin_amdgcn_raw_buffer_load_b16(lr, o0, 0, 0);
            xb1 = __builtin_amdgcn_raw_buffer_load_b16(lr, o1, 0, 0);
        }
    }
    if (!hist_first) {
        P = plan_of(a, r);
        if (P.flags & RF_FULL) return;   // k_full's row
    }
    const bool greedy = (P.flags & RF_GREEDY) != 0;
    const bool pen = (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;
    const bool masked = (P.flags & RF_MASK) != 0;
    const int k = P.top_k;
    if (tid == 0) {
        st.flags = 0;
        st.nan0 = 0;
        st.n = 0;
        st.theta = kThetaFloor;
        st.thmax = 0u;
    }
    if (!hist_first) hist_prefetch(a, P, r, pen, pre);
    const int32_t bias_t = (FAST && (P.flags & RF_BIAS) && tid < P.bias_cnt) ? a.bias_ids[P.bias_off + tid] : -1;
    auto logit_of = [&](uint32_t b) -> float { return __uint_as_float(a.dtype == 0 ? b : (b << 16)); };
    const float x0 = logit_of(xb0);
    const bool nan_at0 = greedy && tid == 0 && x0 != x0 && (!masked || (a.mask[(int64_t)r * a.mask_stride] & 1u));
    const float tail_x = logit_of(xb1);
    bool tail_ok = true;
    if (masked && tail_t >= 0) tail_ok = (a.mask[(int64_t)r * a.mask_stride + (tail_t >> 5)] >> (tail_t & 31)) & 1u;
    // u goes to LDS once the loads issued before it are needed anyway
    const double ur = a.u[r];
    if (tid == 0) {
        sa = a;
        sP = P;
    }
    if (tid < 32) {
        // expf's table from immediates (an indexed read would wait for every
        // load issued so far)
        uint64_t e = 0ull;
#pragma unroll
        for (int i = 0; i < 32; ++i) e = (tid == i) ? kExpT[i] : e;
        st.expT[tid] = e;
    }
    __syncthreads();
    if (tid < S) {
        st.soff[tid] = cnt_raw & 0x1FFFFFFF;
        if (cnt_raw & (1 << 30)) atomicOr(&st.flags, 4);   // a NaN logit in the slice
        if ((cnt_raw & 0x1FFFFFFF) > W) atomicOr(&st.flags, 8);   // a list past the window
        if (hist_first) atomicMax(&st.thmax, th_raw);
    }
    if (FAST) {
        merge_fast<NW, LM>(a, P, r, pre, bias_t, bias_h, nan_at0, tail_t, tail_x, tail_ok, ur, win, smem, st, sa, sP);
        return;
    }
    if (tid == 0) st.u = ur;
    HSAMP_PHASE(9500 + r, 0);
    // LDS: [row penalty table | finalize scratch] aliased, then the buffer.
    const PenaltyLds pl = pen_table<GT>(a, r, smem);
    if (pen) pen_build_row(a, P, r, pl, pre);   // its barriers publish the counts too
    else __syncthreads();
    HSAMP_PHASE(9500 + r, 1);
    u64* buf = reinterpret_cast<u64*>(smem + (a.merge_lds - (uint32_t)a.buf_cap * 8u));
    u64* ovf = a.ovf + (int64_t)r * a.ovf_cap;
    u64 best = 0ull;   // greedy

    if (pen) {
        // stages 1-6 for every penalised id (sampler.cpp:235-264), 8 slots per thread per pass
        const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
        const uint32_t* mrow = masked ? a.mask + (int64_t)r * a.mask_stride : nullptr;
        for (int base = 0; base < a.mhash_slots; base += 8 * kBlock) {
            int32_t t[8];
            float x[8];
            uint32_t mw[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int i = base + q * kBlock + tid;
                t[q] = (i < a.mhash_slots) ? (int32_t)tab_ld(&pl.hkey[i]) : -1;   // kEmpty reads as -1
            }
            load_logits<8>(rowp, a.dtype, t, x);
#pragma unroll
            for (int q = 0; q < 8; ++q) mw[q] = (masked && t[q] >= 0) ? mrow[t[q] >> 5] : 0xFFFFFFFFu;
            u64 c[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                c[q] = 0ull;
                if (t[q] < 0) continue;
                float y = ((mw[q] >> (t[q] & 31)) & 1u) ? x[q] : -__builtin_inff();
                y = pen_apply(y, t[q], sa, sP, pl);
                if (greedy) {
                    if (y != y) {
                        atomicOr(&st.flags, 4);
                        if (t[q] == 0) atomicOr(&st.nan0, 1);
                        continue;
                    }
                } else {
                    if (P.flags & RF_TEMP) y = y * P.inv_temp;
                    if (y != y) {
                        atomicOr(&st.flags, 4);
                        y = -__builtin_inff();
                    }
                }
                c[q] = comp(key32(y), t[q]);
            }
            if (greedy) {
#pragma unroll
                for (int q = 0; q < 8; ++q) best = c[q] > best ? c[q] : best;
            } else {
                offer_regs<8>(buf, ovf, a.buf_cap, k, c, st);
            }
        }
    }

    HSAMP_PHASE(9500 + r, 2);
    // the ragged end, unless penalised
    u64 ct = 0ull;
    if (tail_t >= 0) {
        bool pt = false;
        if (pen) {
            uint32_t s0 = hslot(tail_t, pl);
            uint32_t kk;
            while ((kk = tab_ld(&pl.hkey[s0])) != kEmpty && kk != (uint32_t)tail_t) s0 = (s0 + 1) & pl.hmask;
            pt = kk == (uint32_t)tail_t;
        }
        if (!pt) ct = tail_candidate(tail_x, tail_ok, tail_t, greedy, P.inv_temp, st);
    }
    best = ct > best ? ct : best;
    // the slices' lists: the window entries, then whatever lies beyond it
    int extra = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int g = tid + j * kBlock;
        const int sl = (int)__umulhi((uint32_t)g, a.win_magic);   // g / W
        if (sl >= S || g - sl * W >= st.soff[sl]) win[j] = 0ull;
    }
    extra = (st.flags & 8) ? 1 : 0;   // some slice's list runs past the window
    if (greedy) {
#pragma unroll
        for (int j = 0; j < NW; ++j) best = win[j] > best ? win[j] : best;
        best = block_max_u64(best, st);
        __syncthreads();
        int32_t gtok = 0;
        if (tid == 0) {
            bool pen0 = false;   // id 0 penalised: settled with the table
            if (pen) {
                uint32_t s0 = hslot(0, pl);
                uint32_t kk;
                while ((kk = tab_ld(&pl.hkey[s0])) != kEmpty && kk != 0u) s0 = (s0 + 1) & pl.hmask;
                pen0 = kk == 0u;
            }
            const bool nan0 = pen0 ? st.nan0 != 0 : nan_at0;
            gtok = nan0 ? 0 : comp_idx(best);
            if (a.row_flags != nullptr) a.row_flags[r] = ROWF_GREEDY | ((st.flags & 4) ? ROWF_NAN : 0u);
            if (a.topk_count != nullptr) a.topk_count[r] = -1;
            if (a.kept_count != nullptr) a.kept_count[r] = 0;
        }
        if (wave_id() == 0) emit_token_wave(a, r, gtok);
        return;
    }
    {
        const u64 c1[1] = {ct};
        offer_regs<1>(buf, ovf, a.buf_cap, k, c1, st);
    }
    offer_regs<NW>(buf, ovf, a.buf_cap, k, win, st);
    HSAMP_PHASE(9500 + r, 3);
    if (extra > 0) {
        for (int sl = 0; sl < S; ++sl) {
            const int n = st.soff[sl];
            for (int e0 = W; e0 < n; e0 += 8 * kBlock) {
                u64 c[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int e = e0 + q * kBlock + tid;
                    c[q] = cand[(int64_t)sl * a.cand_cap + min(e, n - 1)];   // (clamped: no branch)
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) c[q] = (e0 + q * kBlock + tid < n) ? c[q] : 0ull;
                offer_regs<8>(buf, ovf, a.buf_cap, k, c, st);
            }
        }
    }
    __syncthreads();
    HSAMP_PHASE(9500 + r, 4);
    const uint32_t rflags = (st.flags & 4) ? ROWF_NAN : 0u;
    // the finalize scratch: sort keys in the candidate buffer (each entry is
    // read into its key in place), the rest where the penalty table was
    FinLds f;
    f.sortk = buf;
    f.fidx = reinterpret_cast<int32_t*>(smem);
    f.fv = reinterpret_cast<float*>(f.fidx + a.kmax);
    f.fe = f.fv + a.kmax;
    f.fp = f.fe;
    f.keep = reinterpret_cast<uint8_t*>(f.fe + a.kmax);
    select_and_finalize(sa, sP, r, buf, f, st, rflags);
}

// ---- the merge of exact lists -------------------------------------------------------

// A greedy row's argmax from its exact lists (sampler.cpp:220-228): the
// largest final logit, -0 counted as +0, the lowest id among equal ones (the
// composites order them so once the key is made canonical); id 0 when its
// final logit is NaN (nan0: thread 0 holds slice 0's flag); id 0 when no id
// is above -inf (none is then greater than id 0's). win: NW entries of the
// windows already loaded (0 = none); entries past a window (more) are read
// here.
template <int NW>
__device__ __forceinline__ void pick_greedy(const StreamArgs& a, int r, const u64* cand, int S, int W, bool more,
                                            const u64 (&win)[NW], bool nan0, bool nan_any, Shared& st) {
    const int tid = threadIdx.x;
    auto canon = [](u64 c) -> u64 {
        return c == 0ull ? 0ull : ((u64)key32(key_to_float((uint32_t)(c >> 32))) << 32) | (c & 0xFFFFFFFFull);
    };
    u64 best = 0ull;
#pragma unroll
    for (int j = 0; j < NW; ++j) best = max(best, canon(win[j]));
    if (more) {
        for (int sl = 0; sl < S; ++sl) {
            const int n = st.soff[sl];
            for (int e = W + tid; e < n; e += kBlock) best = max(best, canon(cand[(int64_t)sl * a.cand_cap + e]));
        }
    }
    if (tid == 0) st.nan0 = nan0 ? 1 : 0;
    best = block_max_u64(best, st);   // (its barriers publish st.nan0)
    if (wave_id() == 0) emit_token_wave(a, r, (st.nan0 || best == 0ull) ? 0 : comp_idx(best));
    if (tid == 0) {
        if (a.row_flags != nullptr) a.row_flags[r] = ROWF_GREEDY | (nan_any ? ROWF_NAN : 0u);
        if (a.topk_count != nullptr) a.topk_count[r] = -1;
        if (a.kept_count != nullptr) a.kept_count[r] = 0;
    }
}

// One block per sampling row whose slices left exact lists (k_stream's EX
// kernels; k <= 64): the row's exact top-k and the rest of the ladder
// (sampler.cpp:267-277). No history work and no logit reads: every
// candidate carries its final logit before temperature, which is applied here.
// A greedy row takes the argmax of its lists instead (pick_greedy).
//  - The slice counts, a window of W entries of every slice's list (NW per
//    thread; entry g is slice g / W, position g % W), the plan and u are
//    requested together.
//  - Selection: the candidates' key range gives the bits they all share; a
//    256-bin LDS histogram of the next 8 bits finds the bin holding the k-th
//    largest key. The candidates above that bin are all kept; those in it (at
//    most 64) are ranked among themselves (composite order, ties to the lower
//    id) and the best join. A fuller bin sends every candidate in it or above
//    to an exact rank: by wave 0 when at most 128, else by the block (after a
//    radix compaction to the k largest when more than 256).
//  - A list longer than its window (ties, flat rows) takes the buffer path.
template <int NW>
__global__ __launch_bounds__(kBlock) void k_pick(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Shared st;
    const int tid = threadIdx.x, lane = lane_id();
    uint32_t bid = blockIdx.x;
    // the launch arguments the first loads need, in registers together: one
    // round of scalar loads instead of one per branch that uses them (an asm
    // statement that reads them; it touches no memory)
    __asm__("" : "+s"(bid)
            : "s"(a.blocks_per_xcd), "s"(a.ns_magic), "s"(a.rows), "s"(a.nslices), "s"(a.win), "s"(a.cand),
              "s"(a.cand_cap), "s"(a.cand_n), "s"(a.win_magic), "s"(a.plans), "s"(a.u));
    const int S = a.nslices, W = a.win;
    // the row whose slices k_stream handed over on this block's XCD
    const int x = (int)(bid % kXcds);
    const int r0 = min(a.rows, div_slices(x * a.blocks_per_xcd + S - 1, a));
    const int r1 = min(a.rows, div_slices((x + 1) * a.blocks_per_xcd + S - 1, a));
    const int r = r0 + (int)(bid / kXcds);
    if (r >= r1) return;
    const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
    const int cnt_raw = (tid < S) ? a.cand_n[(int64_t)r * S + tid] : 0;
    u64 win[NW];
    {
        // one buffer resource over the row's lists: entries past the last
        // slice read as 0
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<u64*>(cand), (short)0, S * a.cand_cap * 8, 0x00020000);
        const uint32_t magic = a.win_magic;
        const int cap = a.cand_cap;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int g = tid + j * kBlock;
            const int sl = (int)__umulhi((uint32_t)g, magic);   // g / W
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (sl * cap + (g - sl * W)) * 8, 0, 0);
            win[j] = ((u64)v[1] << 32) | v[0];
        }
    }
    // the plan and u after the lists (scalar loads: a wait for them placed
    // ahead of the lists' loads would delay those by a memory round trip)
    __builtin_amdgcn_sched_barrier(0);
    const RowPlan P = plan_of(a, r);
    const double ur = a.u[r];
    // expf's table, loaded after the lists (its wait then costs nothing) and
    // put in LDS once they are in
    const uint64_t etab = kExpT[tid & 31];
    HSAMP_PHASE(8192 + r, 0);
    // (u goes to LDS once the lists are in)
    if (tid == 0) {
        st.n = 0;
        st.nst = 0;
        st.theta = kThetaFloor;
    }
    st.hist[tid] = 0u;
    // the lists' lengths, and per wave whether a slice saw a NaN logit (4) or
    // a list runs past the window (8), all published by one barrier
    if (tid < S) st.soff[tid] = cnt_raw & 0x1FFFFFFF;
    {
        const u64 bn = __ballot(tid < S && (cnt_raw & (1 << 30)) != 0);
        const u64 bw = __ballot(tid < S && (cnt_raw & 0x1FFFFFFF) > W);
        if (lane == 0) st.fw[wave_id()] = (bn != 0ull ? 4 : 0) | (bw != 0ull ? 8 : 0);
    }
    __syncthreads();
    HSAMP_PHASE(8192 + r, 1);
    const int fl0 = st.fw[0] | st.fw[1] | st.fw[2] | st.fw[3];
    const int k = P.top_k;
    const float inv_t = P.inv_temp;
    const uint32_t rflags = (fl0 & 4) ? ROWF_NAN : 0u;
    if (P.flags & RF_GREEDY) {
        pick_greedy(a, r, cand, S, W, (fl0 & 8) != 0, win, tid == 0 && (cnt_raw & (1 << 29)) != 0,
                    (fl0 & 4) != 0, st);
        return;
    }
    // the lists carry final logits before temperature: composites of the
    // scaled keys (sampler.cpp:101-106)
    auto scaled = [&](u64 c) -> u64 {
        return ((u64)scaled_key((uint32_t)(c >> 32), inv_t) << 32) | (c & 0xFFFFFFFFull);
    };
    // (k_stream leaves each window's entries past its list at 0, and the
    // buffer resource reads 0 past the last slice)
    uint32_t lm = 0u;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        win[j] = (win[j] != 0ull) ? scaled(win[j]) : 0ull;
        lm = max(lm, (uint32_t)(win[j] >> 32));
    }
    if (tid < 32) st.expT[tid] = etab;   // read by wave 0 after later barriers
    u64* list = reinterpret_cast<u64*>(smem);
    uint32_t bstar = 0u;
    int shift = 0;
    bool blk = false;   // the buffer path: the block ranks the buffer
    if (fl0 & 8) {
        // buffer path: every entry offered under a rising threshold
        if (tid == 0) st.flags = fl0;
        __syncthreads();
        u64* ovf = a.ovf + (int64_t)r * a.ovf_cap;
        offer_regs<NW>(list, ovf, a.buf_cap, k, win, st);
        for (int sl = 0; sl < S; ++sl) {
            const int n = st.soff[sl];
            for (int e0 = W; e0 < n; e0 += 8 * kBlock) {
                u64 c[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int e = e0 + q * kBlock + tid;
                    c[q] = cand[(int64_t)sl * a.cand_cap + min(e, n - 1)];   // (clamped: no branch)
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) c[q] = (e0 + q * kBlock + tid < n) ? scaled(c[q]) : 0ull;
                offer_regs<8>(list, ovf, a.buf_cap, k, c, st);
            }
        }
        // the buffer's entries are ranked by the block below
        if (tid == 0) st.u = ur;
        __syncthreads();
        blk = true;
    } else {
    // The k-th largest key's 8-bit bin under the prefix every candidate
    // shares (the block's key range), from a 256-bin LDS histogram; the
    // candidates in that bin or above go to the list.
    uint32_t kmn = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NW; ++j)
        if (win[j] != 0ull) kmn = min(kmn, (uint32_t)(win[j] >> 32));
    kmn = wave_min_u32(kmn);
    uint32_t kmx = wave_max_u32(lm);
    if (lane == 0) {
        st.twave[wave_id()] = kmn;
        st.minv_w[wave_id()] = kmx;
    }
    __syncthreads();
    HSAMP_PHASE(8192 + r, 2);
    kmn = st.twave[0];
    kmx = (uint32_t)st.minv_w[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) {
        kmn = min(kmn, st.twave[i]);
        kmx = max(kmx, (uint32_t)st.minv_w[i]);
    }
    const int hb = (kmx > kmn) ? 31 - __clz((int)(kmn ^ kmx)) : 0;
    shift = max(0, hb - 7);
#pragma unroll
    for (int j = 0; j < NW; ++j)
        if (win[j] != 0ull) atomicAdd(&st.hist[((uint32_t)(win[j] >> 32) >> shift) & 255u], 1u);
    __syncthreads();
    HSAMP_PHASE(8192 + r, 11);
    if (tid < 64) {
        // bins from the top: lane l holds 255-4l .. 252-4l
        const int c0 = st.hist[255 - 4 * lane], c1 = st.hist[254 - 4 * lane];
        const int c2 = st.hist[253 - 4 * lane], c3 = st.hist[252 - 4 * lane];
        const int s4 = c0 + c1 + c2 + c3;
        const int incl = wave_incl_sum_i(s4);
        const int excl = incl - s4;
        if (lane == 0) st.sel_d = 0;   // fewer than k candidates: all of them
        if (excl < k && k <= incl) {
            const int q = (excl + c0 >= k) ? 0 : (excl + c0 + c1 >= k) ? 1 : (excl + c0 + c1 + c2 >= k) ? 2 : 3;
            st.sel_d = 255 - 4 * lane - q;
        }
    }
    __syncthreads();
    HSAMP_PHASE(8192 + r, 12);
    bstar = (uint32_t)__builtin_amdgcn_readfirstlane(st.sel_d);
    {
        // the candidates in the k-th's bin or above, packed into the list in
        // (slot, lane) order: one ballot per slot, one LDS atomic per wave
        int pj[NW];
        uint32_t sel = 0u;
        int wtot = 0;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const bool in = (win[j] != 0ull) & ((((uint32_t)(win[j] >> 32) >> shift) & 255u) >= bstar);
            const u64 m = __ballot(in);
            pj[j] = wtot + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            sel |= (uint32_t)in << j;
            wtot += __popcll(m);
        }
        int base = 0;
        if (lane == 0 && wtot > 0) base = atomicAdd(&st.n, wtot);
        base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
        for (int j = 0; j < NW; ++j)
            if ((sel >> j) & 1u) list[base + pj[j]] = win[j];
    }
    if (tid == 0) st.u = ur;
    __syncthreads();
    }
    HSAMP_PHASE(8192 + r, 3);
    int n = st.n;
    int nk;   // wave 0: the row's top-k set in st.wv[0, nk), any order
    if (!blk && n <= 128) {
        // Wave 0 holds the n entries (two per lane). Those above the k-th's
        // bin are all in; the ones in it (bcnt) are packed aside, ranked among
        // themselves (composite order, ties to the lower id) and the best
        // bneed join. More than 64 in the bin: every entry is ranked.
        if (tid >= 64) return;
        const u64 m0 = (lane < n) ? list[lane] : 0ull;
        const u64 m1 = (lane + 64 < n) ? list[lane + 64] : 0ull;
        const uint32_t b0 = ((uint32_t)(m0 >> 32) >> shift) & 255u, b1 = ((uint32_t)(m1 >> 32) >> shift) & 255u;
        const bool a0 = (m0 != 0ull) & (b0 > bstar), a1 = (m1 != 0ull) & (b1 > bstar);
        const bool i0 = (m0 != 0ull) & (b0 == bstar), i1 = (m1 != 0ull) & (b1 == bstar);
        const u64 ma0 = __ballot(a0), ma1 = __ballot(a1), mi0 = __ballot(i0), mi1 = __ballot(i1);
        const int above = __popcll(ma0) + __popcll(ma1);
        const int bcnt = __popcll(mi0) + __popcll(mi1);
        if (bcnt <= 64) {
            const int bneed = k - above;
            u64* bl = list + 128;   // the bin's entries, packed (after the n <= 128 entries)
            auto mb = [&](u64 m) -> int {
                return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            };
            if (i0) bl[mb(mi0)] = m0;
            if (i1) bl[__popcll(mi0) + mb(mi1)] = m1;
            if (lane == 0) bl[bcnt] = 0ull;   // pad to pairs
            wave_sync();
            const u64 e = (lane < bcnt) ? bl[lane] : 0ull;
            int q = 0;
            const ulonglong2* b2 = reinterpret_cast<const ulonglong2*>(bl);
#pragma unroll 4
            for (int j = 0; j < (bcnt + 1) >> 1; ++j) {
                const ulonglong2 x2 = b2[j];
                q += (x2.x > e) + (x2.y > e);
            }
            wave_sync();
            if (a0) st.wv[mb(ma0)] = m0;
            if (a1) st.wv[__popcll(ma0) + mb(ma1)] = m1;
            if (lane < bcnt && q < bneed) st.wv[above + q] = e;
            nk = min(k, above + min(bneed, bcnt));
        } else {
            // rank = entries above, over the (distinct) entries
            if (lane == 0) list[n] = 0ull;   // pad to pairs
            wave_sync();
            int q0 = 0, q1 = 0;
            const ulonglong2* l2 = reinterpret_cast<const ulonglong2*>(list);
#pragma unroll 4
            for (int j = 0; j < (n + 1) >> 1; ++j) {
                const ulonglong2 x2 = l2[j];
                q0 += (x2.x > m0) + (x2.y > m0);
                q1 += (x2.x > m1) + (x2.y > m1);
            }
            wave_sync();
            if (lane < n && q0 < k) st.wv[q0] = m0;
            if (lane + 64 < n && q1 < k) st.wv[q1] = m1;
            nk = min(k, n);
        }
        wave_sync();
    } else {
        if (n > 256) {
            buf_compact(list, k, st);
            n = st.n;
        }
        block_rank_topk(list, n, k, st);
        if (tid >= 64) return;
        nk = min(k, n);
    }
    // one finalize for every path
    const u64 c = (lane < nk) ? st.wv[lane] : 0ull;
    wave_sync();
    HSAMP_PHASE(8192 + r, 4);
    wave_finalize(a, P, r, c, nk, rflags, st);
    HSAMP_PHASE(8192 + r, 5);
}

// ---- the merge of exact lists, large k ---------------------------------------------

constexpr int kLRegs = 24;   // list entries per thread k_pick_l's direct selection holds

// The top k of a row's S lists (counts in st.soff) into buf[0 .. min(k, n)),
// when all n entries fit kLRegs per thread; returns false (nothing done)
// otherwise. Entry e of the concatenated lists is thread e % kBlock's slot
// e / kBlock; its slice comes from the lists' start offsets (st.hist holds
// them while the entries load). The k-th largest composite: 8-bit radix
// passes from the highest bit in which the entries differ, each a 256-bin
// LDS histogram under the prefix fixed so far, until the bin holding the
// k-th holds exactly what is still needed. Composites are distinct (ids
// differ), so exactly min(k, n) entries are at or above it.
template <class Scale>
__device__ __forceinline__ bool direct_select(const u64* cand, int cap, int S, int k, Scale scaled, u64* buf,
                                              Shared& st, int r) {
    (void)r;   // (phase clocks of an instrumented build)
    const int tid = threadIdx.x, lane = lane_id();
    if (tid == 0) {
        int acc = 0;
        for (int sl = 0; sl < S; ++sl) {
            st.hist[sl] = (uint32_t)acc;
            acc += st.soff[sl];
        }
        st.hist[S] = (uint32_t)acc;
    }
    __syncthreads();
    const int n = (int)st.hist[S];
    if (n > kLRegs * kBlock) return false;   // (uniform: every thread read the same total)
    u64 v[kLRegs];
    {
        // (entries past n read the last one, clamped, and count as empty)
        int sl = 0;
        int at[kLRegs];
#pragma unroll
        for (int m = 0; m < kLRegs; ++m) {
            const int e = min(tid + m * kBlock, max(n - 1, 0));
            while (sl + 1 < S && e >= (int)st.hist[sl + 1]) ++sl;
            at[m] = sl * cap + (e - (int)st.hist[sl]);
        }
#pragma unroll
        for (int m = 0; m < kLRegs; ++m) v[m] = cand[at[m]];
#pragma unroll
        for (int m = 0; m < kLRegs; ++m) v[m] = (tid + m * kBlock < n) ? scaled(v[m]) : 0ull;
    }
    __syncthreads();   // the offsets are read before st.hist becomes the histogram
    HSAMP_PHASE(9500 + r, 1);
    if (n <= k) {
        int cnt = 0;
#pragma unroll
        for (int m = 0; m < kLRegs; ++m) cnt += v[m] != 0ull ? 1 : 0;
        int total;
        int pos = block_excl_scan(cnt, &total, st);
#pragma unroll
        for (int m = 0; m < kLRegs; ++m)
            if (v[m] != 0ull) buf[pos++] = v[m];
        __syncthreads();
        if (tid == 0) st.n = total;
        __syncthreads();
        return true;
    }
    u64 lo = ~0ull, hi = 0ull;
#pragma unroll
    for (int m = 0; m < kLRegs; ++m) {
        if (v[m] != 0ull) {
            lo = v[m] < lo ? v[m] : lo;
            hi = v[m] > hi ? v[m] : hi;
        }
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const u64 a2 = shfl_xor_u64(lo, d), b2 = shfl_xor_u64(hi, d);
        lo = a2 < lo ? a2 : lo;
        hi = b2 > hi ? b2 : hi;
    }
    if (lane == 0) {
        st.ured[wave_id()] = lo;
        st.minv_w[wave_id()] = hi;
    }
    __syncthreads();
    lo = st.ured[0];
    hi = st.minv_w[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) {
        lo = st.ured[i] < lo ? st.ured[i] : lo;
        hi = st.minv_w[i] > hi ? st.minv_w[i] : hi;
    }
    const int hb = 63 - __clzll((long long)(lo ^ hi));   // highest differing bit (n > k >= 1: n >= 2)
    u64 pmask = (hb >= 63) ? 0ull : ~((2ull << hb) - 1ull);
    u64 prefix = hi & pmask;
    int need = k;
    u64 kth = 0ull;
    HSAMP_PHASE(9500 + r, 2);
    for (int shift = hb >= 7 ? hb - 7 : 0;;) {
        st.hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < kLRegs; ++m)
            if (v[m] != 0ull && (v[m] & pmask) == prefix) atomicAdd(&st.hist[(uint32_t)(v[m] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 64) {
            const int c0 = st.hist[255 - 4 * lane], c1 = st.hist[254 - 4 * lane];
            const int c2 = st.hist[253 - 4 * lane], c3 = st.hist[252 - 4 * lane];
            const int s4 = c0 + c1 + c2 + c3;
            const int incl = wave_incl_sum_i(s4);
            const int excl = incl - s4;
            if (excl < need && need <= incl) {
                int q, cnt, before;
                if (excl + c0 >= need) { q = 0; cnt = c0; before = excl; }
                else if (excl + c0 + c1 >= need) { q = 1; cnt = c1; before = excl + c0; }
                else if (excl + c0 + c1 + c2 >= need) { q = 2; cnt = c2; before = excl + c0 + c1; }
                else { q = 3; cnt = c3; before = excl + c0 + c1 + c2; }
                st.sel_d = 255 - 4 * lane - q;
                st.sel_need = need - before;
                st.sel_cnt = cnt;
            }
        }
        __syncthreads();
        const int dgt = st.sel_d, cnt = st.sel_cnt;
        need = st.sel_need;
        prefix = (prefix & ~((u64)0xFF << shift)) | ((u64)dgt << shift);
        pmask |= (u64)0xFF << shift;
        __syncthreads();   // every thread has read sel_* before the next pass may write them
        if (cnt == need || shift == 0) {
            // every entry under this prefix is in: the k-th is their minimum
            u64 mn = ~0ull;
#pragma unroll
            for (int m = 0; m < kLRegs; ++m)
                if (v[m] != 0ull && (v[m] & pmask) == prefix && v[m] < mn) mn = v[m];
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) {
                const u64 o = shfl_xor_u64(mn, d);
                mn = o < mn ? o : mn;
            }
            if (lane == 0) st.ured[wave_id()] = mn;
            __syncthreads();
            kth = st.ured[0];
#pragma unroll
            for (int i = 1; i < kBlock / 64; ++i) kth = st.ured[i] < kth ? st.ured[i] : kth;
            break;
        }
        shift = shift >= 8 ? shift - 8 : 0;
    }
    HSAMP_PHASE(9500 + r, 3);
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < kLRegs; ++m) cnt += (v[m] != 0ull && v[m] >= kth) ? 1 : 0;
    int total;
    int pos = block_excl_scan(cnt, &total, st);
#pragma unroll
    for (int m = 0; m < kLRegs; ++m)
        if (v[m] != 0ull && v[m] >= kth) buf[pos++] = v[m];
    __syncthreads();
    if (tid == 0) {
        st.n = total;
        st.theta = kth;
    }
    __syncthreads();
    return true;
}

// One block per sampling row whose slices left exact lists with 64 < k <= 1024
// (the exact stream's block-level bound): every entry of the row's lists, its
// final raw key scaled by the row's temperature, is offered into the LDS
// candidate buffer under a rising threshold (a per-row overflow area past
// it), then the exact top-k and the rest of the ladder as the general merge
// finishes its rows (select_and_finalize: radix select, finalize_row). The
// lists are final: no history, no logit reads, no ragged end (the stream's
// last slice took it). LDS: [finalize scratch][candidate buffer], sized by
// the host so that four blocks share a CU (with 128 registers per lane, four
// waves per SIMD): a batch of up to 1024 such rows runs in one round.
__global__ __launch_bounds__(kBlock, 4) void k_pick_l(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Shared st;
    __shared__ StreamArgs sa;
    __shared__ RowPlan sP;
    const int tid = threadIdx.x;
    const int S = a.nslices;
    const int x = (int)(blockIdx.x % kXcds);
    const int r0 = min(a.rows, div_slices(x * a.blocks_per_xcd + S - 1, a));
    const int r1 = min(a.rows, div_slices((x + 1) * a.blocks_per_xcd + S - 1, a));
    const int r = r0 + (int)(blockIdx.x / kXcds);
    if (r >= r1) return;
    HSAMP_PHASE(9500 + r, 0);
    const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
    const int cnt_raw = (tid < S) ? a.cand_n[(int64_t)r * S + tid] : 0;
    const RowPlan P = plan_of(a, r);
    const double ur = a.u[r];
    const float inv_t = P.inv_temp;
    if (tid == 0) {
        st.flags = 0;
        st.n = 0;
        st.theta = kThetaFloor;
        st.u = ur;
        sa = a;
        sP = P;
    }
    if (tid < 32) st.expT[tid] = kExpT[tid];
    __syncthreads();
    if (tid < S) {
        st.soff[tid] = cnt_raw & 0x1FFFFFFF;
        if (cnt_raw & (1 << 30)) atomicOr(&st.flags, 4);   // a NaN logit in the slice
    }
    __syncthreads();
    const int k = P.top_k;
    u64* buf = reinterpret_cast<u64*>(smem + (a.merge_lds - (uint32_t)a.buf_cap * 8u));
    u64* ovf = a.ovf + (int64_t)r * a.ovf_cap;
    auto scaled = [&](u64 c) -> u64 {
        return ((u64)scaled_key((uint32_t)(c >> 32), inv_t) << 32) | (c & 0xFFFFFFFFull);
    };
    // Rows whose lists hold at most kLRegs entries per thread in all: every
    // entry in registers at once (one round of loads), the exact k-th by radix
    // passes over them, and only the top k written to the buffer.
    if (P.flags & RF_GREEDY) {
        const u64 none[1] = {0ull};
        pick_greedy(a, r, cand, S, 0, true, none, tid == 0 && (cnt_raw & (1 << 29)) != 0, (st.flags & 4) != 0, st);
        return;
    }
    if (S < 256 && direct_select(cand, a.cand_cap, S, k, scaled, buf, st, r)) {
        HSAMP_PHASE(9500 + r, 4);
        const uint32_t rflags = (st.flags & 4) ? ROWF_NAN : 0u;
        FinLds f;
        f.sortk = buf;
        f.fidx = reinterpret_cast<int32_t*>(smem);
        f.fv = reinterpret_cast<float*>(f.fidx + a.kmax);
        f.fe = f.fv + a.kmax;
        f.fp = f.fe;
        f.keep = reinterpret_cast<uint8_t*>(f.fe + a.kmax);
        select_and_finalize(sa, sP, r, buf, f, st, rflags);
        return;
    }
    for (int sl = 0; sl < S; ++sl) {
        const int n = st.soff[sl];
        const u64* lst = cand + (int64_t)sl * a.cand_cap;
        for (int e0 = 0; e0 < n; e0 += 8 * kBlock) {
            u64 c[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) c[q] = lst[min(e0 + q * kBlock + tid, n - 1)];   // (clamped: no branch)
#pragma unroll
            for (int q = 0; q < 8; ++q) c[q] = (e0 + q * kBlock + tid < n) ? scaled(c[q]) : 0ull;
            offer_regs<8>(buf, ovf, a.buf_cap, k, c, st);
        }
    }
    __syncthreads();
    HSAMP_PHASE(9500 + r, 4);
    const uint32_t rflags = (st.flags & 4) ? ROWF_NAN : 0u;
    FinLds f;
    f.sortk = buf;
    f.fidx = reinterpret_cast<int32_t*>(smem);
    f.fv = reinterpret_cast<float*>(f.fidx + a.kmax);
    f.fe = f.fv + a.kmax;
    f.fp = f.fe;
    f.keep = reinterpret_cast<uint8_t*>(f.fe + a.kmax);
    select_and_finalize(sa, sP, r, buf, f, st, rflags);
}

// ---- writeback -------------------------------------------------------------------

template <bool GT>
__global__ __launch_bounds__(kBlock) void k_writeback(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ StreamArgs sa;
    __shared__ RowPlan sP;
    const int tid = threadIdx.x;
    const int logical = (int)(blockIdx.x % kXcds) * a.blocks_per_xcd + (int)(blockIdx.x / kXcds);
    const int r = div_slices(logical, a), s = logical - r * a.nslices;
    if (r >= a.rows) return;
    const RowPlan P = plan_of(a, r);
    if (P.flags & RF_FULL) return;   // k_full writes its rows back itself
    if (tid == 0) {
        sa = a;
        sP = P;
    }
    const int V = a.vocab;
    const int lo = s * a.slice_len;
    const int hi = min(V, lo + a.slice_len);
    const bool greedy = (P.flags & RF_GREEDY) != 0;
    const bool pen = (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;
    // LDS: [row penalty table (when not global)] [kept ids of this slice]
    const PenaltyLds pl = pen_table<GT>(a, r, smem);
    uint32_t* keepbm = reinterpret_cast<uint32_t*>(smem) + (GT ? 0 : 2 * a.mhash_slots);
    int32_t pre[8];
    hist_prefetch(a, P, r, pen && !GT, pre);
    for (int i = tid; i < a.bitmap_words; i += kBlock) keepbm[i] = 0u;
    // a global table is the one k_merge built for this row; an LDS one is rebuilt
    if (pen && !GT) pen_build_row(a, P, r, pl, pre);
    else __syncthreads();
    if (!greedy) {
        const int n = a.fin_n[r];
        for (int j = tid; j < n; j += kBlock) {
            const int t = a.fin_idx[(int64_t)r * a.fin_cap + j];
            if (t >= lo && t < hi) atomicOr(&keepbm[(t - lo) >> 5], 1u << ((t - lo) & 31));
        }
        __syncthreads();
    }
    float* row = static_cast<float*>(const_cast<void*>(a.logits)) + (int64_t)r * a.logits_stride;
    const uint32_t* mrow = (P.flags & RF_MASK) ? a.mask + (int64_t)r * a.mask_stride : nullptr;
    for (int e = lo + tid; e < hi; e += kBlock) {
        float x = row[e];
        if (mrow != nullptr && !((mrow[e >> 5] >> (e & 31)) & 1u)) x = -__builtin_inff();
        if (pen) {
            // ids without a table entry pass through unchanged
            uint32_t sl = hslot(e, pl);
            uint32_t hk;
            while ((hk = tab_ld(&pl.hkey[sl])) != kEmpty && hk != (uint32_t)e) sl = (sl + 1) & pl.hmask;
            if (hk == (uint32_t)e) x = pen_apply(x, e, sa, sP, pl);
        }
        if (!greedy) {
            if (P.flags & RF_TEMP) x = x * P.inv_temp;
            if (!((keepbm[(e - lo) >> 5] >> ((e - lo) & 31)) & 1u)) x = -__builtin_inff();
        }
        row[e] = x;
    }
}

// ---- full-vocabulary rows ---------------------------------------------------------
// (the exact-sum engine, block helpers and the top-p driver are in hsamp_xsum.h)

// Window-order helpers: wave `wid` takes windows wid, wid + kFW, ...; lane l
// holds ids w * WS + g * 512 + l * 8 + j of each 512-step g.

// e = expf(x - m) for every finite x of the row (0 for -inf and padding),
// into pv, with each window's approximate sum in f.winA.
__device__ void full_exp(const float* fv, float* pv, float m, int nW, int G, FullLds f, FullShared& st) {
    const int lane = lane_id();
    const int WS = kFWin * G;
    float ws = 0.0f;
    wpass(fv, nW, G, [&](int w, int g, const float (&x)[8]) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = (x[j] == -__builtin_inff()) ? 0.0f : libm_expf_t(x[j] - m, st.expT);
            ws += v[j];
        }
        float4* dst = reinterpret_cast<float4*>(pv + (size_t)w * WS + g * kFWin + lane * 8);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
        if (g == G - 1) {
            ws = wave_tree_prefix_f(ws);
            if (lane == 63) f.winA[w] = ws;
            ws = 0.0f;
        }
    });
    __syncthreads();
}

// ---- full-vocabulary rows, their whole-row passes over many blocks ------------------
// k_full runs one block per row; a row of the batch has V ids. For its rows
// with a plain transform (RF_FPRE: mask and temperature, no penalties, no
// logit bias, no top-k), the passes over the whole row that need no
// sequential order run first over B x nW waves, one index-order window
// (512 G ids) per wave, in the layout k_full uses (fullv / fullp, windows of
// full_stride), and leave per-window tables (FS_*) for it:
//   k_fs_max: the transform into fullv (the row's -inf padding included),
//             each window's maximum m_w, whether it held a NaN, how many ids
//             it leaves in and its sum of exp(x - m_w) (fast exp; a
//             prediction only);
//   k_fs_exp: the row's maximum m, the numerators expf(x - m) into fullp,
//             each window's sum in double (rows without top-p and min-p: the
//             draw's window prefixes) or its smallest numerator above 0
//             (rows with them: top-p's key range), and its binade -- predicted from
//             the windows before it, sum over v < w of exp(m_v - m) times
//             k_fs_max's sums -- with its values' integer increments there
//             (as exact_index_sum forms them; lane tables when the window's
//             own approximate sum takes it to another binade).
// k_full then composes the exact sum from the tables and goes on as for its
// other rows. The binades are predictions: the compose checks each against
// the exact running sum and resolves a window that misses by its values, so
// they decide speed, not results. Every value is computed as k_full computes
// it, in the same order where order matters.
__device__ __forceinline__ int fs_windows(const StreamArgs& a) { return a.full_stride / (kFWin * a.full_g); }
__device__ __forceinline__ uint32_t* fs_table(const StreamArgs& a, int r, int k) {
    const int nW = fs_windows(a);
    return a.fs_tab + ((size_t)r * FS_TABLES + k) * (size_t)nW;
}
// The lane tables (kGLanes) after every row's tables: 64 uint4 per window
// (the lane's pair at the window's binade E, then at E + 1).
__device__ __forceinline__ uint4* fs_lanes(const StreamArgs& a, int r) {
    const size_t nW = (size_t)fs_windows(a);
    const size_t base = ((size_t)a.rows * FS_TABLES * nW + 3) & ~(size_t)3;
    return reinterpret_cast<uint4*>(a.fs_tab + base) + (size_t)r * nW * 64;
}

// k_fs_* blocks: kFsWaves waves, one window each.
constexpr int kFsWaves = 4;

template <int DT>
__global__ __launch_bounds__(64 * kFsWaves) void k_fs_max(StreamArgs a) {
    const int nW = fs_windows(a);
    const int gw = (int)blockIdx.x * kFsWaves + wave_id();
    const int r = gw / nW, w = gw - r * nW;
    if (r >= a.rows) return;
    const RowPlan P = plan_of(a, r);
    if (!(P.flags & RF_FPRE)) return;
    const int lane = lane_id(), V = a.vocab, G = a.full_g, WS = kFWin * G;
    float* fv = a.fullv + (size_t)r * a.full_stride;
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (DT == 0 ? 4 : 2);
    const uint32_t* mrow = (P.flags & RF_MASK) ? a.mask + (int64_t)r * a.mask_stride : nullptr;
    float mloc = -__builtin_inff(), lsum = 0.0f;
    bool nanv = false;
    int cnt = 0;
    // 16-byte loads where the row is aligned and the step lies inside it
    const bool al = (reinterpret_cast<uintptr_t>(rowp) & 15u) == 0u;
    for (int g = 0; g < G; ++g) {
        const int i0 = w * WS + g * kFWin + lane * 8;
        float x[8];
        uint32_t mw = 0xFFFFFFFFu;
        if (al && w * WS + (g + 1) * kFWin <= V) {
            if (DT == 0) {
                const float4 c0 = reinterpret_cast<const float4*>(rowp + (size_t)i0 * 4)[0];
                const float4 c1 = reinterpret_cast<const float4*>(rowp + (size_t)i0 * 4)[1];
                x[0] = c0.x; x[1] = c0.y; x[2] = c0.z; x[3] = c0.w;
                x[4] = c1.x; x[5] = c1.y; x[6] = c1.z; x[7] = c1.w;
            } else {
                const uint4 c = *reinterpret_cast<const uint4*>(rowp + (size_t)i0 * 2);
                const uint32_t h[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[2 * j] = __uint_as_float(h[j] << 16);
                    x[2 * j + 1] = __uint_as_float(h[j] & 0xFFFF0000u);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = load_logit<DT>(rowp, min(i0 + j, V - 1));
        }
        if (mrow != nullptr) mw = mrow[min(i0, V - 1) >> 5];   // (eight ids share one mask word)
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j;
            float v = -__builtin_inff();
            if (i < V) {
                v = x[j];
                if (!((mw >> (i & 31)) & 1u)) v = -__builtin_inff();
                v = v * P.inv_temp;
                if (v != v) {
                    nanv = true;
                    v = -__builtin_inff();
                }
            }
            y[j] = v;
            cnt += v != -__builtin_inff();
        }
        // this step's maximum and sum of exp(y - max), folded into the lane's
        // running pair (lmax, lsum)
        float sm = y[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) sm = fmaxf(sm, y[j]);
        if (sm != -__builtin_inff()) {
            float s8 = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) s8 += __expf(y[j] - sm);
            if (sm > mloc) {
                lsum = lsum * __expf(mloc - sm) + s8;
                mloc = sm;
            } else {
                lsum += s8 * __expf(sm - mloc);
            }
        }
        float4* dst = reinterpret_cast<float4*>(fv + i0);
        dst[0] = make_float4(y[0], y[1], y[2], y[3]);
        dst[1] = make_float4(y[4], y[5], y[6], y[7]);
    }
    const float mw = wave_max_f(mloc);
    float rel = mloc == -__builtin_inff() ? 0.0f : lsum * __expf(mloc - mw);
    rel = readlane_f(wave_tree_prefix_f(rel), 63);
    cnt = __builtin_amdgcn_readlane(wave_incl_sum_i(cnt), 63);
    const bool anynan = __ballot(nanv) != 0ull;
    if (lane == 0) {
        fs_table(a, r, FS_MAX)[w] = __float_as_uint(mw);
        fs_table(a, r, FS_NAN)[w] = anynan ? 1u : 0u;
        fs_table(a, r, FS_CNT)[w] = (uint32_t)cnt;
        fs_table(a, r, FS_A)[w] = __float_as_uint(rel);
    }
}

// k_fs_exp: each wave takes fs_run consecutive windows of a row (one pass
// over the row's window tables for all of them; a window's binade is
// predicted from the approximate sum before the wave's first window plus the
// approximate sums of the windows it has done): four when the batch has
// windows enough to keep every CU busy with a quarter of them, else one (a
// few rows: the latency of a wave's windows one after another would show).
__host__ __device__ __forceinline__ int fs_run(int rows, int nW) {
    return (int64_t)rows * nW >= 16384 ? 4 : 1;
}

__global__ __launch_bounds__(64 * kFsWaves) void k_fs_exp(StreamArgs a) {
    __shared__ uint64_t expT[32];
    if (threadIdx.x < 32) expT[threadIdx.x] = kExpT[threadIdx.x];
    __syncthreads();   // (the block's only barrier: the waves go their own ways below)
    const int nW = fs_windows(a);
    const int run = fs_run(a.rows, nW);
    const int nq = (nW + run - 1) / run;
    const int gw = (int)blockIdx.x * kFsWaves + wave_id();
    const int r = gw / nq, q = gw - r * nq;
    if (r >= a.rows) return;
    const RowPlan P = plan_of(a, r);
    if (!(P.flags & RF_FPRE)) return;
    const int lane = lane_id(), G = a.full_g, WS = kFWin * G;
    const int wb = q * run, we = min(wb + run, nW);
    const float* fv = a.fullv + (size_t)r * a.full_stride;
    float* pv = a.fullp + (size_t)r * a.full_stride;
    // the first window's first step in flight while the row's maximum is found
    float4 c0 = reinterpret_cast<const float4*>(fv + wb * WS + lane * 8)[0];
    float4 c1 = reinterpret_cast<const float4*>(fv + wb * WS + lane * 8)[1];
    // the row's maximum over the window maxima and, in the same reads, the
    // approximate sum before the first window from k_fs_max's window sums
    // relative to their own maxima (each lane's windows before wb rescaled to
    // its running maximum pm, then to m)
    const uint32_t* wm = fs_table(a, r, FS_MAX);
    const uint32_t* wa = fs_table(a, r, FS_A);
    float m = -__builtin_inff(), pm = -__builtin_inff(), ps = 0.0f;
    for (int k = lane; k < nW; k += 64) {
        const float mv = __uint_as_float(wm[k]);
        const float av = __uint_as_float(wa[k]);
        m = fmaxf(m, mv);
        if (k < wb && mv != -__builtin_inff()) {
            if (mv > pm) {
                ps = ps * __expf(pm - mv) + av;
                pm = mv;
            } else {
                ps += av * __expf(mv - pm);
            }
        }
    }
    m = wave_max_f(m);
    float pre = (pm == -__builtin_inff()) ? 0.0f : ps * __expf(pm - m);
    pre = readlane_f(wave_tree_prefix_f(pre), 63);
    // rows with top-p or min-p take the smallest numerator (top-p's key
    // range) and draw from sums of their own; the others the double sums
    const bool cut = (P.flags & (RF_TOPP | RF_MINP)) != 0;
    for (int w = wb; w < we; ++w) {
        const int E = w == 0 ? -126 : xs_binade(pre);
        float ws = 0.0f;
        double wd = 0.0;
        uint32_t emn = 0xFFFFFFFFu;
        XPair wp{0u, 0u};
        bool nz = false, lanes_on = false;
        for (int g = 0; g < G; ++g) {
            const int i0 = w * WS + g * kFWin + lane * 8;
            // the next step's (or window's) values in flight while these are worked on
            const bool more = g + 1 < G || w + 1 < we;
            const int in = more ? (g + 1 < G ? i0 + kFWin : (w + 1) * WS + lane * 8) : i0;
            const float4 n0 = reinterpret_cast<const float4*>(fv + in)[0];
            const float4 n1 = reinterpret_cast<const float4*>(fv + in)[1];
            const float x[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // (x = -inf: libm_expf_t(-inf) is +0; m = -inf, the whole row, decided once)
                v[j] = m == -__builtin_inff() ? 0.0f : libm_expf_t(x[j] - m, expT);
                ws += v[j];
            }
            if (cut) {
#pragma unroll
                for (int j = 0; j < 8; ++j) emn = min(emn, v[j] > 0.0f ? __float_as_uint(v[j]) : 0xFFFFFFFFu);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) wd += (double)v[j];
            }
            float4* dst = reinterpret_cast<float4*>(pv + i0);
            dst[0] = make_float4(v[0], v[1], v[2], v[3]);
            dst[1] = make_float4(v[4], v[5], v[6], v[7]);
            // the values' increments at E: plain (saturating) sums while no
            // value is half-way, the parity pairs in order otherwise
            bool tie = false;
            uint32_t ls = 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                bool t;
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
            if (G == 1) {
                // a window whose approximate end lies in a higher binade (or
                // within 0.1% below one) keeps its lanes' pairs at E and E + 1
                const float wsum = readlane_f(wave_tree_prefix_f(ws), 63);
                lanes_on = w > 0 && xs_binade((pre + wsum) * 1.001f) != E;
                if (lanes_on) {
                    XPair l1{0u, 0u};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        bool t;
                        l1 = xcomp(l1, xinc2f(v[j], E + 1, t));
                    }
                    fs_lanes(a, r)[(size_t)w * 64 + lane] = make_uint4(lp.d0, lp.d1, l1.d0, l1.d1);
                }
            }
            const XPair sp = wave_scan_pair_any(lp);
            wp = xcomp(wp, XPair{(uint32_t)__builtin_amdgcn_readlane((int)sp.d0, 63),
                                 (uint32_t)__builtin_amdgcn_readlane((int)sp.d1, 63)});
            c0 = n0;
            c1 = n1;
        }
        if (cut) {
            emn = wave_min_u32(emn);
            if (lane == 63) fs_table(a, r, FS_EMIN)[w] = emn;
        } else {
            wd = wave_tree_prefix_d(wd);
            if (lane == 63) reinterpret_cast<double*>(fs_table(a, r, FS_SD))[w] = wd;
        }
        const bool empty = __ballot(nz) == 0ull;
        if (lane == 0) {
            fs_table(a, r, FS_D0)[w] = wp.d0;
            fs_table(a, r, FS_D1)[w] = wp.d1;
            fs_table(a, r, FS_EF)[w] = gpack(E, (empty ? kGEmpty : 0u) | (lanes_on ? kGLanes : 0u));
        }
        pre += readlane_f(wave_tree_prefix_f(ws), 63);
    }
}

// ids[0, n) (n <= 64 Q, distinct) sorted ascending in place by one wave (a
// descending sort of their complements; the padding 0 stays last), and
// eb[q] = the bits of x[ids[q]].
template <int Q>
__device__ __forceinline__ void wave_ids_ascending(uint32_t* ids, int n, const float* x, uint32_t* eb) {
    const int lane = lane_id();
    uint32_t v[Q];
#pragma unroll
    for (int t = 0; t < Q; ++t) v[t] = t * 64 + lane < n ? ~ids[t * 64 + lane] : 0u;
    bsort_all<Q>(v);
    wave_sync();
#pragma unroll
    for (int t = 0; t < Q; ++t) {
        const int q = t * 64 + lane;
        if (q < n) {
            const uint32_t id = ~v[t];
            ids[q] = id;
            eb[q] = __float_as_uint(x[id]);
        }
    }
    wave_sync();
}

// Full-vocabulary rows, one block of kFT threads per row. PRE: the
// instantiations for the RF_FPRE rows (k_fs_* did the transform and left the
// window tables; no penalties, logit bias or top-k), PLAIN among them for the
// rows without top-p and min-p (the CLI's identity() + temperature: without
// those stages' code the kernel keeps its state in registers); the other one
// for the remaining full rows.
template <bool GT, bool PRE, bool PLAIN>
__global__ __launch_bounds__(kFT) void k_full(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ FullShared st;
    const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
    const int r = (int)blockIdx.x;
    if (r >= a.rows) return;
    const RowPlan P = plan_of(a, r);
    if (!(P.flags & RF_FULL) || PRE != ((P.flags & RF_FPRE) != 0)) return;
    if (PRE && PLAIN != ((P.flags & (RF_TOPP | RF_MINP)) == 0)) return;
    HSAMP_PHASE(12000 + r, 0);
    const int V = a.vocab, G = a.full_g;
    const int WS = kFWin * G;
    const int Vp = a.full_stride, nW = Vp / WS;
    float* fv = a.fullv + (size_t)r * Vp;
    float* pv = a.fullp + (size_t)r * Vp;
    const bool pen = !PRE && (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;
    const bool masked = !PRE && (P.flags & RF_MASK) != 0;
    const PenaltyLds pl = pen_table<GT>(a, r, smem);
    const FullLds f = full_lds(smem + (GT || PRE ? 0 : 8 * (size_t)a.mhash_slots));
    if (tid < 32) st.expT[tid] = kExpT[tid];
    if (tid == 0) {
        st.u = a.u[r];
        st.flags = 0;
    }
    if (pen) {
        // the row's penalty table (every id of the history window, bias ids)
        for (int i = tid; i < a.mhash_slots; i += kFT) {
            pl.hkey[i] = kEmpty;
            pl.hval[i] = 0u;
        }
        __syncthreads();
        const int L = hist_len_of(a, P, r), p0 = L - P.scan_len;
        const int32_t* h = a.hist + (int64_t)r * a.hist_stride;
        for (int p = p0 + tid; p < L; p += kFT) pen_add(a, P, L, p, h[p], pl);
        if (P.flags & RF_BIAS) {
            for (int j = tid; j < P.bias_cnt; j += kFT) {
                const uint32_t sl = pen_insert(a.bias_ids[P.bias_off + j], pl);
                atomicOr(&pl.hval[sl], HV_BIAS);
            }
        }
    }
    __syncthreads();
    HSAMP_PHASE(12000 + r, 1);
    uint32_t rflags = ROWF_U_USED;

    // ---- stages 1-6 (sampler.cpp:235-265): mask, penalties, temperature; max ----
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * (a.dtype == 0 ? 4 : 2);
    float mloc = -__builtin_inff();
    bool nanv = false;
    // Eight logits (and mask words) per thread in flight, then the ladder.
    // The loads take clamped ids and no condition, the element type and the
    // mask are template parameters: a load under a branch would be waited
    // for at the join, one memory round trip per load.
    auto transform = [&](auto dt_c, auto mask_c) {
        constexpr int DT = decltype(dt_c)::value;
        constexpr bool MK = decltype(mask_c)::value;
        const uint32_t* mrow = MK ? a.mask + (int64_t)r * a.mask_stride : nullptr;
        for (int b = tid; b < Vp; b += 8 * kFT) {
            float x[8];
            uint32_t mw[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int ic = min(b + q * kFT, V - 1);
                x[q] = load_logit<DT>(rowp, ic);
                mw[q] = MK ? mrow[ic >> 5] : 0xFFFFFFFFu;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int i = b + q * kFT;
                if (i >= Vp) break;
                float y = -__builtin_inff();
                if (i < V) {
                    y = x[q];
                    if (!((mw[q] >> (i & 31)) & 1u)) y = -__builtin_inff();
                    if (pen) {
                        uint32_t s0 = hslot(i, pl);
                        uint32_t kk;
                        while ((kk = tab_ld(&pl.hkey[s0])) != kEmpty && kk != (uint32_t)i) s0 = (s0 + 1) & pl.hmask;
                        if (kk == (uint32_t)i) y = pen_value(y, i, tab_ld(&pl.hval[s0]), a, P);
                    }
                    y = y * P.inv_temp;
                    if (y != y) {
                        nanv = true;
                        y = -__builtin_inff();
                    }
                }
                fv[i] = y;
                mloc = fmaxf(mloc, y);
            }
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using BT = std::integral_constant<bool, true>;
    using BF = std::integral_constant<bool, false>;
    constexpr bool pre = PRE;
    static_assert(kFMaxWin <= 2 * kFT, "two windows per thread");
    double sdr[2] = {0.0, 0.0};   // PRE: the draw's window sums of the numerators ...
    uint32_t cnr[2] = {0u, 0u};   // ... and counts (windows tid, tid + kFT)
    uint32_t emn = 0xFFFFFFFFu;   // PRE: the smallest numerator above 0 of those windows
    if constexpr (PRE) {
        // k_fs_* transformed the row and left its window tables, all loaded at
        // once: maxima and NaN flags for the row's maximum, the exact sum's
        // binades and pairs into LDS, the draw's sums and counts kept here
        const uint32_t* wm = fs_table(a, r, FS_MAX);
        const uint32_t* wn = fs_table(a, r, FS_NAN);
        const uint32_t* we = fs_table(a, r, FS_EF);
        const uint32_t* w0 = fs_table(a, r, FS_D0);
        const uint32_t* w1 = fs_table(a, r, FS_D1);
        const double* wsd = reinterpret_cast<const double*>(fs_table(a, r, FS_SD));
        const uint32_t* wcn = fs_table(a, r, FS_CNT);
        const uint32_t* wen = fs_table(a, r, FS_EMIN);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int k = tid + i * kFT;
            if (k < nW) {
                const uint32_t mx = wm[k], nn = wn[k], ef = we[k], d0 = w0[k], d1 = w1[k];
                sdr[i] = wsd[k];
                cnr[i] = wcn[k];
                if (!PLAIN) emn = min(emn, wen[k]);
                mloc = fmaxf(mloc, __uint_as_float(mx));
                nanv |= nn != 0u;
                f.winEF[k] = ef;
                f.winD0[k] = d0;
                f.winD1[k] = d1;
            }
        }
    } else if (a.dtype == 0) {
        if (masked) transform(I0{}, BT{});
        else transform(I0{}, BF{});
    } else {
        if (masked) transform(I1{}, BT{});
        else transform(I1{}, BF{});
    }
    if (nanv) atomicOr(&st.flags, 4);
    float m = fblock_max(mloc, st);
    HSAMP_PHASE(12000 + r, 2);

    // ---- top-k above kLimitK (sampler.cpp:109-121): the k-th largest key by four
    // 8-bit digit passes, ties to the lower ids ----
    if (!PRE && (P.flags & RF_TOPK)) {
        const int k = P.top_k;
        uint32_t prefix = 0u, kmask = 0u;
        int need = k;
        uint32_t* hist = f.bcnt;
        for (int shift = 24; shift >= 0; shift -= 8) {
            if (tid < 256) hist[tid] = 0u;
            __syncthreads();
            for (int i = tid; i < V; i += kFT) {
                const uint32_t key = key32(fv[i]);
                if ((key & kmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid < 64) {
                const int c0 = hist[255 - 4 * lane], c1 = hist[254 - 4 * lane];
                const int c2 = hist[253 - 4 * lane], c3 = hist[252 - 4 * lane];
                const int s4 = c0 + c1 + c2 + c3;
                const int incl = wave_incl_sum_i(s4);
                const int excl = incl - s4;
                if (excl < need && need <= incl) {
                    int q, before;
                    if (excl + c0 >= need) { q = 0; before = excl; }
                    else if (excl + c0 + c1 >= need) { q = 1; before = excl + c0; }
                    else if (excl + c0 + c1 + c2 >= need) { q = 2; before = excl + c0 + c1; }
                    else { q = 3; before = excl + c0 + c1 + c2; }
                    st.sel_d = 255 - 4 * lane - q;
                    st.sel_need = need - before;
                }
            }
            __syncthreads();
            prefix |= (uint32_t)st.sel_d << shift;
            kmask |= 0xFFu << shift;
            need = st.sel_need;
            __syncthreads();
        }
        // keep key > K and the `need` lowest ids with key == K; then the
        // finite members in index order (contiguous chunks per thread)
        const int C = (V + kFT - 1) / kFT;
        const int c0 = min(V, tid * C), c1 = min(V, c0 + C);
        int eq = 0;
        for (int i = c0; i < c1; ++i) eq += key32(fv[i]) == prefix;
        int tot;
        int before = fblock_excl_scan(eq, &tot, st);
        int fin = 0;
        for (int i = c0; i < c1; ++i) {
            const uint32_t key = key32(fv[i]);
            bool keep = key > prefix;
            if (key == prefix) keep = before++ < need;
            if (!keep) fv[i] = -__builtin_inff();
            else fin += fv[i] != -__builtin_inff();
        }
        int nfin;
        int pos = fblock_excl_scan(fin, &nfin, st);
        if (a.topk_idx != nullptr) {
            for (int i = c0; i < c1; ++i) {
                if (fv[i] == -__builtin_inff()) continue;
                if (pos < a.set_cap) a.topk_idx[(int64_t)r * a.set_cap + pos] = i;
                ++pos;
            }
        }
        if (tid == 0 && a.topk_count != nullptr) a.topk_count[r] = nfin;
        __syncthreads();
    } else if (tid == 0 && a.topk_count != nullptr) {
        a.topk_count[r] = -1;
    }

    int nkept = 0;
    int32_t tok = 0;
    // top-p's kept set as a predicate (p >= p*, when the cut keeps every id
    // with p* and no later stage removes ids), instead of writing -inf and 0
    // over the removed ids; kKeepAll when the arrays say what is left
    Keep keep = kKeepAll;
    bool listed = false;   // a small kept set's draw and outputs are done (ids in f.gath)
    // an id is left in: its transformed logit is above -inf (and the predicate keeps it)
    auto inset = [&](float e, float x, int i) -> bool {
        return keep.key != 0u ? keep(e, i) > 0.0f : x != -__builtin_inff();
    };
    if (m != -__builtin_inff()) {
        // ---- softmax numerators and their exact index-order sum (sampler.cpp:124-142) ----
        float S;
        if (pre) {
            // k_fs_exp left the numerators; its tables went to
            // LDS at the start (ordered by fblock_max's barriers)
            HSAMP_PHASE(12000 + r, 4);
            S = xs_value(exact_index_compose(pv, nW, G, f, st, fs_lanes(a, r)));
        } else {
            full_exp(fv, pv, m, nW, G, f, st);
            HSAMP_PHASE(12000 + r, 4);
            S = xs_value(exact_index_sum(pv, nW, G, f, st));
        }
        HSAMP_PHASE(12000 + r, 5);
        bool changed = false;   // a stage removed ids since S was taken
        bool touched = false;   // top-p or min-p removed ids
        int nleft = -1;         // ids left in (finite transformed logit) once a stage has counted them
        bool mk_same = true;    // the largest logit left in is still m
        int list_need = -1;     // top-p's candidates (p >= p*) fit one wave's list: the ids with p* it keeps
        uint32_t list_key = 0u; // ... and p*

        // ---- top-p (sampler.cpp:146-164) ----
        if (!PLAIN && (P.flags & RF_TOPP)) {
            uint32_t cut_key = 0u;
            int cut_count = 0, ngt = 0, neq = 0;
            const float inv = 1.0f / S;
            // the key range: from the smallest numerator above 0 (k_fs_exp's
            // window minima) to the largest, expf(0) = 1, whose p is inv
            uint32_t rlo = 0u, rhi = 0u;
            if (pre) {
                const float plo = __uint_as_float(fblock_min_u(emn, st)) * inv;
                if (plo > 0.0f) {
                    rlo = __float_as_uint(plo);
                    rhi = __float_as_uint(inv);
                }
            }
            if (full_top_p(pv, V, Vp, inv, P.top_p, f, st, rlo, rhi, &cut_key, &cut_count, &ngt, &neq)) {
                if (fabs(st.dS - (double)P.top_p) <= 1e-6) rflags |= ROWF_TOPP_NEAR;
                // kept: p > p*, and the lowest ids with p == p* up to cut_count
                const int need = cut_count - ngt;
                nleft = cut_count;
                // the largest logit's p is fl(1 * inv) = inv: it stays in unless
                // the cut falls among the ids with that p
                if (cut_key == __float_as_uint(inv) && need < neq) mk_same = false;
                if (!(P.flags & RF_MINP) && ngt + neq <= kFSort) {
                    // few candidates: the list below keeps the lowest `need` ids with p*
                    keep = Keep{inv, cut_key, 0x7FFFFFFF};
                    list_need = need;
                    list_key = cut_key;
                } else if (need >= neq && !(P.flags & RF_MINP)) {
                    keep = Keep{inv, cut_key, 0x7FFFFFFF};
                } else if (!(P.flags & RF_MINP) && mk_same && neq <= kFSort) {
                    // the cut splits the ids with p* (not the top ones): the
                    // lowest `need` of them by id stay; their ids, gathered and
                    // sorted, give the predicate's id limit
                    uint32_t* ids = f.gath;
                    if (tid == 0) st.sel_d = 0;
                    __syncthreads();
                    wpass(pv, nW, G, [&](int w, int g, const float (&e)[8]) {
                        int c = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) c += __float_as_uint(e[j] * inv) == cut_key;
                        const int incl = wave_incl_sum_i(c);
                        const int tot = __builtin_amdgcn_readlane(incl, 63);
                        if (tot == 0) return;
                        int base = 0;
                        if (lane == 0) base = atomicAdd(&st.sel_d, tot);
                        int pos = __builtin_amdgcn_readfirstlane(base) + incl - c;
                        const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            if (__float_as_uint(e[j] * inv) == cut_key) {
                                if (pos < kFSort) ids[pos] = (uint32_t)(i0 + j);
                                ++pos;
                            }
                    });
                    __syncthreads();
                    const int ne = min(st.sel_d, kFSort);
                    if (wid == 0) {
                        if (ne <= 64) wave_ids_ascending<1>(ids, ne, pv, f.sortb);
                        else if (ne <= 128) wave_ids_ascending<2>(ids, ne, pv, f.sortb);
                        else if (ne <= 256) wave_ids_ascending<4>(ids, ne, pv, f.sortb);
                        else wave_ids_ascending<8>(ids, ne, pv, f.sortb);
                        if (lane == 0) st.sel_need = (int)ids[min(need, ne) - 1] + 1;
                    }
                    __syncthreads();
                    keep = Keep{inv, cut_key, st.sel_need};
                } else if (need >= neq) {
                    fpass(pv, Vp, [&](int i, float e) {
                        if (__float_as_uint(e * inv) < cut_key) {
                            fv[i] = -__builtin_inff();
                            pv[i] = 0.0f;
                        }
                    });
                } else {
                    // equal keys at the cut, ranked by id: each window's count
                    // of them, the windows' prefix, then each one's rank
                    uint32_t* wc = f.winEF;
                    {
                        int c = 0;
                        wpass(pv, nW, G, [&](int w, int g, const float (&e)[8]) {
#pragma unroll
                            for (int j = 0; j < 8; ++j) c += __float_as_uint(e[j] * inv) == cut_key;
                            if (g == G - 1) {
                                c = __builtin_amdgcn_readlane(wave_incl_sum_i(c), 63);
                                if (lane == 0) wc[w] = (uint32_t)c;
                                c = 0;
                            }
                        });
                    }
                    __syncthreads();
                    {
                        const int w0 = 2 * tid;
                        const int c0 = w0 < nW ? (int)wc[w0] : 0, c1 = w0 + 1 < nW ? (int)wc[w0 + 1] : 0;
                        int tot;
                        const int ex = fblock_excl_scan(c0 + c1, &tot, st);
                        if (w0 < nW) wc[w0] = (uint32_t)ex;
                        if (w0 + 1 < nW) wc[w0 + 1] = (uint32_t)(ex + c0);
                    }
                    __syncthreads();
                    int pos = 0;
                    wpass(pv, nW, G, [&](int w, int g, const float (&e)[8]) {
                        if (g == 0) pos = (int)wc[w];
                        int c = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) c += __float_as_uint(e[j] * inv) == cut_key;
                        const int li = wave_incl_sum_i(c);
                        int rank = pos + li - c;
                        const size_t i0 = (size_t)w * WS + g * kFWin + lane * 8;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t key = __float_as_uint(e[j] * inv);
                            const bool keep = key > cut_key || (key == cut_key && rank < need);
                            rank += key == cut_key;
                            if (!keep) {
                                fv[i0 + j] = -__builtin_inff();
                                pv[i0 + j] = 0.0f;
                            }
                        }
                        pos += __builtin_amdgcn_readlane(li, 63);
                    });
                }
                changed = true;
                touched = true;
                __syncthreads();
            }
        }

        // A small kept set (top-p's candidates, p >= p*, at most 512 ids): the
        // candidates are gathered and sorted by id, the lowest `need` with p*
        // kept, and the rest is done on the list by wave 0 -- the largest kept
        // logit (and the numerators again when it is below m), the exact
        // index-order sum of the numerators (float adds), the draw and the kept
        // ids -- with no more passes over the row.
        if (list_need >= 0) {
            uint32_t* ids = f.gath;   // (the window and bucket tables are free now)
            if (tid == 0) st.sel_d = 0;
            __syncthreads();
            wpass(pv, nW, G, [&](int w, int g, const float (&e)[8]) {
                int c = 0;
                const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                for (int j = 0; j < 8; ++j) c += keep(e[j], i0 + j) > 0.0f;
                const int incl = wave_incl_sum_i(c);
                const int tot = __builtin_amdgcn_readlane(incl, 63);
                if (tot == 0) return;
                int base = 0;
                if (lane == 0) base = atomicAdd(&st.sel_d, tot);
                int pos = __builtin_amdgcn_readfirstlane(base) + incl - c;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (keep(e[j], i0 + j) > 0.0f) {
                        if (pos < kFSort) ids[pos] = (uint32_t)(i0 + j);
                        ++pos;
                    }
            });
            __syncthreads();
            const int n0 = min(st.sel_d, kFSort);
            if (wid == 0) {
                // ids ascending, their numerators beside them
                uint32_t* eb = f.sortb;
                if (n0 <= 64) wave_ids_ascending<1>(ids, n0, pv, eb);
                else if (n0 <= 128) wave_ids_ascending<2>(ids, n0, pv, eb);
                else if (n0 <= 256) wave_ids_ascending<4>(ids, n0, pv, eb);
                else wave_ids_ascending<8>(ids, n0, pv, eb);
                // the candidates with p* past the first `need` of them leave;
                // the largest kept logit m'; the rest close ranks
                uint32_t li_[8], le_[8];
                bool kq[8];
                int ce = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = lane * 8 + j;
                    li_[j] = q < n0 ? ids[q] : 0u;
                    le_[j] = q < n0 ? eb[q] : 0u;
                    ce += q < n0 && __float_as_uint(__uint_as_float(le_[j]) * keep.inv) == list_key;
                }
                int eqr = wave_incl_sum_i(ce) - ce;   // equal keys before this lane's first entry
                int ck = 0;
                float mk = -__builtin_inff();
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = lane * 8 + j;
                    const bool eq = q < n0 && __float_as_uint(__uint_as_float(le_[j]) * keep.inv) == list_key;
                    kq[j] = q < n0 && (!eq || eqr < list_need);
                    eqr += eq;
                    ck += kq[j];
                    if (kq[j]) mk = fmaxf(mk, fv[li_[j]]);
                }
                mk = wave_max_f(mk);
                int kpos = wave_incl_sum_i(ck) - ck;
                wave_sync();
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (kq[j]) {
                        uint32_t e = le_[j];
                        // numerators relative to m' when the cut left the maximum out
                        if (mk != m) e = __float_as_uint(libm_expf_t(fv[li_[j]] - mk, st.expT));
                        ids[kpos] = li_[j];
                        eb[kpos] = e;
                        ++kpos;
                    }
                }
                const int n = __builtin_amdgcn_readlane(kpos, 63);
                wave_sync();
                XState s2{-126, 0u};
                chain_replay(s2, eb, n, __builtin_inff());
                const float inv2 = 1.0f / xs_value(s2);
                // the draw (sampler.cpp:178-182): q = p / S_d over the kept ids in index order
                float pq[8];
                int32_t iq[8];
                double ls = 0.0;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = lane * 8 + j;
                    pq[j] = q < n ? __uint_as_float(eb[q]) * inv2 : 0.0f;
                    iq[j] = q < n ? (int32_t)ids[q] : -1;
                    ls += (double)pq[j];
                }
                const double li = wave_tree_prefix_d(ls);
                const double Sd = readlane_d(li, 63);
                const double u = st.u;
                int tk = V - 1;   // no running sum reaches u: cp[V - 1] = 1 takes it
                double dS = -1.0;
                if (!(u > 0.0)) {
                    tk = 0;
                } else {
                    double c = li - ls, cat = 0.0, pat = 0.0;
                    int first = 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const double qj = (double)pq[j] / Sd;
                        const double before = c;
                        c = c + qj;
                        const double cc = (iq[j] == V - 1) ? 1.0 : c;
                        if (first == 8 && iq[j] >= 0 && qj > 0.0 && cc >= u) {
                            first = j;
                            cat = cc;
                            pat = before;
                        }
                    }
                    const u64 hm = __ballot(first < 8);
                    if (hm != 0ull) {
                        const int L = __ffsll((long long)hm) - 1;
                        int sel = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) sel = j == first ? iq[j] : sel;
                        tk = __builtin_amdgcn_readlane(sel, L);
                        dS = readlane_d(fmin(fabs(cat - u), fabs(pat - u)), L);
                    } else {
                        dS = fmin(fabs(1.0 - u), fabs(readlane_d(c, 63) - u));
                    }
                }
                if (a.kept_idx != nullptr) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = lane * 8 + j;
                        if (q < n && q < a.set_cap) {
                            a.kept_idx[(int64_t)r * a.set_cap + q] = iq[j];
                            a.kept_prob[(int64_t)r * a.set_cap + q] = pq[j];
                        }
                    }
                }
                if (lane == 0) {
                    st.tok = tk;
                    st.dS = dS;
                    st.sel_need = n;
                }
            }
            __syncthreads();
            tok = st.tok;
            if (st.dS >= 0.0 && st.dS <= 1e-6) rflags |= ROWF_CDF_NEAR;
            nkept = st.sel_need;
            listed = true;
            changed = false;
        }

        // the numerators of what is left: relative to the largest kept logit
        // (the maximum unless a tie in p kept a lower id first), window sums
        // (PRE rows: also each window's kept numerators summed in double and
        // counted, in the FS_SD / FS_CNT tables, for the draw: fresh)
        bool fresh = false;
        auto refresh = [&]() {
            float mk = m;
            if (nleft == 0) {
                mk = -__builtin_inff();
            } else if (!mk_same) {
                mk = -__builtin_inff();
                fpass(fv, Vp, [&](int, float x) { mk = fmaxf(mk, x); });
                mk = fblock_max(mk, st);
            }
            mk_same = true;
            if (mk == -__builtin_inff()) {
                m = mk;
                return;
            }
            if (mk != m) {
                m = mk;
                full_exp(fv, pv, m, nW, G, f, st);
            } else {
                float ws = 0.0f;
                double wd = 0.0;
                int wn = 0;
                wpass(pv, nW, G, [&](int w, int g, const float (&u)[8]) {
                    float v[8];
                    const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        v[j] = keep(u[j], i0 + j);
                        if (pre) {
                            wd += (double)v[j];
                            wn += v[j] > 0.0f;
                        }
                    }
                    if (!pre) ws += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                    if (g == G - 1) {
                        if (pre) {
                            // (the double sum, rounded, is the window's approximate sum)
                            wd = wave_tree_prefix_d(wd);
                            wn = wave_incl_sum_i(wn);
                            if (lane == 63) {
                                reinterpret_cast<double*>(fs_table(a, r, FS_SD))[w] = wd;
                                fs_table(a, r, FS_CNT)[w] = (uint32_t)wn;
                                f.winA[w] = (float)wd;
                            }
                        } else {
                            ws = wave_tree_prefix_f(ws);
                            if (lane == 63) f.winA[w] = ws;
                        }
                        ws = 0.0f;
                        wd = 0.0;
                        wn = 0;
                    }
                });
                fresh = pre;
                __syncthreads();
            }
            S = xs_value(exact_index_sum(pv, nW, G, f, st, keep, pre ? fs_lanes(a, r) : nullptr));
        };

        // ---- min-p (sampler.cpp:167-176) ----
        if (!PLAIN && (P.flags & RF_MINP)) {
            if (changed) refresh();
            changed = false;
            const float inv = 1.0f / S;
            // (a threshold of 0 -- min_p * inv below the smallest float -- removes nothing)
            if (m != -__builtin_inff() && P.min_p * inv > 0.0f) {
                if (nleft < 0) {
                    // the ids in before min-p: the finite transformed logits
                    int c = 0;
                    if (pre) {
                        c = (int)(cnr[0] + cnr[1]);
                    } else {
                        fpass(fv, Vp, [&](int, float x) { c += x != -__builtin_inff(); });
                    }
                    nleft = fblock_sum_i(c, st);
                }
                // the largest p is the largest logit's, fl(1 * inv) = inv; the
                // ids left in are those with p >= thr > 0 (a removed id's p is 0)
                const float thr = P.min_p * inv;
                int left = 0;
                fpass(pv, Vp, [&](int i, float e) {
                    if (e * inv < thr) {
                        fv[i] = -__builtin_inff();
                        pv[i] = 0.0f;
                    } else {
                        ++left;
                    }
                });
                left = fblock_sum_i(left, st);
                changed = left != nleft;
                nleft = left;
                touched |= changed;
            }
        }
        HSAMP_PHASE(12000 + r, 6);
        if (changed) refresh();
        HSAMP_PHASE(12000 + r, 7);
        if (m != -__builtin_inff() && !listed) {
            // ---- the draw (sampler.cpp:178-182, discrete_distribution) ----
            // p = e * fl(1/S); S_d = sum of p (double); q = p / S_d; the first id
            // whose running sum of q reaches u (the last id's is 1). One pass
            // gives each window's sum of p and its kept count; the window where
            // the running sum reaches u is then walked value by value.
            const float inv = 1.0f / S;
            double* wq = reinterpret_cast<double*>(f.winA);   // [kFMaxWin] window sums of p, then prefixes
            uint32_t* wc = f.winEF;                            // [kFMaxWin] kept counts, then prefixes
            if (pre && !touched && !(P.flags & (RF_TOPP | RF_MINP))) {
                // k_fs_* left each window's numerators summed in double and
                // its count: the window sums of p are taken as fl(1/S) times
                // those (within 2^-24 of the sums of fl(e fl(1/S)) relative,
                // where CDF_NEAR's 1e-6 flags every draw they could move)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int k = tid + i * kFT;
                    if (k < nW) {
                        wq[k] = (double)inv * sdr[i];
                        wc[k] = cnr[i];
                    }
                }
            } else if (fresh && (keep.key != 0u || a.kept_idx == nullptr)) {
                // the refresh left each window's kept numerators summed in
                // double and counted: the window sums of p as fl(1/S) times
                // those (as above)
                const double* wsd = reinterpret_cast<const double*>(fs_table(a, r, FS_SD));
                const uint32_t* wcn = fs_table(a, r, FS_CNT);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int k = tid + i * kFT;
                    if (k < nW) {
                        wq[k] = (double)inv * wsd[k];
                        wc[k] = wcn[k];
                    }
                }
            } else if (touched && a.kept_idx == nullptr) {
                // top-p / min-p counted the ids left in (nleft); the window
                // sums of p from the numerators alone
                double ws = 0.0;
                wpass(pv, nW, G, [&](int w, int g, const float (&e)[8]) {
                    const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) ws += (double)(keep(e[j], i0 + j) * inv);
                    if (g == G - 1) {
                        ws = wave_sum_d(ws);
                        if (lane == 0) {
                            wq[w] = ws;
                            wc[w] = 0u;
                        }
                        ws = 0.0;
                    }
                });
            } else {
                double ws = 0.0;
                int c = 0;
                wpass2(pv, fv, nW, G, [&](int w, int g, const float (&e)[8], const float (&x)[8]) {
                    const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        ws += (double)(keep(e[j], i0 + j) * inv);
                        c += inset(e[j], x[j], i0 + j);
                    }
                    if (g == G - 1) {
                        ws = wave_sum_d(ws);
                        c = __builtin_amdgcn_readlane(wave_incl_sum_i(c), 63);
                        if (lane == 0) {
                            wq[w] = ws;
                            wc[w] = (uint32_t)c;
                        }
                        ws = 0.0;
                        c = 0;
                    }
                });
            }
            __syncthreads();
            HSAMP_PHASE(12000 + r, 8);
            if (tid == 0) {
                st.tok = V - 1;   // no running sum reaches u: cp[V - 1] = 1 takes it
                st.dS = -1.0;
                st.fgroup = nW - 1;
            }
            const double u = st.u;
            double Sd;
            {
                // exclusive prefixes over the windows, 2 per thread
                const int w0 = 2 * tid;
                const double q0 = w0 < nW ? wq[w0] : 0.0, q1 = w0 + 1 < nW ? wq[w0 + 1] : 0.0;
                const int c0 = w0 < nW ? (int)wc[w0] : 0, c1 = w0 + 1 < nW ? (int)wc[w0 + 1] : 0;
                const double incl = wave_tree_prefix_d(q0 + q1);
                if (lane == 63) st.rd[wid] = incl;
                int tot;
                const int cex = fblock_excl_scan(c0 + c1, &tot, st);   // (its barriers publish st.rd)
                nkept = (touched && a.kept_idx == nullptr) ? nleft : tot;
                double base = 0.0;
                Sd = 0.0;
                for (int i = 0; i < kFW; ++i) {
                    base += (i < wid) ? st.rd[i] : 0.0;
                    Sd += st.rd[i];
                }
                const double ex = base + incl - (q0 + q1);
                __syncthreads();
                if (w0 < nW) {
                    wq[w0] = ex;
                    wc[w0] = (uint32_t)cex;
                }
                if (w0 + 1 < nW) {
                    wq[w0 + 1] = ex + q0;
                    wc[w0 + 1] = (uint32_t)(cex + c0);
                }
                // the first window whose end reaches u (by its prefix of p /
                // S_d): one candidate per wave
                if (u > 0.0) {
                    const bool h0 = w0 < nW && ((w0 + 1 < nW) ? (ex + q0) / Sd : 2.0) >= u;
                    const bool h1 = w0 + 1 < nW && ((w0 + 2 < nW) ? (ex + q0 + q1) / Sd : 2.0) >= u;
                    const u64 hm = __ballot(h0 || h1);
                    if (hm != 0ull && lane == __ffsll((long long)hm) - 1) atomicMin(&st.fgroup, h0 ? w0 : w0 + 1);
                }
            }
            __syncthreads();
            HSAMP_PHASE(12000 + r, 9);
            if (!(u > 0.0)) {
                tok = 0;
            } else {
                HSAMP_PHASE(12000 + r, 10);
                if (G == 1) {
                    // from a window before it (the prefixes are sums in another
                    // order), sixteen windows at a time, one per wave: each from
                    // its prefix, the first window where a running sum of q
                    // reaches u gives the id
                    for (int base = max(0, st.fgroup - 1); base < nW; base += kFW) {
                        const int w = base + wid;
                        int wt = -1;
                        double wd = 0.0, cpe = 0.0;
                        if (w < nW) {
                            const double cp = wq[w] / Sd;
                            const int i0 = w * WS + lane * 8;
                            const float4 e0 = reinterpret_cast<const float4*>(pv + i0)[0];
                            const float4 e1 = reinterpret_cast<const float4*>(pv + i0)[1];
                            const float e[8] = {keep(e0.x, i0), keep(e0.y, i0 + 1), keep(e0.z, i0 + 2),
                                                keep(e0.w, i0 + 3), keep(e1.x, i0 + 4), keep(e1.y, i0 + 5),
                                                keep(e1.z, i0 + 6), keep(e1.w, i0 + 7)};
                            double q[8], ls = 0.0;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                q[j] = (double)(e[j] * inv) / Sd;
                                ls += q[j];
                            }
                            const double li = wave_tree_prefix_d(ls);
                            double c = cp + (li - ls), cat = 0.0, pat = 0.0;
                            int first = 8;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const double before = c;
                                c = c + q[j];
                                const int i = i0 + j;
                                const double cc = (i == V - 1) ? 1.0 : c;
                                if (first == 8 && i < V && q[j] > 0.0 && cc >= u) {
                                    first = j;
                                    cat = cc;
                                    pat = before;
                                }
                            }
                            const u64 hm = __ballot(first < 8);
                            if (hm != 0ull) {
                                const int L = __ffsll((long long)hm) - 1;
                                wt = __builtin_amdgcn_readlane(i0 + first, L);
                                wd = readlane_d(fmin(fabs(cat - u), fabs(pat - u)), L);
                            }
                            cpe = cp + readlane_d(li, 63);
                        }
                        if (lane == 0) {
                            st.wtok[wid] = wt;
                            st.wds[wid] = wd;
                            st.wcp[wid] = cpe;
                        }
                        __syncthreads();
                        HSAMP_PHASE(12000 + r, 3);
                        int k = 0;
                        while (k < kFW && st.wtok[k] < 0) ++k;
                        const bool last = base + kFW >= nW;
                        if (tid == 0) {
                            if (k < kFW) {
                                st.tok = st.wtok[k];
                                st.dS = st.wds[k];
                            } else if (last) {
                                st.dS = fmin(fabs(1.0 - u), fabs(st.wcp[nW - 1 - base] - u));
                            }
                        }
                        __syncthreads();
                        if (k < kFW) break;
                    }
                } else if (wid == 0) {
                    // walk from a window before it (the prefixes are sums in
                    // another order) until a running sum of q reaches u
                    int w = max(0, st.fgroup - 1);
                    bool hit = false;
                    double cp = wq[w] / Sd;
                    for (; w < nW && !hit; ++w) {
                        cp = wq[w] / Sd;
                        for (int g = 0; g < G && !hit; ++g) {
                            const int i0 = w * WS + g * kFWin + lane * 8;
                            const float* src = pv + i0;
                            double q[8], ls = 0.0;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                q[j] = (double)(keep(src[j], i0 + j) * inv) / Sd;
                                ls += q[j];
                            }
                            const double li = wave_tree_prefix_d(ls);
                            double c = cp + (li - ls), prev = c, cat = 0.0, pat = 0.0;
                            int first = 8;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const double before = c;
                                c = c + q[j];
                                const int i = i0 + j;
                                const double cc = (i == V - 1) ? 1.0 : c;
                                if (first == 8 && i < V && q[j] > 0.0 && cc >= u) {
                                    first = j;
                                    cat = cc;
                                    pat = before;
                                }
                            }
                            (void)prev;
                            const u64 hm = __ballot(first < 8);
                            if (hm != 0ull) {
                                const int L = __ffsll((long long)hm) - 1;
                                if (lane == L) {
                                    st.tok = i0 + first;
                                    st.dS = fmin(fabs(cat - u), fabs(pat - u));
                                }
                                hit = true;
                            }
                            cp = cp + readlane_d(li, 63);
                        }
                    }
                    if (!hit && lane == 0) st.dS = fmin(fabs(1.0 - u), fabs(cp - u));
                }
                __syncthreads();
                tok = st.tok;
                if (st.dS >= 0.0 && st.dS <= 1e-6) rflags |= ROWF_CDF_NEAR;
            }
            HSAMP_PHASE(12000 + r, 11);
            // kept ids and probabilities in index order
            if (a.kept_idx != nullptr) {
                int pos = 0;
                wpass2(pv, fv, nW, G, [&](int w, int g, const float (&e)[8], const float (&x)[8]) {
                    if (g == 0) pos = (int)wc[w];
                    int c = 0;
                    const int i0 = w * WS + g * kFWin + lane * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j) c += inset(e[j], x[j], i0 + j);
                    const int li = wave_incl_sum_i(c);
                    int p = pos + li - c;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if (inset(e[j], x[j], i0 + j)) {
                            if (p < a.set_cap) {
                                a.kept_idx[(int64_t)r * a.set_cap + p] = i0 + j;
                                a.kept_prob[(int64_t)r * a.set_cap + p] = e[j] * inv;
                            }
                            ++p;
                        }
                    }
                    pos += __builtin_amdgcn_readlane(li, 63);
                });
            }
        }
    }
    HSAMP_PHASE(12000 + r, 12);
    if (nkept == 0) {
        rflags |= ROWF_UNIFORM;
        if (tid == 0) tok = uniform_draw(V, st.u);
    }
    // the state sample() leaves the logits in (f32 only)
    if (a.fin_idx != nullptr) {
        float* row = static_cast<float*>(const_cast<void*>(a.logits)) + (int64_t)r * a.logits_stride;
        if (listed) {
            // the kept ids (the list in f.gath, nkept of them) over -inf
            for (int i = tid; i < V; i += kFT) row[i] = -__builtin_inff();
            __syncthreads();
            for (int q = tid; q < nkept; q += kFT) row[f.gath[q]] = fv[f.gath[q]];
        } else if (keep.key != 0u) {
            for (int i = tid; i < V; i += kFT) row[i] = keep(pv[i], i) > 0.0f ? fv[i] : -__builtin_inff();
        } else {
            for (int i = tid; i < V; i += kFT) row[i] = fv[i];
        }
    }
    if (wid == 0) emit_token_wave(a, r, tok);
    if (tid == 0) {
        if (a.row_flags != nullptr) a.row_flags[r] = rflags | ((st.flags & 4) ? ROWF_NAN : 0u);
        if (a.kept_count != nullptr) a.kept_count[r] = nkept;
    }
    HSAMP_PHASE(12000 + r, 13);
}

// ---- diagnostics: a plain read with the stream kernel's launch shape --------------

// The same grid, block-to-slice mapping, buffer resources and 16-byte
// non-temporal loads as the exact-list k_stream (aligned rows), and nothing
// else: each block reads its slice, takes the maximum and writes it to
// out[logical block]. Its duration is the floor any pass over these bytes
// with this launch shape can reach.
template <int DT, int NT>
__global__ __launch_bounds__(kBlock) void k_read_probe(StreamArgs a, float* out) {
    using T = Tile<DT>;
    constexpr int NC = T::NCH * NT;
    __shared__ float red[kBlock / 64];
    const uint32_t bid = blockIdx.x;
    const int logical = (int)(bid % kXcds) * a.blocks_per_xcd + (int)(bid / kXcds);
    const int r = div_slices(logical, a), s = logical - r * a.nslices;
    if (r >= a.rows) return;
    const int lo = s * a.slice_len;
    const int hi = min(a.vocab - a.vec_tail, lo + a.slice_len);
    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * T::ES;
    uint4 raw[NC];
    load_tile<DT, true, NC>(row_rsrc(rowp, hi, T::ES), lo, raw);
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int c = 0; c < T::VW; ++c) m = fmaxf(m, elem<DT>(raw[j], c));
    m = wave_max_f(m);
    if (lane_id() == 0) red[wave_id()] = m;
    __syncthreads();
    if (threadIdx.x == 0) out[logical] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

hipError_t launch_read_probe(const StreamArgs& a, int dtype, int tiles, int grid, float* out, hipStream_t stream) {
    const dim3 g(grid), b(kBlock);
    if (tiles == 1) {
        if (dtype == 0) hipLaunchKernelGGL((k_read_probe<0, 1>), g, b, 0, stream, a, out);
        else hipLaunchKernelGGL((k_read_probe<1, 1>), g, b, 0, stream, a, out);
    } else if (tiles == 2) {
        if (dtype == 0) hipLaunchKernelGGL((k_read_probe<0, 2>), g, b, 0, stream, a, out);
        else hipLaunchKernelGGL((k_read_probe<1, 2>), g, b, 0, stream, a, out);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- launchers -------------------------------------------------------------------

template <bool GR>
static void launch_stream_kind(const StreamArgs& a, int dtype, bool vec, bool pen, bool mask, int grid,
                               hipStream_t stream) {
    const dim3 g(grid), b(kBlock);
    const uint32_t l = a.lds_bytes;
#define HSAMP_STREAM(DT_, V_, P_, M_) hipLaunchKernelGGL((k_stream<DT_, V_, P_, M_, GR>), g, b, l, stream, a)
    if (!vec) {   // unaligned rows: one general kernel per element type
        if (dtype == 0) HSAMP_STREAM(0, false, true, true);
        else HSAMP_STREAM(1, false, true, true);
    } else if (dtype == 0) {
        if (pen) {
            if (mask) HSAMP_STREAM(0, true, true, true);
            else HSAMP_STREAM(0, true, true, false);
        } else {
            if (mask) HSAMP_STREAM(0, true, false, true);
            else HSAMP_STREAM(0, true, false, false);
        }
    } else {
        if (pen) {
            if (mask) HSAMP_STREAM(1, true, true, true);
            else HSAMP_STREAM(1, true, true, false);
        } else {
            if (mask) HSAMP_STREAM(1, true, false, true);
            else HSAMP_STREAM(1, true, false, false);
        }
    }
#undef HSAMP_STREAM
}

// Exact lists: the sampling kernel with final keys (every row samples), slices
// of one tile, or of two (aligned rows), or of four (aligned bf16 rows).
// LEAN: the launch has no greedy rows, no logit bias and one count window per
// row (see stream_exact).
template <int NT, bool LEAN>
static void launch_stream_exact(const StreamArgs& a, int dtype, bool vec, bool pen, bool mask, int grid,
                                hipStream_t stream) {
    const dim3 g(grid), b(kBlock);
    const uint32_t l = a.lds_bytes;
#define HSAMP_STREAM(DT_, V_, P_, M_) hipLaunchKernelGGL((k_stream<DT_, V_, P_, M_, false, NT, LEAN>), g, b, l, stream, a)
    if (!vec) {
        if constexpr (NT == 1) {
            if (dtype == 0) HSAMP_STREAM(0, false, true, true);
            else HSAMP_STREAM(1, false, true, true);
        }
    } else if (dtype == 0) {
        if constexpr (NT <= 2) {   // (four f32 tiles would not fit the registers)
            if (pen) {
                if (mask) HSAMP_STREAM(0, true, true, true);
                else HSAMP_STREAM(0, true, true, false);
            } else {
                if (mask) HSAMP_STREAM(0, true, false, true);
                else HSAMP_STREAM(0, true, false, false);
            }
        }
    } else {
        if (pen) {
            if (mask) HSAMP_STREAM(1, true, true, true);
            else HSAMP_STREAM(1, true, true, false);
        } else {
            if (mask) HSAMP_STREAM(1, true, false, true);
            else HSAMP_STREAM(1, true, false, false);
        }
    }
#undef HSAMP_STREAM
}

hipError_t launch_stream_ex(const StreamArgs& a, int dtype, bool vec, bool pen, bool mask, int tiles, bool lean,
                            int grid, hipStream_t stream) {
    // two-tile slices are for aligned rows only (the host never asks otherwise)
    // (four-tile slices: aligned bf16 rows only, whose four tiles take the
    // registers two f32 tiles take)
    if (tiles > 1 && !vec) return hipErrorInvalidValue;
    if (tiles == 4 && dtype == 0) return hipErrorInvalidValue;
    if (lean) {
        if (tiles == 4) launch_stream_exact<4, true>(a, dtype, vec, pen, mask, grid, stream);
        else if (tiles == 2) launch_stream_exact<2, true>(a, dtype, vec, pen, mask, grid, stream);
        else launch_stream_exact<1, true>(a, dtype, vec, pen, mask, grid, stream);
    } else {
        if (tiles == 4) launch_stream_exact<4, false>(a, dtype, vec, pen, mask, grid, stream);
        else if (tiles == 2) launch_stream_exact<2, false>(a, dtype, vec, pen, mask, grid, stream);
        else launch_stream_exact<1, false>(a, dtype, vec, pen, mask, grid, stream);
    }
    return hipGetLastError();
}

// Blocks of the per-row kernels: kXcds times the most rows whose first slice
// one XCD streamed (each row is merged on that XCD).
static int row_blocks(const StreamArgs& a) {
    int most = 0;
    for (int x = 0; x < kXcds; ++x) {
        const int r0 = std::min(a.rows, (x * a.blocks_per_xcd + a.nslices - 1) / a.nslices);
        const int r1 = std::min(a.rows, ((x + 1) * a.blocks_per_xcd + a.nslices - 1) / a.nslices);
        most = std::max(most, r1 - r0);
    }
    return kXcds * most;
}

hipError_t launch_pick(const StreamArgs& a, int nw, hipStream_t stream) {
    const dim3 g(row_blocks(a)), b(kBlock);
    switch (nw) {
        case 4: hipLaunchKernelGGL((k_pick<4>), g, b, a.merge_lds, stream, a); break;
        case 8: hipLaunchKernelGGL((k_pick<8>), g, b, a.merge_lds, stream, a); break;
        case 12: hipLaunchKernelGGL((k_pick<12>), g, b, a.merge_lds, stream, a); break;
        default: hipLaunchKernelGGL((k_pick<16>), g, b, a.merge_lds, stream, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_pick_l(const StreamArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(k_pick_l, dim3(row_blocks(a)), dim3(kBlock), a.merge_lds, stream, a);
    return hipGetLastError();
}

#ifdef HSAMP_PHASE_CLOCKS
extern "C" int hsamp_phase_read(void* dst, size_t bytes) {
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_phase), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_stream(const StreamArgs& a, int dtype, bool vec, bool pen_greedy, bool pen_sample, bool mask,
                         bool greedy_rows, bool sample_rows, int grid, hipStream_t stream) {
    if (greedy_rows) launch_stream_kind<true>(a, dtype, vec, pen_greedy, mask, grid, stream);
    if (sample_rows) launch_stream_kind<false>(a, dtype, vec, pen_sample, mask, grid, stream);
    return hipGetLastError();
}

hipError_t launch_merge(const StreamArgs& a, hipStream_t stream) {
    const dim3 g(row_blocks(a));
    if (a.fast && a.pen_flag) hipLaunchKernelGGL((k_merge<false, true, true>), g, dim3(kBlock), a.merge_lds, stream, a);
    else if (a.fast) hipLaunchKernelGGL((k_merge<false, true, false>), g, dim3(kBlock), a.merge_lds, stream, a);
    else if (a.gtab != nullptr) hipLaunchKernelGGL((k_merge<true, false, false>), g, dim3(kBlock), a.merge_lds, stream, a);
    else hipLaunchKernelGGL((k_merge<false, false, false>), g, dim3(kBlock), a.merge_lds, stream, a);
    return hipGetLastError();
}

// The RF_FPRE rows: k_fs_max, k_fs_exp over B x nW waves, then
// k_full's PRE instantiations (no penalty table in their LDS): PLAIN for the
// rows without top-p and min-p (plain), the other for the rows with them (tp).
hipError_t launch_full_pre(const StreamArgs& a, bool plain, bool tp, hipStream_t stream) {
    const int nW = a.full_stride / (kFWin * a.full_g);
    const dim3 g((unsigned)(((int64_t)a.rows * nW + kFsWaves - 1) / kFsWaves)), b(64 * kFsWaves);
    if (a.dtype == 0) hipLaunchKernelGGL((k_fs_max<0>), g, b, 0, stream, a);
    else hipLaunchKernelGGL((k_fs_max<1>), g, b, 0, stream, a);
    const int run = fs_run(a.rows, nW), nq = (nW + run - 1) / run;
    const dim3 ge((unsigned)(((int64_t)a.rows * nq + kFsWaves - 1) / kFsWaves));
    hipLaunchKernelGGL(k_fs_exp, ge, b, 0, stream, a);
    if (plain) hipLaunchKernelGGL((k_full<false, true, true>), dim3(a.rows), dim3(kFT), (uint32_t)kFullLdsBytes, stream, a);
    if (tp) hipLaunchKernelGGL((k_full<false, true, false>), dim3(a.rows), dim3(kFT), (uint32_t)kFullLdsBytes, stream, a);
    return hipGetLastError();
}

// The other full rows.
hipError_t launch_full(const StreamArgs& a, uint32_t lds, hipStream_t stream) {
    if (a.gtab != nullptr) hipLaunchKernelGGL((k_full<true, false, false>), dim3(a.rows), dim3(kFT), lds, stream, a);
    else hipLaunchKernelGGL((k_full<false, false, false>), dim3(a.rows), dim3(kFT), lds, stream, a);
    return hipGetLastError();
}

size_t full_lds_bytes() { return kFullLdsBytes; }

hipError_t launch_writeback(const StreamArgs& a, int grid, uint32_t lds, hipStream_t stream) {
    if (a.gtab != nullptr) hipLaunchKernelGGL((k_writeback<true>), dim3(grid), dim3(kBlock), lds, stream, a);
    else hipLaunchKernelGGL((k_writeback<false>), dim3(grid), dim3(kBlock), lds, stream, a);
    return hipGetLastError();
}

}  // namespace hsamp
