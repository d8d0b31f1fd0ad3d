// HIP kernels of the gfx950 token sampler.
//
// k_stream: one workgroup per (row, slice) of the [B, V] logits. Each block
//   1. builds, in LDS, the penalty bookkeeping of its slice from the row's
//      history (bitmap of touched ids + open-addressing table of counts),
//   2. streams its slice in 8192-element tiles with 16-byte loads, applies
//      mask -> bias -> repetition -> DRY -> frequency/presence -> temperature
//      to each logit in registers (reference src/sampler/sampler.cpp:235-264),
//   3. keeps a candidate buffer of (value, index) composites in LDS, filtered
//      by a threshold that only rises: a per-tile lower bound from the k/4-th
//      largest group maximum of each wave (ballot radix select), and the exact
//      k-th composite after each buffer compaction (LDS radix select),
//   4. hands its candidates to the row's last block (atomic counter), which
//      merges them into the exact top-k (value desc, index asc) and runs the
//      rest of the ladder over the <= k kept logits: softmax with glibc-exact
//      expf and index-order float sums, top-p over the (p desc, index asc)
//      order, min-p, the double-precision CDF and the draw against u.
// Greedy rows (T <= 0) take the argmax of the penalised logits instead.
//
// k_writeback: optional second pass leaving the logits exactly as the
//   reference's sample() leaves them (kept logits post-temperature, the rest
//   -inf; post-penalty logits for greedy rows).
//
// No MFMA: nothing here is a contraction. The stream phase is HBM-bound.
#include <hip/hip_runtime.h>

#include "hsamp_plan.h"
#include "libm_expf.h"

#pragma clang fp contract(off)

namespace hsamp {

using u64 = unsigned long long;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kKeyNegInf = 0x007FFFFFu;        // key32(-inf)
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
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

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

struct Shared {
    u64 theta;          // current survival threshold (composite)
    u64 minv;
    int n;              // entries in the candidate buffer
    int last;           // this block merges its row
    int sel_d, sel_need, sel_cnt;
    int scan[8];
    uint32_t twave[4];
    float fred[4];
    int ired[4];
    u64 ured[4];
    uint32_t hist[256];
    int soff[257];      // slice offsets during the merge
    int flags;
    int nan0;
    float sm_m, sm_inv;
    int cutoff;
    double dS;
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

// k-th largest (1 <= k <= n) of n distinct composites in buf, by 8-bit radix
// passes from the top with early exit.
__device__ __attribute__((noinline)) u64 block_select_kth(const u64* buf, int n, int k, Shared& st) {
    u64 prefix = 0, pmask = 0;
    int need = k;
    const int tid = threadIdx.x;
    for (int shift = 56; shift >= 0; shift -= 8) {
        st.hist[tid] = 0u;
        if (tid == 0) st.minv = ~0ull;
        __syncthreads();
        for (int i = tid; i < n; i += kBlock) {
            const u64 v = buf[i];
            if ((v & pmask) == prefix) atomicAdd(&st.hist[(uint32_t)(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            const int l = tid;
            const int c0 = st.hist[255 - 4 * l], c1 = st.hist[254 - 4 * l];
            const int c2 = st.hist[253 - 4 * l], c3 = st.hist[252 - 4 * l];
            const int s4 = c0 + c1 + c2 + c3;
            int incl = s4;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int y = __shfl_up(incl, d, 64);
                if (l >= d) incl += y;
            }
            const int excl = incl - s4;
            const bool mine = excl < need && need <= incl;
            const u64 bal = __ballot(mine);
            if (mine && (int)(__ffsll((long long)bal) - 1) == l) {
                int cum = excl;
                const int cs[4] = {c0, c1, c2, c3};
                for (int q = 0; q < 4; ++q) {
                    if (cum + cs[q] >= need) {
                        st.sel_d = 255 - 4 * l - q;
                        st.sel_need = need - cum;
                        st.sel_cnt = cs[q];
                        break;
                    }
                    cum += cs[q];
                }
            }
        }
        __syncthreads();
        const int d = st.sel_d, cnt = st.sel_cnt;
        need = st.sel_need;
        prefix |= (u64)d << shift;
        pmask |= (u64)0xFF << shift;
        if (cnt == need) {
            for (int i = tid; i < n; i += kBlock) {
                const u64 v = buf[i];
                if ((v & pmask) == prefix) atomicMin(&st.minv, v);
            }
            __syncthreads();
            const u64 r = st.minv;
            __syncthreads();
            return r;
        }
        __syncthreads();
    }
    return prefix;
}

// Keep the k largest of the buffer's entries (exactly k; they are distinct).
__device__ __attribute__((noinline)) void buf_compact(u64* buf, int k, Shared& st) {
    const int n = st.n;
    if (n <= k) return;
    const u64 kth = block_select_kth(buf, n, k, st);
    constexpr int MAXE = 16;  // buf_cap <= 4096
    u64 v[MAXE];
    int cnt = 0;
    const int tid = threadIdx.x;
#pragma unroll
    for (int m = 0; m < MAXE; ++m) {
        const int i = tid + m * kBlock;
        v[m] = (i < n) ? buf[i] : 0ull;
        cnt += (i < n && v[m] >= kth) ? 1 : 0;
    }
    int total;
    int pos = block_excl_scan(cnt, &total, st);  // syncs: every read above is done
#pragma unroll
    for (int m = 0; m < MAXE; ++m) {
        const int i = tid + m * kBlock;
        if (i < n && v[m] >= kth) buf[pos++] = v[m];
    }
    __syncthreads();
    if (tid == 0) {
        st.n = total;
        st.theta = kth;
    }
    __syncthreads();
}

// Offer register-held candidates to the LDS buffer. Slot i of every thread
// holds an order key kv[i] (0 = empty) of id idx(i); it survives when its
// composite is >= the threshold. Survivors reserve entries with one LDS atomic
// per wave and slot; entries past the buffer's capacity go to the block's
// global overflow area `ovf` (drained by drain_overflow).
template <int NE, typename Idx>
__device__ __forceinline__ void append_regs(u64* buf, int cap, const uint32_t (&kv)[NE], Idx idx,
                                            u64* ovf, Shared& st) {
    const int lane = lane_id();
    const u64 th = st.theta;
    const uint32_t thk = (uint32_t)(th >> 32);
    const uint32_t thi = ~(uint32_t)th;   // largest index that survives a tie on thk
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const uint32_t key = kv[i];
        const bool sv = key > thk || (key == thk && (uint32_t)idx(i) <= thi);
        const u64 bal = __ballot(sv);
        if (bal == 0ull) continue;
        const int leader = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane == leader) base = atomicAdd(&st.n, __popcll(bal));
        base = __shfl(base, leader, 64);
        if (sv) {
            const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
            const u64 c = comp(key, idx(i));
            if (pos < cap) buf[pos] = c;
            else ovf[pos - cap] = c;
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

__device__ __attribute__((noinline)) void bitonic_sort(u64* a, int P, bool descending) {
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += kBlock) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const u64 x = a[i], y = a[ixj];
                    const bool up = ((i & k) == 0) != descending;
                    if ((x > y) == up) {
                        a[i] = y;
                        a[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int next_pow2(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// ---- penalty bookkeeping -----------------------------------------------------

struct PenaltyLds {
    uint32_t* bitmap;   // bit (t - lo): t has an entry in the table
    uint32_t* hkey;
    uint32_t* hval;
    uint32_t hmask;
    uint32_t hshift;
};

__device__ __forceinline__ uint32_t hslot(int32_t t, const PenaltyLds& pl) {
    return ((uint32_t)t * 0x9E3779B1u) >> pl.hshift;
}

__device__ uint32_t pen_insert(int32_t t, const PenaltyLds& pl) {
    uint32_t s = hslot(t, pl);
    for (;;) {
        const uint32_t old = atomicCAS(&pl.hkey[s], kEmpty, (uint32_t)t);
        if (old == kEmpty || old == (uint32_t)t) return s;
        s = (s + 1) & pl.hmask;
    }
}

// Build the table for ids in [lo, hi) from the row's history suffix and bias.
__device__ __attribute__((noinline)) void pen_build(const StreamArgs& a, const RowPlan& P, int r, int lo, int hi,
                          const PenaltyLds& pl) {
    const int tid = threadIdx.x;
    for (int i = tid; i < a.bitmap_words; i += kBlock) pl.bitmap[i] = 0u;
    for (int i = tid; i < a.hash_slots; i += kBlock) {
        pl.hkey[i] = kEmpty;
        pl.hval[i] = 0u;
    }
    __syncthreads();
    const int L = P.hist_len;
    const int32_t* h = a.hist + (int64_t)r * a.hist_stride;
    for (int p = L - P.scan_len + tid; p < L; p += kBlock) {
        const int32_t t = h[p];
        if (t < lo || t >= hi) continue;
        uint32_t add = 0u, orv = 0u;
        if (p >= L - P.rep_win) orv |= HV_REP;
        if (p >= L - P.dry_win) add += 1u << HV_DRY_SHIFT;
        if (p >= L - P.fp_win) add += 1u;
        const uint32_t s = pen_insert(t, pl);
        if (add) atomicAdd(&pl.hval[s], add);
        if (orv) atomicOr(&pl.hval[s], orv);
        atomicOr(&pl.bitmap[(t - lo) >> 5], 1u << ((t - lo) & 31));
    }
    if (P.flags & RF_BIAS) {
        for (int j = tid; j < P.bias_cnt; j += kBlock) {
            const int32_t t = a.bias_ids[P.bias_off + j];
            if (t < lo || t >= hi) continue;
            const uint32_t s = pen_insert(t, pl);
            atomicOr(&pl.hval[s], HV_BIAS);
            atomicOr(&pl.bitmap[(t - lo) >> 5], 1u << ((t - lo) & 31));
        }
    }
    __syncthreads();
}

// Stages 1-4 of the ladder for one id with a table entry (sampler.cpp:28-99).
__device__ __attribute__((noinline)) float pen_apply(float x, int32_t t, const StreamArgs& a,
                                           const RowPlan& P, const PenaltyLds& pl) {
    uint32_t s = hslot(t, pl);
    while (pl.hkey[s] != (uint32_t)t) s = (s + 1) & pl.hmask;
    const uint32_t v = pl.hval[s];
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

// ---- tile loading --------------------------------------------------------------

template <int DT>
struct Tile {
    static constexpr int VW = DT == 0 ? 4 : 8;    // elements per 16-byte chunk
    static constexpr int NCH = DT == 0 ? 8 : 4;   // chunks per thread per tile
    static constexpr int NE = VW * NCH;           // 32 elements per thread
    static constexpr int ES = DT == 0 ? 4 : 2;    // bytes per element
    static constexpr int ELEMS = kBlock * NE;     // 8192 per tile
};

template <int DT, bool VEC>
__device__ __forceinline__ void load_tile(const char* rowp, const uint32_t* mrow, int tb, int hi,
                                          uint4 (&raw)[Tile<DT>::NCH],
                                          uint32_t (&mw)[Tile<DT>::NCH]) {
    using T = Tile<DT>;
#pragma unroll
    for (int j = 0; j < T::NCH; ++j) {
        const int e0 = tb + (j * kBlock + (int)threadIdx.x) * T::VW;
        if (VEC && e0 + T::VW <= hi) {
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp + (size_t)e0 * T::ES));
            raw[j] = make_uint4(v.x, v.y, v.z, v.w);
        } else {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            for (int c = 0; c < T::VW; ++c) {
                if (e0 + c < hi) {
                    uint32_t b;
                    if (DT == 0) b = reinterpret_cast<const uint32_t*>(rowp)[e0 + c];
                    else b = reinterpret_cast<const uint16_t*>(rowp)[e0 + c];
                    if (DT == 0) w[c] = b;
                    else w[c >> 1] |= b << ((c & 1) * 16);
                }
            }
            raw[j] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        mw[j] = (mrow != nullptr && e0 < hi) ? mrow[e0 >> 5] : 0xFFFFFFFFu;
    }
}

template <int DT>
__device__ __forceinline__ float elem(const uint4& r, int c) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if (DT == 0) return __uint_as_float(w[c]);
    const uint32_t x = w[c >> 1];
    return __uint_as_float((c & 1) ? (x & 0xFFFF0000u) : (x << 16));
}

// ---- finalize over the kept set ------------------------------------------------

struct FinLds {
    u64* sortk;     // [P2]; also the double q_i
    int32_t* fidx;  // [kmax] kept ids, index order
    float* fv;      // values (post-temperature)
    float* fe;      // expf(v - m)
    float* fp;      // probabilities
    int32_t* keep;  // still kept
};

// softmax_probs over the kept entries (sampler.cpp:124-142): m, e, float
// index-order sum, p = e * fl(1/sum). Returns false when nothing is kept.
__device__ __attribute__((noinline)) bool fin_softmax(const FinLds& f, int nk, Shared& st) {
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (int j = tid; j < nk; j += kBlock)
        if (f.keep[j]) m = fmaxf(m, f.fv[j]);
    m = block_max_f(m, st);
    if (m == -__builtin_inff()) return false;
    for (int j = tid; j < nk; j += kBlock) f.fe[j] = f.keep[j] ? libm_expf(f.fv[j] - m) : 0.0f;
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int j = 0; j < nk; ++j)
            if (f.keep[j]) s = s + f.fe[j];
        st.sm_inv = (s <= 0.0f) ? __builtin_nanf("") : 1.0f / s;
        st.sm_m = s;
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
__device__ __attribute__((noinline)) void finalize_row(const StreamArgs& a, const RowPlan& P, int r, const u64* buf, int nk,
                             const FinLds& f, Shared& st, uint32_t rflags) {
    const int tid = threadIdx.x;
    const int V = a.vocab;
    const double u = a.u[r];
    const bool single = (P.flags & RF_SINGLE) != 0;
    if (!single) rflags |= ROWF_U_USED;
    int32_t tok = 0;
    int nkept = nk;
    if (nk > 0) {
        const int P2 = next_pow2(nk);
        for (int i = tid; i < P2; i += kBlock)
            f.sortk[i] = (i < nk) ? (((u64)(uint32_t)comp_idx(buf[i]) << 32) | (buf[i] >> 32)) : ~0ull;
        __syncthreads();
        bitonic_sort(f.sortk, P2, false);
        for (int j = tid; j < nk; j += kBlock) {
            const u64 e = f.sortk[j];
            f.fidx[j] = (int32_t)(e >> 32);
            f.fv[j] = key_to_float((uint32_t)e);
            f.keep[j] = 1;
        }
        __syncthreads();
        if (a.topk_idx != nullptr) {
            for (int j = tid; j < nk && j < a.set_cap; j += kBlock)
                a.topk_idx[(int64_t)r * a.set_cap + j] = f.fidx[j];
        }
        if (a.topk_count != nullptr && tid == 0) a.topk_count[r] = single ? -1 : nk;

        bool have = fin_softmax(f, nk, st);
        bool fresh = true;  // fp matches the current kept set
        if (have && (P.flags & RF_TOPP)) {
            // sampler.cpp:146-164
            for (int i = tid; i < P2; i += kBlock)
                f.sortk[i] = (i < nk && f.keep[i])
                                 ? (((u64)key32(f.fp[i]) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)i))
                                 : 0ull;
            __syncthreads();
            bitonic_sort(f.sortk, P2, true);
            if (tid == 0) {
                float c = 0.0f;
                int cutoff = -1;
                for (int i = 0; i < nk; ++i) {
                    const u64 e = f.sortk[i];
                    if (e == 0ull) break;
                    const int j = (int)(0xFFFFFFFFu - (uint32_t)e);
                    c = c + f.fp[j];
                    if (c >= P.top_p) {
                        cutoff = i + 1;
                        break;
                    }
                }
                if (cutoff > 0 && fabsf(c - P.top_p) <= 1e-6f) rflags |= ROWF_TOPP_NEAR;
                st.cutoff = cutoff;
                st.flags = (int)rflags;
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
        if (have && (P.flags & RF_MINP)) {
            // sampler.cpp:167-176
            if (!fresh) have = fin_softmax(f, nk, st);
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
        if (have && !fresh) have = fin_softmax(f, nk, st);
        if (have) {
            // sampler.cpp:178-182 / discrete_distribution: double sum, q, partial sums.
            double* fq = reinterpret_cast<double*>(f.sortk);
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
                if (single) {
                    t = 0;
                } else if (!(u > 0.0)) {
                    t = 0;
                } else {
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
                }
                if (near <= 1e-6) rflags |= ROWF_CDF_NEAR;
                st.tok = t;
                st.flags = (int)rflags;
            }
            __syncthreads();
            tok = st.tok;
            rflags = (uint32_t)st.flags;
        } else {
            nkept = 0;
        }
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
    if (tid == 0) {
        a.token[r] = tok;
        if (a.row_flags != nullptr) a.row_flags[r] = rflags;
        if (a.kept_count != nullptr) a.kept_count[r] = nkept;
        if (a.fin_n != nullptr) a.fin_n[r] = nkept;
    }
}

// ---- the fused stream kernel ---------------------------------------------------

template <int DT, bool VEC>
__global__ __launch_bounds__(kBlock) void k_stream(StreamArgs a) {
    using T = Tile<DT>;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ Shared st;
    const int tid = threadIdx.x;
    const int logical = (int)(blockIdx.x % kXcds) * a.blocks_per_xcd + (int)(blockIdx.x / kXcds);
    const int r = logical / a.nslices, s = logical % a.nslices;
    if (r >= a.rows) return;
    const RowPlan P = a.plans[r];
    const int V = a.vocab;
    const int lo = s * a.slice_len;
    const int hi = min(V, lo + a.slice_len);
    const bool greedy = (P.flags & RF_GREEDY) != 0;
    const bool pen = (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;

    // LDS carve: [penalty region | finalize region] aliased, then the buffer.
    PenaltyLds pl;
    pl.bitmap = reinterpret_cast<uint32_t*>(smem);
    pl.hkey = pl.bitmap + ((a.bitmap_words + 3) & ~3);
    pl.hval = pl.hkey + a.hash_slots;
    pl.hmask = (uint32_t)a.hash_slots - 1u;
    pl.hshift = 32u - (uint32_t)__popc(pl.hmask);
    const int kP2 = next_pow2(max(a.kmax, 1));
    FinLds f;
    f.sortk = reinterpret_cast<u64*>(smem);
    f.fidx = reinterpret_cast<int32_t*>(f.sortk + kP2);
    f.fv = reinterpret_cast<float*>(f.fidx + a.kmax);
    f.fe = f.fv + a.kmax;
    f.fp = f.fe + a.kmax;
    f.keep = reinterpret_cast<int32_t*>(f.fp + a.kmax);
    u64* buf = reinterpret_cast<u64*>(smem + (a.lds_bytes - (uint32_t)a.buf_cap * 8u));
    u64* ovf = a.ovf + (int64_t)logical * a.ovf_cap;

    const char* rowp = static_cast<const char*>(a.logits) + (size_t)r * (size_t)a.logits_stride * T::ES;
    const uint32_t* mrow = (P.flags & RF_MASK) ? a.mask + (int64_t)r * a.mask_stride : nullptr;

    if (tid == 0) {
        st.theta = kThetaFloor;
        st.n = 0;
        st.nan0 = 0;
        st.flags = 0;
    }
    uint4 raw[T::NCH];
    uint32_t mw[T::NCH];
    load_tile<DT, VEC>(rowp, mrow, lo, hi, raw, mw);
    if (pen) pen_build(a, P, r, lo, hi, pl);
    __syncthreads();

    const int k = P.top_k;
    const int kw = (k + 3) >> 2;
    const int G = min(4, max(1, (kw + 63) >> 6));
    const float inv_t = P.inv_temp;
    const bool temp = (P.flags & RF_TEMP) != 0;
    u64 best = 0ull;          // greedy: best composite of this thread
    int nanseen = 0;

    for (int tb = lo; tb < hi; tb += T::ELEMS) {
        // Transform each logit of the tile and keep only its order key:
        // mask -> bias/penalties -> (temperature) -> key32; 0 marks "absent".
        uint32_t kv[T::NE];
#pragma unroll
        for (int j = 0; j < T::NCH; ++j) {
            const int e0 = tb + (j * kBlock + tid) * T::VW;
            const uint32_t mbits = mw[j] >> (e0 & 31);
            uint32_t pbits = 0u;
            if (pen && e0 < hi) pbits = pl.bitmap[(e0 - lo) >> 5] >> ((e0 - lo) & 31);
#pragma unroll
            for (int c = 0; c < T::VW; ++c) {
                float x = elem<DT>(raw[j], c);
                if (!((mbits >> c) & 1u)) x = -__builtin_inff();
                if ((pbits >> c) & 1u) x = pen_apply(x, e0 + c, a, P, pl);
                uint32_t key;
                if (greedy) {
                    // argmax of sampler.cpp:220-228: NaN never wins; element 0 NaN -> 0.
                    const bool nan = x != x;
                    if (nan && e0 + c < hi) {
                        nanseen = 1;
                        if (e0 + c == 0) st.nan0 = 1;
                    }
                    key = nan ? 0u : key32(x);
                } else {
                    if (temp) x = x * inv_t;                    // sampler.cpp:101-106
                    if (x != x) {
                        if (e0 + c < hi) nanseen = 1;
                        x = -__builtin_inff();
                    }
                    key = key32(x);
                }
                kv[j * T::VW + c] = (e0 + c < hi) ? key : 0u;
            }
        }
        // The raw registers are free: start the next tile's loads now.
        if (tb + T::ELEMS < hi) load_tile<DT, VEC>(rowp, mrow, tb + T::ELEMS, hi, raw, mw);
        if (greedy) {
#pragma unroll
            for (int j = 0; j < T::NCH; ++j) {
                const int e0 = tb + (j * kBlock + tid) * T::VW;
#pragma unroll
                for (int c = 0; c < T::VW; ++c) {
                    const u64 cc = (e0 + c < hi) ? comp(kv[j * T::VW + c], e0 + c) : 0ull;
                    best = cc > best ? cc : best;
                }
            }
            continue;
        }
        // Per-tile lower bound on the k-th largest: the kw-th largest group
        // maximum of each wave (kw = ceil(k/4)), minimum over the 4 waves.
        uint32_t gk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < T::NCH; ++j) {
            const int g = (j * 4) / T::NCH;
            const int gg = (G == 4) ? g : (G == 2 ? (g >> 1) : 0);
#pragma unroll
            for (int c = 0; c < T::VW; ++c) gk[gg] = max(gk[gg], kv[j * T::VW + c]);
        }
        const uint32_t tw = (kw <= 64 * G) ? wave_kth_largest(gk, G, kw) : 0u;
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
        const int bt = tb + tid * T::VW;
        auto idx = [&](int i) -> int32_t { return bt + (i / T::VW) * (kBlock * T::VW) + (i % T::VW); };
        append_regs<T::NE>(buf, a.buf_cap, kv, idx, ovf, st);
        drain_overflow(buf, a.buf_cap, k, ovf, st);
    }

    // ---- slice result -----------------------------------------------------------
    uint32_t rflags = 0u;
    if (nanseen) atomicOr(&st.flags, 1);
    __syncthreads();
    if (st.flags & 1) rflags |= ROWF_NAN;
    if (greedy) {
        best = block_max_u64(best, st);
        if (a.nslices == 1) {
            if (tid == 0) {
                a.token[r] = st.nan0 ? 0 : comp_idx(best);
                if (a.row_flags != nullptr) a.row_flags[r] = rflags | ROWF_GREEDY;
                if (a.topk_count != nullptr) a.topk_count[r] = -1;
                if (a.kept_count != nullptr) a.kept_count[r] = 0;
            }
            return;
        }
        if (tid == 0) {
            u64* out = a.cand + ((int64_t)r * a.nslices + s) * a.cand_cap;
            out[0] = best;
            out[1] = (u64)(st.nan0 | (rflags ? 2 : 0));
            a.cand_n[(int64_t)r * a.nslices + s] = 2;
        }
    } else if (a.nslices == 1) {
        buf_compact(buf, k, st);
        finalize_row(a, P, r, buf, st.n, f, st, rflags);
        return;
    } else {
        if (st.n > a.cand_cap) buf_compact(buf, k, st);
        const int n = st.n;
        u64* out = a.cand + ((int64_t)r * a.nslices + s) * a.cand_cap;
        for (int i = tid; i < n; i += kBlock) out[i] = buf[i];
        if (tid == 0) a.cand_n[(int64_t)r * a.nslices + s] = n | (rflags ? (1 << 30) : 0);
    }

    // ---- last block of the row merges -----------------------------------------
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&a.counters[r], 1u);
        st.last = (prev == (unsigned)(a.nslices - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!st.last) return;
    __threadfence();
    if (tid == 0) a.counters[r] = 0u;

    const int S = a.nslices;
    const u64* cand = a.cand + (int64_t)r * S * a.cand_cap;
    const int32_t* cn = a.cand_n + (int64_t)r * S;
    if (greedy) {
        u64 b = 0ull;
        int nan0 = 0, anynan = 0;
        for (int i = tid; i < S; i += kBlock) {
            const u64 c = cand[(int64_t)i * a.cand_cap];
            b = c > b ? c : b;
            const int fl = (int)cand[(int64_t)i * a.cand_cap + 1];
            nan0 |= fl & 1;
            anynan |= (fl >> 1) & 1;
        }
        b = block_max_u64(b, st);
        if (nan0) atomicOr(&st.nan0, 1);
        if (anynan) atomicOr(&st.flags, 2);
        __syncthreads();
        if (tid == 0) {
            a.token[r] = st.nan0 ? 0 : comp_idx(b);
            if (a.row_flags != nullptr)
                a.row_flags[r] = ROWF_GREEDY | ((st.flags & 2) ? ROWF_NAN : 0u);
            if (a.topk_count != nullptr) a.topk_count[r] = -1;
            if (a.kept_count != nullptr) a.kept_count[r] = 0;
        }
        return;
    }
    // slice offsets
    int myc = 0, mynan = 0;
    if (tid < S) {
        const int v = cn[tid];
        myc = v & 0x3FFFFFFF;
        mynan = (v >> 30) & 1;
    }
    int M;
    const int off = block_excl_scan(myc, &M, st);
    if (tid < S) st.soff[tid] = off;
    if (tid == 0) {
        st.soff[S] = M;
        st.n = 0;
        st.theta = kThetaFloor;
    }
    if (mynan) atomicOr(&st.flags, 4);
    __syncthreads();
    rflags = (st.flags & 4) ? ROWF_NAN : 0u;
    append_fetch(buf, a.buf_cap, k, M, [&](int fi) {
        int lo2 = 0, hi2 = S;  // last slice with soff <= fi
        while (hi2 - lo2 > 1) {
            const int mid = (lo2 + hi2) >> 1;
            if (st.soff[mid] <= fi) lo2 = mid;
            else hi2 = mid;
        }
        return cand[(int64_t)lo2 * a.cand_cap + (fi - st.soff[lo2])];
    }, st);
    buf_compact(buf, k, st);
    finalize_row(a, P, r, buf, st.n, f, st, rflags);
}

// ---- writeback -------------------------------------------------------------------

template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_writeback(StreamArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int logical = (int)(blockIdx.x % kXcds) * a.blocks_per_xcd + (int)(blockIdx.x / kXcds);
    const int r = logical / a.nslices, s = logical % a.nslices;
    if (r >= a.rows) return;
    const RowPlan P = a.plans[r];
    const int V = a.vocab;
    const int lo = s * a.slice_len;
    const int hi = min(V, lo + a.slice_len);
    const bool greedy = (P.flags & RF_GREEDY) != 0;
    const bool pen = (P.flags & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) != 0;
    PenaltyLds pl;
    pl.bitmap = reinterpret_cast<uint32_t*>(smem);
    pl.hkey = pl.bitmap + ((a.bitmap_words + 3) & ~3);
    pl.hval = pl.hkey + a.hash_slots;
    pl.hmask = (uint32_t)a.hash_slots - 1u;
    pl.hshift = 32u - (uint32_t)__popc(pl.hmask);
    uint32_t* keepbm = pl.hval + a.hash_slots;  // kept ids of this slice
    if (pen) pen_build(a, P, r, lo, hi, pl);
    for (int i = tid; i < a.bitmap_words; i += kBlock) keepbm[i] = 0u;
    __syncthreads();
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
        if (pen && ((pl.bitmap[(e - lo) >> 5] >> ((e - lo) & 31)) & 1u)) x = pen_apply(x, e, a, P, pl);
        if (!greedy) {
            if (P.flags & RF_TEMP) x = x * P.inv_temp;
            if (!((keepbm[(e - lo) >> 5] >> ((e - lo) & 31)) & 1u)) x = -__builtin_inff();
        }
        row[e] = x;
    }
}

// ---- launchers -------------------------------------------------------------------

hipError_t launch_stream(const StreamArgs& a, int dtype, bool vec, int grid, hipStream_t stream) {
    const dim3 g(grid), b(kBlock);
    if (dtype == 0) {
        if (vec) hipLaunchKernelGGL((k_stream<0, true>), g, b, a.lds_bytes, stream, a);
        else hipLaunchKernelGGL((k_stream<0, false>), g, b, a.lds_bytes, stream, a);
    } else {
        if (vec) hipLaunchKernelGGL((k_stream<1, true>), g, b, a.lds_bytes, stream, a);
        else hipLaunchKernelGGL((k_stream<1, false>), g, b, a.lds_bytes, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_writeback(const StreamArgs& a, int grid, uint32_t lds, hipStream_t stream) {
    hipLaunchKernelGGL((k_writeback<true>), dim3(grid), dim3(kBlock), lds, stream, a);
    return hipGetLastError();
}

}  // namespace hsamp
