// Host side of the C ABI in include/ultima_hsamp.h.
//
// Each run() turns the per-row knobs into RowPlans with the reference's own
// stage predicates (src/sampler/sampler.cpp:230-277), packs them with the DRY
// penalty tables and the sorted logit-bias entries into one blob, uploads the
// blob through a small ring of pinned staging buffers (skipped when the same
// blob is already resident), picks the slicing of the vocabulary and launches
// the stream kernel (one block per row slice) and the merge kernel (one block
// per row) on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <tuple>
#include <vector>

#include "hsamp_plan.h"
#include "hsamp_run.h"
#include "ultima_hsamp.h"

namespace hsamp {
hipError_t launch_stream(const StreamArgs& a, int dtype, bool vec, bool pen_greedy, bool pen_sample, bool mask,
                         bool greedy_rows, bool sample_rows, int grid, hipStream_t stream);
hipError_t launch_writeback(const StreamArgs& a, int grid, uint32_t lds, hipStream_t stream);
hipError_t launch_full_pre(const StreamArgs& a, bool plain, bool tp, hipStream_t stream);
hipError_t launch_merge(const StreamArgs& a, hipStream_t stream);
hipError_t launch_pick_l(const StreamArgs& a, hipStream_t stream);
hipError_t launch_stream_ex(const StreamArgs& a, int dtype, bool vec, bool pen, bool mask, int tiles, bool lean, int grid,
                            hipStream_t stream);
hipError_t launch_pick(const StreamArgs& a, int nw, hipStream_t stream);
hipError_t launch_full(const StreamArgs& a, uint32_t lds, hipStream_t stream);
hipError_t launch_read_probe(const StreamArgs& a, int dtype, int tiles, int grid, float* out, hipStream_t stream);
size_t full_lds_bytes();
}  // namespace hsamp

using namespace hsamp;

namespace {

constexpr int kSlots = 16;   // resident plan blobs (a graph pins the ones it reads)
constexpr int kTile = kBlock * 32;      // elements of one k_stream tile (32 per thread)
constexpr int kTargetBlocks = 4096;     // most blocks a launch spreads rows over
constexpr int kTwoTileBlocks = 512;     // exact lists: two-tile slices while B * S stays at or above this
constexpr int kMergeRound = kBlock * 16;  // candidates k_merge offers per round
constexpr int kMergeWindow = kBlock * 16; // list entries k_merge loads up front, over all slices
constexpr int kFullMaxWin = 2048;       // k_full: index-order windows its LDS tables hold

struct Slot {
    char* host = nullptr;   // pinned
    char* dev = nullptr;
    size_t cap = 0;
    size_t size = 0;
    hipEvent_t ev = nullptr;
    bool used = false;
    bool pinned = false;    // referenced by a captured graph: never rewritten
};

int next_pow2(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}
size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

}  // namespace

struct ultima_hsamp {
    int device = 0;
    int32_t max_rows = 0;
    int32_t max_vocab = 0;
    DevCaps caps;
    hipStream_t own_stream = nullptr;
    hipEvent_t phase_ev = nullptr;   // recorded between the stream and merge kernels when set
    Slot slots[kSlots];
    int next_slot = 0;
    HostScratch hs;
    // device scratch, grown on demand
    unsigned long long* cand = nullptr;
    size_t cand_elems = 0;
    int32_t* cand_n = nullptr;    // [slots] counts, then [slots] bounds
    size_t cand_slots = 0;
    uint32_t* gtab = nullptr;            // per-row penalty tables too large for LDS
    size_t gtab_words = 0;
    int32_t* fin_idx = nullptr;
    int32_t* fin_n = nullptr;
    unsigned long long* ovf = nullptr;   // per-row overflow of the LDS candidate buffer
    size_t ovf_elems = 0;
    float* fullv = nullptr;              // full-vocabulary rows: transformed logits
    size_t fullv_elems = 0;
    float* fullp = nullptr;              // full-vocabulary rows: probabilities
    size_t fullp_elems = 0;
    uint32_t* fs_tab = nullptr;          // full-vocabulary rows: k_fs_* per-window tables
    size_t fs_elems = 0;
    // A graph captured from this handle holds the scratch pointers of its
    // launches: once one has been captured, scratch that grows is kept (not
    // freed) until destroy, so that replaying an earlier graph stays valid.
    bool captured = false;
    std::vector<void*> retired;
    // sample_host staging
    float* d_row = nullptr;
    float* h_row = nullptr;       // pinned
    int32_t* d_hist = nullptr;
    int32_t* h_hist = nullptr;    // pinned
    size_t hist_cap = 0;
    double* d_u = nullptr;
    int32_t* d_tok = nullptr;
    double* h_u = nullptr;        // pinned
    int32_t* h_tok = nullptr;     // pinned
};

namespace hsamp {

// ULTIMA_HSAMP_DEBUG=1 prints each failing HIP call to stderr.
int hip_fail(hipError_t e, const char* what, int line) {
    static const bool debug = [] {
        const char* v = std::getenv("ULTIMA_HSAMP_DEBUG");
        return v != nullptr && v[0] == '1';
    }();
    if (debug) std::fprintf(stderr, "ultima_hsamp: %s failed (%s) at hsamp_api.cpp:%d\n", what,
                            hipGetErrorString(e), line);
    (void)hipGetLastError();
    return e == hipErrorOutOfMemory ? ULTIMA_HSAMP_ERR_NOMEM : ULTIMA_HSAMP_ERR_HIP;
}

}  // namespace hsamp

#define HIP_TRY(x)                                                   \
    do {                                                             \
        hipError_t e_ = (x);                                         \
        if (e_ != hipSuccess) return hip_fail(e_, #x, __LINE__);     \
    } while (0)

namespace {

bool isnan_f(float x) { return x != x; }

// DRY table key: (multiplier bits, base bits, allowed, window).
using DryKey = std::tuple<uint32_t, uint32_t, int32_t, int32_t>;

uint32_t fbits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

}  // namespace

namespace hsamp {

// RowPlans + DRY tables + bias into hs.blob; the reference's predicates in [].
int build_blob(HostScratch& hs, const ultima_hsamp_batch* b, Built& out) {
    const int B = b->rows, V = b->vocab;
    hs.plans.assign(B, RowPlan{});
    std::vector<float>& dry = hs.dry;
    dry.clear();
    // DRY tables already built for this batch (a handful of distinct settings:
    // a linear search over a reused vector, no allocation once warm)
    auto& dry_seen = hs.dry_seen;
    dry_seen.clear();
    std::vector<int32_t>& bids = hs.bias_ids;
    std::vector<float>& bvals = hs.bias_vals;
    bids.clear();
    bvals.clear();
    std::vector<std::pair<int32_t, float>>& tmp = hs.tmp;
    for (int r = 0; r < B; ++r) {
        const ultima_hsamp_params& q = b->params[r];
        RowPlan& P = hs.plans[r];
        P.inv_temp = 1.0f;   // x * 1.0f == x: rows without temperature multiply by one
        if (isnan_f(q.rep_penalty) || isnan_f(q.dry_multiplier) || isnan_f(q.dry_base) ||
            isnan_f(q.frequency_penalty) || isnan_f(q.presence_penalty) ||
            isnan_f(q.temperature) || isnan_f(q.top_p) || isnan_f(q.min_p))
            return ULTIMA_HSAMP_ERR_INVALID;
        // hist_stride 0: one history shared by every row, row r its first
        // hist_len ids
        if (q.hist_len < 0 || (b->hist_stride > 0 && q.hist_len > b->hist_stride) ||
            (q.hist_len > 0 && b->hist == nullptr))
            return ULTIMA_HSAMP_ERR_INVALID;
        if (q.bias_count < 0 || q.bias_count > ULTIMA_HSAMP_MAX_BIAS ||
            (q.bias_count > 0 && (b->bias_ids == nullptr || b->bias_vals == nullptr || q.bias_offset < 0)))
            return ULTIMA_HSAMP_ERR_INVALID;
        // A history whose length is read on the device (hist_len_dev): the
        // windows here are the caps its rows can reach (the stride), each
        // row's own taken on the device (RF_DEVWIN, plan_of in the kernels)
        const bool devwin = b->hist_len_dev != nullptr;
        const int64_t L = devwin ? b->hist_stride : q.hist_len;
        auto win = [&](uint64_t n) -> int64_t { return (int64_t)std::min<uint64_t>(n, (uint64_t)L); };
        uint32_t fl = 0;
        bool bias_up = false;   // a bias entry can raise a logit
        const bool greedy = q.temperature <= 0.0f;                             // [261]
        if (greedy) fl |= RF_GREEDY;
        int64_t rep_w = 0, dry_w = 0, fp_w = 0;
        if (q.rep_penalty != 1.0f && q.repeat_last_n > 0 && win(q.repeat_last_n) > 0) {  // [239, 44]
            fl |= RF_REP;
            rep_w = win(q.repeat_last_n);
        }
        if (q.dry_multiplier > 0.0f && q.dry_last_n > 0 && win(q.dry_last_n) >= 2) {     // [246, 69]
            fl |= RF_DRY;
            dry_w = win(q.dry_last_n);
        }
        if ((q.frequency_penalty != 0.0f || q.presence_penalty != 0.0f) &&             // [254-256, 89]
            win(std::max(q.repeat_last_n, q.dry_last_n)) > 0) {
            fl |= RF_FP;
            fp_w = win(std::max(q.repeat_last_n, q.dry_last_n));
        }
        const int64_t scan = std::max({rep_w, dry_w, fp_w});
        if (scan > ULTIMA_HSAMP_MAX_WINDOW) return ULTIMA_HSAMP_ERR_CAPACITY;
        P.rep = q.rep_penalty;
        P.freq = q.frequency_penalty;
        P.pres = q.presence_penalty;
        P.hist_len = (int32_t)L;
        P.rep_win = (int32_t)rep_w;
        P.dry_win = (int32_t)dry_w;
        P.fp_win = (int32_t)fp_w;
        P.scan_len = (int32_t)scan;
        if (devwin) {
            fl |= RF_DEVWIN;
            P.win_caps[0] = (uint32_t)rep_w | ((uint32_t)dry_w << 16);
            P.win_caps[1] = (uint32_t)fp_w;
        }
        P.dry_allowed = (int32_t)std::min<uint64_t>(q.dry_allowed_len, 0x7fff);
        if (fl & RF_DRY) {
            // sampler.cpp:79-81: pen = multiplier * powf(base, float(n - allowed_len))
            const DryKey key{fbits(q.dry_multiplier), fbits(q.dry_base), P.dry_allowed, (int32_t)dry_w};
            auto it = std::find_if(dry_seen.begin(), dry_seen.end(), [&](const auto& e) { return e.first == key; });
            if (it == dry_seen.end()) {
                const int32_t off = (int32_t)dry.size();
                for (int64_t c = 0; c <= dry_w; ++c) {
                    const bool on = (uint64_t)c > q.dry_allowed_len;
                    dry.push_back(on ? q.dry_multiplier *
                                           std::pow(q.dry_base, static_cast<float>((uint64_t)c - q.dry_allowed_len))
                                     : 0.0f);
                }
                dry_seen.emplace_back(key, off);
                it = dry_seen.end() - 1;
            }
            P.dry_tab = it->second;
        }
        if (q.bias_count > 0) {
            tmp.clear();
            for (int64_t j = 0; j < q.bias_count; ++j) {
                const int32_t id = b->bias_ids[q.bias_offset + j];
                if (id < 0 || id >= V) continue;                                  // [32]
                tmp.emplace_back(id, b->bias_vals[q.bias_offset + j]);
            }
            std::sort(tmp.begin(), tmp.end(),
                      [](const auto& x, const auto& y) { return x.first < y.first; });
            for (size_t j = 1; j < tmp.size(); ++j)
                if (tmp[j].first == tmp[j - 1].first) return ULTIMA_HSAMP_ERR_INVALID;
            if (!tmp.empty()) {
                fl |= RF_BIAS;
                P.bias_off = (int32_t)bids.size();
                P.bias_cnt = (int32_t)tmp.size();
                for (auto& [id, v] : tmp) {
                    bids.push_back(id);
                    bvals.push_back(v);
                    if (!(v <= 0.0f)) bias_up = true;
                }
            }
        }
        if (b->mask != nullptr) {
            fl |= RF_MASK;
            out.any_mask = true;
        }
        if (!greedy) {
            P.temp = q.temperature;
            if (q.temperature != 1.0f) {                                          // [102]
                fl |= RF_TEMP;
                P.inv_temp = 1.0f / q.temperature;                                // [104]
                if (!(P.inv_temp > 0.0f && P.inv_temp < INFINITY)) out.inv_ok = false;
            }
            if (V == 1) {
                fl |= RF_SINGLE | RF_TOPK;
                P.top_k = 1;
            } else if (q.top_k > 0 && q.top_k < (uint64_t)V) {                   // [267, 110]
                fl |= RF_TOPK;
                P.top_k = (int32_t)q.top_k;
                if (P.top_k > kLimitK) fl |= RF_FULL;
            } else {
                fl |= RF_FULL;                                                    // top-k off
            }
            if (fl & RF_FULL) out.any_full = true;
            // plain transform (no penalties, no bias, no top-k): the row's whole-row
            // passes run over many blocks ahead of k_full
            if ((fl & RF_FULL) && !(fl & (RF_TOPK | RF_REP | RF_DRY | RF_FP | RF_BIAS))) {
                fl |= RF_FPRE;
                out.any_fpre = true;
            }
            else out.any_topk = out.any_sample = true;
            if ((fl & RF_FULL) && !(fl & RF_FPRE)) out.any_full_gen = true;
            if (q.top_p < 1.0f && !(q.top_p <= 0.0f)) fl |= RF_TOPP;             // [270, 147]
            if (q.min_p > 0.0f) fl |= RF_MINP;                                    // [273, 168]
            if (fl & RF_FPRE) {
                if (fl & (RF_TOPP | RF_MINP)) out.any_fpre_tp = true;
                else out.any_fpre_plain = true;
            }
            P.top_p = q.top_p;
            P.min_p = q.min_p;
            if (!(fl & RF_FULL)) out.kmax = std::max(out.kmax, P.top_k);
        } else {
            out.any_topk = out.any_greedy = true;
        }
        P.flags = fl;
        if (fl & RF_DRY) out.any_dry = true;
        // DRY and frequency/presence counting over different windows (DRY looks
        // back fewer ids than repetition): two counts per id, general kernels
        if ((fl & RF_DRY) && (fl & RF_FP) && fp_w != dry_w) out.dry_split = true;
        // the repetition window and the count window (DRY's, else frequency /
        // presence's) both on and different: a count entry is a count plus a
        // repetition bit
        // (windows taken on the device vary with the length: any row with both)
        {
            const int64_t cw = dry_w > 0 ? dry_w : fp_w;
            if (rep_w > 0 && cw > 0 && (rep_w != cw || devwin)) out.two_windows = true;
        }
        if (fl & (RF_REP | RF_DRY | RF_FP | RF_BIAS)) {
            out.any_pen = true;
            out.max_pen = std::max(out.max_pen, (int)scan + P.bias_cnt);
            out.max_scan = std::max(out.max_scan, (int)scan);
            out.max_bias = std::max(out.max_bias, (int)P.bias_cnt);
            // x/p, x*p (p >= 1), x - n*f - pp (f, pp >= 0), x - dry term (>= 0),
            // x + b (b <= 0) never raise x (sampler.cpp:28-99)
            if (((fl & RF_REP) && !(P.rep >= 1.0f)) || ((fl & RF_FP) && !(P.freq >= 0.0f && P.pres >= 0.0f)) ||
                ((fl & RF_DRY) && !(q.dry_multiplier >= 0.0f && q.dry_base >= 0.0f)))
                out.pen_lowers = out.pen_lowers_nb = false;
            if (bias_up) out.pen_lowers = false;
        }
    }
    out.off_dry = align16(sizeof(RowPlan) * B);
    out.off_bias_ids = align16(out.off_dry + sizeof(float) * dry.size());
    out.off_bias_vals = align16(out.off_bias_ids + sizeof(int32_t) * bids.size());
    out.total = align16(out.off_bias_vals + sizeof(float) * bvals.size());
    hs.blob.assign(out.total, 0);
    std::memcpy(hs.blob.data(), hs.plans.data(), sizeof(RowPlan) * B);
    if (!dry.empty()) std::memcpy(hs.blob.data() + out.off_dry, dry.data(), sizeof(float) * dry.size());
    if (!bids.empty()) {
        std::memcpy(hs.blob.data() + out.off_bias_ids, bids.data(), sizeof(int32_t) * bids.size());
        std::memcpy(hs.blob.data() + out.off_bias_vals, bvals.data(), sizeof(float) * bvals.size());
    }
    return ULTIMA_HSAMP_OK;
}

int validate_batch(const ultima_hsamp_batch* b, int32_t max_rows, int32_t max_vocab) {
    if (b == nullptr || b->params == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->rows < 1 || b->vocab < 1) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->rows > max_rows || b->vocab > max_vocab) return ULTIMA_HSAMP_ERR_CAPACITY;
    if (b->dtype != ULTIMA_HSAMP_F32 && b->dtype != ULTIMA_HSAMP_BF16) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->logits == nullptr || b->u == nullptr || b->token == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->logits_stride < b->vocab) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->hist != nullptr && b->hist_stride < 0) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->hist_len_dev != nullptr && (b->hist == nullptr || b->hist_stride < 1)) return ULTIMA_HSAMP_ERR_INVALID;
    if (b->mask != nullptr && b->mask_stride < (b->vocab + 31) / 32) return ULTIMA_HSAMP_ERR_INVALID;
    if ((b->flags & ~(ULTIMA_HSAMP_WRITEBACK | ULTIMA_HSAMP_STREAM_ONLY)) != 0) return ULTIMA_HSAMP_ERR_INVALID;
    if ((b->flags & ULTIMA_HSAMP_WRITEBACK) && b->dtype != ULTIMA_HSAMP_F32)
        return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    const bool sets = b->topk_idx || b->kept_idx || b->kept_prob;
    if (sets && b->set_cap < 1) return ULTIMA_HSAMP_ERR_INVALID;
    if ((b->kept_idx == nullptr) != (b->kept_prob == nullptr)) return ULTIMA_HSAMP_ERR_INVALID;
    return ULTIMA_HSAMP_OK;
}

void read_overrides(DevCaps& dc) {
    if (const char* ev = std::getenv("ULTIMA_HSAMP_EXACT")) dc.exact_off = ev[0] == '0';
    if (const char* et = std::getenv("ULTIMA_HSAMP_EXACT_TILES")) {
        const int t = std::atoi(et);
        dc.forced_tiles = t == 4 ? 4 : t == 2 ? 2 : 1;
    }
    if (const char* fs = std::getenv("ULTIMA_HSAMP_SLICES")) dc.forced_slices = std::max(1, std::atoi(fs));
}

int plan_run(const DevCaps& dc, const ultima_hsamp_batch* b, const Built& bl, RunPlan& rp) {
    const int B = b->rows, V = b->vocab;
    const int es = b->dtype == ULTIMA_HSAMP_F32 ? 4 : 2;
    rp = RunPlan{};
    rp.B = B;
    rp.V = V;
    // Exact lists (k_stream's EX kernels + k_pick, or k_pick_l when some
    // row's top-k is above 64): every row samples with top-k <= 1024 or is
    // greedy, with penalties that can only lower a logit (logit bias, at most
    // kBlock entries a row, may raise: the stream evaluates those ids on their
    // own), from windows the stream's registers hold, DRY only where its
    // window is also the frequency/presence window. The stream then leaves every
    // candidate with its final key. ULTIMA_HSAMP_EXACT=0 turns it off (the
    // general kernels take every batch).
    const int kmax = std::max(1, bl.kmax);
    rp.kmax = kmax;
    rp.wb = (b->flags & ULTIMA_HSAMP_WRITEBACK) != 0;
    bool exact_ok = (bl.any_sample || bl.any_greedy) && !bl.any_full && kmax <= kLimitK && bl.inv_ok &&
                    (!bl.any_pen || (bl.pen_lowers_nb && !bl.dry_split && bl.max_bias <= kBlock && bl.max_scan <= 8 * kBlock));
    exact_ok = exact_ok && !dc.exact_off;
    // 16-byte loads: aligned rows holding at least one whole chunk
    const bool vec_rows = (reinterpret_cast<uintptr_t>(b->logits) % 16 == 0) && ((b->logits_stride * es) % 16 == 0) &&
                          V >= 16 / es;
    rp.vec = vec_rows;
    // Slicing: enough blocks to fill the CUs, slices of at most one tile.
    // Exact lists over aligned rows take slices of up to two tiles while the
    // batch still gives two blocks per CU: each block's setup, history scan
    // and bound then cover more ids, and k_pick merges fewer lists. Among
    // those slicings, the one whose busiest CU streams the fewest ids, with
    // a block's fixed work counted as kFixedIds ids (blocks spread evenly).
    const int tiles = (V + kTile - 1) / kTile;
    const int S2 = (V + 2 * kTile - 1) / (2 * kTile);
    int S = std::max(1, std::min({kTargetBlocks / B, tiles, kBlock}));
    const int forced_tiles = dc.forced_tiles;
    // bf16 rows: four tiles of them take the registers two f32 tiles take
    const int max_tiles = (vec_rows && b->dtype == ULTIMA_HSAMP_BF16) ? 4 : vec_rows ? 2 : 1;
    const int S4 = (V + 4 * kTile - 1) / (4 * kTile);
    // exact lists with top-k above 64 (bf16): the largest slices, fewest lists
    const bool four = exact_ok && max_tiles == 4 && (forced_tiles == 4 || (forced_tiles == 0 && kmax > 64));
    if (exact_ok && vec_rows) {
        constexpr int64_t kFixedIds = 4096;
        int want = ((int64_t)B * S2 >= kTwoTileBlocks && S2 < S) ? 2 : 1;
        const bool forced = forced_tiles != 0;   // two tiles asked for: the fewest slices
        if (forced) want = std::min(forced_tiles, 2);
        if (four) want = 1;   // (set below)
        if (want == 2) {
            int best = std::min(S, S2);
            int64_t best_cost = INT64_MAX;
            for (int c = best; !forced && c <= std::min(S, 2 * S2); ++c) {
                const int64_t len = ((V + c - 1) / c + 31) & ~31;
                const int64_t per_cu = ((int64_t)B * c + dc.cus - 1) / dc.cus;
                const int64_t cost = per_cu * (len + kFixedIds);
                if (cost < best_cost) {
                    best_cost = cost;
                    best = c;
                }
            }
            S = best;
        }
    }
    // Large batches: exact lists still need slices their registers hold (two
    // tiles of aligned rows, else one), so they take at least that many.
    if (exact_ok) S = std::max(S, (vec_rows && forced_tiles != 1) ? S2 : tiles);
    if (four) S = S4;
    // diagnostics: a forced slice count (as many slices as the kernels allow)
    if (dc.forced_slices > 0) S = std::min(dc.forced_slices, kBlock);
    const int slice_len = ((V + S - 1) / S + 31) & ~31;
    S = (V + slice_len - 1) / slice_len;
    // block and row indices are divided by S with a 32-bit reciprocal (exact below 2^32 / S)
    if ((uint64_t)(B + 2) * (uint64_t)S * (uint64_t)(S + kXcds) >= (1ull << 32)) return ULTIMA_HSAMP_ERR_CAPACITY;
    rp.S = S;
    rp.slice_len = slice_len;
    // k_merge's LDS candidate buffer: room for 2k (k <= 64), for 4k up to
    // 4096 entries above (each compaction keeps k of them; the general
    // merge's register budget allows two blocks per CU, so LDS is not what
    // limits it), and at least the 1024 entries the finalize's sorts
    // exchange through
    const int buf_cap = kmax > 64 ? std::min(4096, std::max(1024, next_pow2(4 * kmax)))
                                  : std::max(512, next_pow2(2 * kmax));
    const int cand_cap = slice_len;                 // a slice's list holds all its ids
    const int bitmap_words = slice_len / 32;
    rp.buf_cap = buf_cap;
    rp.cand_cap = cand_cap;
    rp.bitmap_words = bitmap_words;
    const size_t statik = 4096;                     // static LDS of the kernels, rounded up
    // k_stream: [penalised-id bitmap] [allowed-id mask words]
    rp.lds = align16(8 * (size_t)bitmap_words);
    if (rp.lds + statik > dc.lds_limit) return ULTIMA_HSAMP_ERR_CAPACITY;
    // k_merge: [penalty table | finalize scratch] [candidate buffer]; the
    // table (load factor <= 1/2) moves to global memory when it does not fit.
    // (the finalize's ids, values and probabilities, 4 B each, and keep flags,
    // 1 B, where the penalty table was; its sort keys use the buffer)
    const size_t regionF = 12 * (size_t)kmax + align16((size_t)kmax);
    const int mhash = bl.any_pen ? std::max(16, next_pow2(2 * bl.max_pen)) : 16;
    rp.mhash = mhash;
    const size_t lds_budget = std::min<size_t>(dc.lds_limit, 64 * 1024) - statik;
    const size_t full_work = full_lds_bytes();   // k_full: window and bucket tables, sort buffer
    const bool gtab = 8 * (size_t)mhash + 8 * (size_t)buf_cap > lds_budget ||
                      8 * (size_t)mhash + 4 * (size_t)bitmap_words > lds_budget ||
                      (bl.any_full && 8 * (size_t)mhash + full_work + statik > dc.lds_limit);
    rp.gtab = gtab;
    rp.full_lds = (gtab ? 0 : 8 * (size_t)mhash) + full_work;
    // k_full's rows: windows of 512 * G ids, at most kFullMaxWin of them
    const int64_t w512 = ((int64_t)V + 511) / 512;
    rp.full_g = (int)std::max<int64_t>(1, (w512 + kFullMaxWin - 1) / kFullMaxWin);
    const int64_t ws = 512 * (int64_t)rp.full_g;
    rp.full_stride = (int)(((int64_t)V + ws - 1) / ws * ws);
    size_t merge_lds = align16(std::max(gtab ? 0 : 8 * (size_t)mhash, regionF)) + 8 * (size_t)buf_cap;
    // k_merge's fast path: [bins 8 KB][list 1 KB][table 12 B/slot | buffer]
    // (flag mode: [bins][list][ids, counts / composites of penalised candidates][buffer])
    const bool fast0 = kmax <= 64 && !gtab && bl.max_scan <= 8 * kBlock && bl.max_bias <= kBlock;
    const bool pen_flag = fast0 && bl.any_pen && bl.pen_lowers;
    // flag mode: after the list, counters of the penalised ids, a bitmap over
    // the vocabulary (16 B per 128 ids) and its rank prefixes (2 B per 128
    // ids), then the buffer of a row read again in full (rare); one merge
    // block per row, so it may use the whole LDS of a CU
    const size_t ngroups = ((size_t)V + 127) / 128;
    const size_t fast_lds = pen_flag ? 9216 + 8 * (size_t)kCntCap + align16(18 * ngroups) + 8 * (size_t)buf_cap
                                     : 9216 + std::max(12 * (size_t)mhash, 8 * (size_t)buf_cap);
    const bool fast = fast0 && fast_lds <= (pen_flag ? dc.lds_limit - statik : lds_budget);
    if (fast) merge_lds = std::max(merge_lds, fast_lds);
    rp.fast = fast;
    rp.pen_flag = fast && pen_flag;
    rp.wb_lds = (gtab ? 0 : 8 * (size_t)mhash) + 4 * (size_t)bitmap_words;
    if (merge_lds + statik > dc.lds_limit || rp.wb_lds + statik > dc.lds_limit ||
        (bl.any_full && rp.full_lds + statik > dc.lds_limit))
        return ULTIMA_HSAMP_ERR_CAPACITY;
    const int nblocks = B * S;
    rp.grid = (nblocks + kXcds - 1) / kXcds * kXcds;
    rp.win = std::max(1, std::min(cand_cap, kMergeWindow / S));
    rp.ex_tiles = slice_len > 2 * kTile ? 4 : slice_len > kTile ? 2 : 1;
    bool exact = exact_ok && slice_len <= kTile * rp.ex_tiles && rp.ex_tiles <= max_tiles;
    // k_stream EX: [history counts (penalties)][allowed-id mask words]
    // [staged chunks: kBlock slots of 32 B (16 B data, the chunk's first id)].
    // The counts take 2 B per slice id, except in four-tile slices (whose
    // 64 KB would hold the blocks per CU to two): there ranked, a bitmap over
    // the slice's ids, a 2 B rank prefix per bitmap word and 2 B entries for
    // the window's distinct ids and the row's bias ids (at most 8 * kBlock
    // and kBlock), at two more block barriers. (the general instantiations for unaligned rows take PEN =
    // true: their counts are cleared and stay zero when no row has penalties)
    rp.cnt_ranked = rp.ex_tiles == 4;
    rp.cnt_bytes = !(bl.any_pen || !vec_rows) ? 0
                   : rp.cnt_ranked ? align16(4 * (size_t)bitmap_words) + align16(2 * (size_t)bitmap_words) +
                                         2 * 9 * (size_t)kBlock
                                   : align16(2 * ((size_t)slice_len + 8));
    rp.stage_off = rp.cnt_bytes + align16(4 * (size_t)bitmap_words);
    rp.lds_ex = rp.stage_off + 32 * (size_t)kBlock;
    // k_pick: each slice's first W entries, NW per thread; W about twice k.
    // k_pick_l (some top-k above 64): every entry through the candidate
    // buffer, [finalize scratch][buffer] as the general merge lays them out.
    if (exact && kmax > 64) {
        rp.win = 1;
        // four k_pick_l blocks per CU: a quarter of the CU's 160 KB for the
        // finalize scratch and a buffer of at least 2k entries (each
        // compaction keeps k), else the general merge's 4k
        const size_t quarter = (size_t)(160 * 1024 / 4) - statik - align16(regionF);
        const int cap4 = (int)(quarter / 8) & ~15;
        if (cap4 >= std::max(1024, 2 * kmax) && cap4 < buf_cap) rp.buf_cap = cap4;
        merge_lds = align16(regionF) + 8 * (size_t)rp.buf_cap;
        if (rp.lds_ex + statik > dc.lds_limit || merge_lds + statik > dc.lds_limit) exact = false;
    } else if (exact) {
        const int w0 = std::min(cand_cap, std::max(32, (2 * kmax + 31) / 32 * 32));
        const int need = (S * w0 + kBlock - 1) / kBlock;
        rp.pick_nw = need <= 4 ? 4 : need <= 8 ? 8 : need <= 12 ? 12 : 16;
        rp.win = std::max(1, std::min(cand_cap, rp.pick_nw * kBlock / S));
        const size_t pick_lds = 8 * std::max<size_t>((size_t)rp.pick_nw * kBlock + 2, (size_t)buf_cap);
        if (rp.lds_ex + statik > dc.lds_limit || pick_lds + statik > dc.lds_limit) exact = false;
        else merge_lds = pick_lds;
    }
    // write-back after the exact lists: k_writeback rebuilds the rows' penalty
    // tables in LDS (no merge kernel leaves a global one)
    if (rp.wb && gtab) exact = false;
    rp.exact = exact;
    rp.merge_lds = merge_lds;
    // scratch
    rp.cand_slots = (size_t)nblocks;
    rp.cand_elems = (size_t)nblocks * (size_t)cand_cap;
    rp.ovf_elems = (size_t)B * kMergeRound;
    rp.gtab_words = gtab ? (size_t)B * 2 * mhash : 0;
    rp.full_elems = bl.any_full ? (size_t)B * rp.full_stride : 0;
    {
        // per-window tables of every row, then (16-byte aligned) 64 lane entries of 4 words per window
        const size_t nWf = (size_t)(rp.full_stride / (512 * rp.full_g));
        rp.fs_elems = bl.any_fpre ? (((size_t)B * FS_TABLES * nWf + 3) & ~(size_t)3) + (size_t)B * nWf * 256 : 0;
    }
    rp.fin_elems = rp.wb ? (size_t)B * kLimitK : 0;
    return ULTIMA_HSAMP_OK;
}

int launch_run(const RunPlan& rp, const Built& bl, const ultima_hsamp_batch* b, const RunBuffers& buf,
               hipStream_t stream, hipEvent_t phase_ev) {
    StreamArgs a{};
    if (const ultima_hsamp_commit* c = buf.commit) {
        a.c_hist = c->hist;
        a.c_stride = c->hist_stride;
        a.c_len = c->hist_len_dev;
        a.c_active = c->active;
        a.c_budget = c->budget;
        a.c_keep = c->keep;
        a.c_nstop = c->n_stop;
        for (int q = 0; q < c->n_stop; ++q) a.c_stop[q] = c->stop_ids[q];
    }
    a.logits = b->logits;
    a.logits_stride = b->logits_stride;
    a.hist = b->hist;
    a.hist_stride = b->hist_stride;
    a.hist_len_dev = b->hist_len_dev;
    a.mask = b->mask;
    a.mask_stride = b->mask_stride;
    a.u = b->u;
    a.plans = reinterpret_cast<const RowPlan*>(buf.blob);
    a.dry_tab = reinterpret_cast<const float*>(buf.blob + bl.off_dry);
    a.bias_ids = reinterpret_cast<const int32_t*>(buf.blob + bl.off_bias_ids);
    a.bias_vals = reinterpret_cast<const float*>(buf.blob + bl.off_bias_vals);
    a.token = b->token;
    a.row_flags = b->row_flags;
    a.topk_idx = b->topk_idx;
    a.topk_count = b->topk_count;
    a.kept_idx = b->kept_idx;
    a.kept_prob = b->kept_prob;
    a.kept_count = b->kept_count;
    a.set_cap = b->set_cap;
    a.rows = rp.B;
    a.vocab = rp.V;
    a.nslices = rp.S;
    a.slice_len = rp.slice_len;
    a.kmax = rp.kmax;
    a.cand_cap = rp.cand_cap;
    a.buf_cap = rp.buf_cap;
    a.mhash_slots = rp.mhash;
    a.bitmap_words = rp.bitmap_words;
    a.blocks_per_xcd = rp.grid / kXcds;
    a.fin_cap = kLimitK;
    a.ovf = buf.ovf;
    a.ovf_cap = kMergeRound;
    a.cand = buf.cand;
    a.cand_n = buf.cand_n;
    a.cand_th = buf.cand_n + buf.cand_slots;
    a.win = rp.win;
    a.win_magic = (uint32_t)((1ull << 32) / (uint64_t)rp.win + 1);
    a.ns_magic = rp.S > 1 ? (uint32_t)((1ull << 32) / (uint64_t)rp.S + 1) : 0u;   // S == 1: the kernels divide by 1 themselves
    a.dtype = b->dtype;
    a.fast = rp.fast ? 1 : 0;
    a.pen_flag = rp.pen_flag ? 1 : 0;
    a.fullv = buf.fullv;
    a.fullp = buf.fullp;
    a.fs_tab = buf.fs_tab;
    a.full_stride = rp.full_stride;
    a.full_g = rp.full_g;
    a.gtab = rp.gtab ? buf.gtab : nullptr;
    a.merge_lds = (uint32_t)rp.merge_lds;
    a.fin_idx = rp.wb ? buf.fin_idx : nullptr;
    a.fin_n = rp.wb ? buf.fin_n : nullptr;
    a.lds_bytes = (uint32_t)(rp.exact ? rp.lds_ex : rp.lds);
    a.exact = rp.exact ? 1 : 0;
    a.mbm_off = (int32_t)(rp.cnt_bytes / 4);
    a.stage_off = (int32_t)rp.stage_off;
    a.hist_direct = (rp.exact && bl.any_pen && b->hist != nullptr && b->hist_stride >= 1 &&
                     b->hist_stride <= 8 * kBlock) ? 1 : 0;
    a.vec_tail = rp.vec ? rp.V % (16 / (b->dtype == ULTIMA_HSAMP_F32 ? 4 : 2)) : 0;
    a.uniform = (bl.any_greedy && !bl.any_sample && !bl.any_full ? 1 : 0) |
                (bl.any_sample && !bl.any_greedy && !bl.any_full ? 2 : 0);
    // In flag mode the sampling rows' stream needs no penalties at all: it
    // bounds on pre-penalty keys, which penalties can only lower, and k_merge
    // finds the penalised candidates' true values (checking the bounds).
    // (exact lists: the lean instantiation when no row is greedy, has a logit
    // bias or counts over two windows)
    const bool lean = !bl.any_greedy && bl.max_bias == 0 && !bl.two_windows;
    if (rp.exact)
        HIP_TRY(launch_stream_ex(a, b->dtype, rp.vec, bl.any_pen, bl.any_mask, rp.ex_tiles, lean, rp.grid, stream));
    else if (bl.any_topk)
        HIP_TRY(launch_stream(a, b->dtype, rp.vec, bl.any_pen, bl.any_pen && !a.pen_flag, bl.any_mask,
                              bl.any_greedy, bl.any_sample, rp.grid, stream));
    if (phase_ev != nullptr) HIP_TRY(hipEventRecord(phase_ev, stream));
    if (!(b->flags & ULTIMA_HSAMP_STREAM_ONLY)) {
        if (rp.exact && rp.kmax > 64) HIP_TRY(launch_pick_l(a, stream));
        else if (rp.exact) HIP_TRY(launch_pick(a, rp.pick_nw, stream));
        else if (bl.any_topk) HIP_TRY(launch_merge(a, stream));
        if (bl.any_full) {
            if (bl.any_fpre) HIP_TRY(launch_full_pre(a, bl.any_fpre_plain, bl.any_fpre_tp, stream));
            if (bl.any_full_gen) HIP_TRY(launch_full(a, (uint32_t)rp.full_lds, stream));
        }
        if (rp.wb) HIP_TRY(launch_writeback(a, rp.grid, (uint32_t)rp.wb_lds, stream));
    }
    return ULTIMA_HSAMP_OK;
}

}  // namespace hsamp

namespace {

// A device copy of hs.blob, reusing a slot that already holds the same bytes.
// Under stream capture nothing is uploaded: the blob must already be resident
// (run the same batch once before capturing), and its slot is pinned so later
// calls never rewrite what the graph reads.
int upload_blob(ultima_hsamp* h, hipStream_t stream, bool capturing, Slot*& used) {
    const std::vector<char>& blob = h->hs.blob;
    const size_t n = blob.size();
    for (auto& s : h->slots) {
        if (s.used && s.size == n && std::memcmp(s.host, blob.data(), n) == 0) {
            if (capturing) s.pinned = true;
            used = &s;
            return ULTIMA_HSAMP_OK;
        }
    }
    if (capturing) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    Slot* pick = nullptr;
    for (int i = 0; i < kSlots && pick == nullptr; ++i) {
        Slot& c = h->slots[(h->next_slot + i) % kSlots];
        if (!c.pinned) {
            pick = &c;
            h->next_slot = (h->next_slot + i + 1) % kSlots;
        }
    }
    if (pick == nullptr) return ULTIMA_HSAMP_ERR_CAPACITY;
    Slot& s = *pick;
    if (s.used) HIP_TRY(hipEventSynchronize(s.ev));   // its last kernel is done with it
    if (s.cap < n) {
        if (s.host) HIP_TRY(hipHostFree(s.host));
        if (s.dev) HIP_TRY(hipFree(s.dev));
        s.host = nullptr;
        s.dev = nullptr;
        const size_t cap = std::max<size_t>(n * 2, 64 * 1024);
        HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&s.host), cap, hipHostMallocDefault));
        HIP_TRY(hipMalloc(reinterpret_cast<void**>(&s.dev), cap));
        s.cap = cap;
    }
    std::memcpy(s.host, blob.data(), n);
    s.size = n;
    s.used = true;
    HIP_TRY(hipMemcpyAsync(s.dev, s.host, n, hipMemcpyHostToDevice, stream));
    used = &s;
    return ULTIMA_HSAMP_OK;
}

// Grow-only device scratch. Growing waits for the device to be idle; once a
// graph has been captured from the handle the old area is kept until destroy.
template <typename T>
int grow(ultima_hsamp* h, bool capturing, T*& ptr, size_t& have, size_t need) {
    if (need <= have) return ULTIMA_HSAMP_OK;
    if (capturing) return ULTIMA_HSAMP_ERR_UNSUPPORTED;   // run once before capturing
    HIP_TRY(hipDeviceSynchronize());
    if (ptr != nullptr) {
        if (h->captured) h->retired.push_back(ptr);
        else HIP_TRY(hipFree(ptr));
    }
    ptr = nullptr;
    have = 0;
    if (hipMalloc(reinterpret_cast<void**>(&ptr), need * sizeof(T)) != hipSuccess) {
        (void)hipGetLastError();
        ptr = nullptr;
        return ULTIMA_HSAMP_ERR_NOMEM;
    }
    have = need;
    return ULTIMA_HSAMP_OK;
}

}  // namespace

extern "C" {

int ultima_hsamp_version(void) { return ULTIMA_HSAMP_VERSION; }

int ultima_hsamp_set_phase_event(ultima_hsamp* h, void* hip_event) {
    if (h == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    h->phase_ev = static_cast<hipEvent_t>(hip_event);
    return ULTIMA_HSAMP_OK;
}

const char* ultima_hsamp_status_str(int s) {
    switch (s) {
        case ULTIMA_HSAMP_OK: return "ok";
        case ULTIMA_HSAMP_ERR_INVALID: return "invalid argument";
        case ULTIMA_HSAMP_ERR_HIP: return "HIP runtime error";
        case ULTIMA_HSAMP_ERR_UNSUPPORTED: return "unsupported by this build";
        case ULTIMA_HSAMP_ERR_NOMEM: return "out of memory";
        case ULTIMA_HSAMP_ERR_CAPACITY: return "exceeds handle or build limits";
        case ULTIMA_HSAMP_ERR_NO_DEVICE: return "no usable gfx950 device";
        default: return "unknown status";
    }
}

void ultima_hsamp_params_default(ultima_hsamp_params* p) {
    if (p == nullptr) return;
    *p = ultima_hsamp_params{};
    p->rep_penalty = 1.1f;
    p->repeat_last_n = 64;
    p->dry_multiplier = 0.8f;
    p->dry_base = 1.75f;
    p->dry_allowed_len = 2;
    p->dry_last_n = 512;
    p->frequency_penalty = 0.0f;
    p->presence_penalty = 0.0f;
    p->temperature = 0.2f;
    p->top_k = 40;
    p->top_p = 0.95f;
    p->min_p = 0.05f;
}

void ultima_hsamp_params_identity(ultima_hsamp_params* p) {
    if (p == nullptr) return;
    ultima_hsamp_params_default(p);
    p->rep_penalty = 1.0f;
    p->repeat_last_n = 0;
    p->dry_multiplier = 0.0f;
    p->dry_last_n = 0;
    p->frequency_penalty = 0.0f;
    p->presence_penalty = 0.0f;
    p->temperature = 1.0f;
    p->top_k = 0;
    p->top_p = 1.0f;
    p->min_p = 0.0f;
}

double ultima_hsamp_uniform_from_u64(uint64_t x) {
    const double r = static_cast<double>(x) / 18446744073709551616.0;
    return r >= 1.0 ? std::nextafter(1.0, 0.0) : r;
}

int ultima_hsamp_create(int device, int32_t max_rows, int32_t max_vocab, ultima_hsamp** out) {
    if (out == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    *out = nullptr;
    if (max_rows < 1 || max_vocab < 1) return ULTIMA_HSAMP_ERR_INVALID;
    if (max_vocab > ULTIMA_HSAMP_MAX_VOCAB) return ULTIMA_HSAMP_ERR_CAPACITY;
    int ndev = 0;
    const hipError_t ce = hipGetDeviceCount(&ndev);
    if (ce != hipSuccess || device < 0 || device >= ndev) {
        hip_fail(ce, "hipGetDeviceCount / device index", __LINE__);
        return ULTIMA_HSAMP_ERR_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    const hipError_t pe = hipGetDeviceProperties(&prop, device);
    if (pe != hipSuccess) {
        hip_fail(pe, "hipGetDeviceProperties", __LINE__);
        return ULTIMA_HSAMP_ERR_NO_DEVICE;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        hip_fail(hipErrorInvalidDevice, prop.gcnArchName, __LINE__);
        return ULTIMA_HSAMP_ERR_NO_DEVICE;
    }
    HIP_TRY(hipSetDevice(device));

    auto* h = new ultima_hsamp();
    h->device = device;
    h->max_rows = max_rows;
    h->max_vocab = max_vocab;
    h->caps.lds_limit = prop.sharedMemPerBlock;
    h->caps.cus = std::max(1, prop.multiProcessorCount);
    read_overrides(h->caps);
    auto fail = [&](int st) {
        ultima_hsamp_destroy(h);
        return st;
    };
#define CREATE_TRY(x)                                   \
    do {                                                \
        hipError_t e_ = (x);                            \
        if (e_ != hipSuccess) return fail(hip_fail(e_, #x, __LINE__)); \
    } while (0)
    CREATE_TRY(hipStreamCreateWithFlags(&h->own_stream, hipStreamNonBlocking));
    for (auto& s : h->slots) CREATE_TRY(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
    // Per-slice counts (8 bytes a slice): at most max(kTargetBlocks,
    // max_rows) slices on the general kernels, up to a slice per tile of
    // every row on the exact lists.
    const size_t tiles = ((size_t)max_vocab + kTile - 1) / kTile;
    const size_t blocks = std::max<size_t>(kTargetBlocks + 8, (size_t)max_rows * tiles + 8);
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->cand_n), blocks * 8));
    h->cand_slots = blocks;
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->fin_idx), (size_t)max_rows * kLimitK * 4));
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->fin_n), (size_t)max_rows * 4));
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->d_row), (size_t)max_vocab * 4 + 64));
    CREATE_TRY(hipHostMalloc(reinterpret_cast<void**>(&h->h_row), (size_t)max_vocab * 4 + 64,
                             hipHostMallocDefault));
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->d_u), 64));
    CREATE_TRY(hipMalloc(reinterpret_cast<void**>(&h->d_tok), 64));
    CREATE_TRY(hipHostMalloc(reinterpret_cast<void**>(&h->h_u), 64, hipHostMallocDefault));
    CREATE_TRY(hipHostMalloc(reinterpret_cast<void**>(&h->h_tok), 64, hipHostMallocDefault));
    CREATE_TRY(hipDeviceSynchronize());
#undef CREATE_TRY
    *out = h;
    return ULTIMA_HSAMP_OK;
}

int ultima_hsamp_destroy(ultima_hsamp* h) {
    if (h == nullptr) return ULTIMA_HSAMP_OK;
    (void)hipSetDevice(h->device);
    (void)hipDeviceSynchronize();
    for (auto& s : h->slots) {
        if (s.host) (void)hipHostFree(s.host);
        if (s.dev) (void)hipFree(s.dev);
        if (s.ev) (void)hipEventDestroy(s.ev);
    }
    for (void* p : {(void*)h->ovf, (void*)h->cand, (void*)h->cand_n,
                    (void*)h->gtab, (void*)h->fullv, (void*)h->fullp, (void*)h->fs_tab,
                    (void*)h->fin_idx,
                    (void*)h->fin_n, (void*)h->d_row, (void*)h->d_hist, (void*)h->d_u, (void*)h->d_tok})
        if (p) (void)hipFree(p);
    for (void* p : h->retired) (void)hipFree(p);
    for (void* p : {(void*)h->h_row, (void*)h->h_hist, (void*)h->h_u, (void*)h->h_tok})
        if (p) (void)hipHostFree(p);
    if (h->own_stream) (void)hipStreamDestroy(h->own_stream);
    (void)hipGetLastError();
    delete h;
    return ULTIMA_HSAMP_OK;
}

namespace {
int run_impl(ultima_hsamp* h, const ultima_hsamp_batch* b, const ultima_hsamp_commit* commit, void* hip_stream);
}

int ultima_hsamp_run(ultima_hsamp* h, const ultima_hsamp_batch* b, void* hip_stream) {
    return run_impl(h, b, nullptr, hip_stream);
}

int ultima_hsamp_run_commit(ultima_hsamp* h, const ultima_hsamp_batch* b, const ultima_hsamp_commit* c,
                            void* hip_stream) {
    if (c == nullptr || c->hist == nullptr || c->hist_len_dev == nullptr || c->active == nullptr)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (c->hist_stride < 2 || c->keep < 1 || (int64_t)c->keep > c->hist_stride / 2 || c->hist_stride > INT32_MAX)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (c->n_stop < 0 || c->n_stop > 8 || (c->n_stop > 0 && c->stop_ids == nullptr)) return ULTIMA_HSAMP_ERR_INVALID;
    if (b != nullptr && (b->flags & ULTIMA_HSAMP_WRITEBACK)) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    return run_impl(h, b, c, hip_stream);
}

namespace {
int run_impl(ultima_hsamp* h, const ultima_hsamp_batch* b, const ultima_hsamp_commit* commit, void* hip_stream) {
    if (h == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    int st = validate_batch(b, h->max_rows, h->max_vocab);
    if (st != ULTIMA_HSAMP_OK) return st;
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    Built bl;
    st = build_blob(h->hs, b, bl);
    if (st != ULTIMA_HSAMP_OK) return st;
    // a compaction to fewer ids than the longest penalty window would drop ids
    // the reference's unbounded history still holds in that window
    if (commit != nullptr && bl.any_pen && commit->keep < bl.max_scan) return ULTIMA_HSAMP_ERR_INVALID;
    RunPlan rp;
    st = plan_run(h->caps, b, bl, rp);
    if (st != ULTIMA_HSAMP_OK) return st;
    if (rp.cand_slots > h->cand_slots) return ULTIMA_HSAMP_ERR_CAPACITY;   // slice counts beyond the handle's

    hipStreamCaptureStatus cap_status = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(stream, &cap_status));
    const bool capturing = cap_status != hipStreamCaptureStatusNone;
    st = grow(h, capturing, h->ovf, h->ovf_elems, rp.ovf_elems);
    if (st == ULTIMA_HSAMP_OK) st = grow(h, capturing, h->cand, h->cand_elems, rp.cand_elems);
    if (st == ULTIMA_HSAMP_OK && rp.gtab_words) st = grow(h, capturing, h->gtab, h->gtab_words, rp.gtab_words);
    if (st == ULTIMA_HSAMP_OK && rp.full_elems) {
        st = grow(h, capturing, h->fullv, h->fullv_elems, rp.full_elems);
        if (st == ULTIMA_HSAMP_OK) st = grow(h, capturing, h->fullp, h->fullp_elems, rp.full_elems);
        if (st == ULTIMA_HSAMP_OK && rp.fs_elems) st = grow(h, capturing, h->fs_tab, h->fs_elems, rp.fs_elems);
    }
    if (st != ULTIMA_HSAMP_OK) return st;

    Slot* slot = nullptr;
    st = upload_blob(h, stream, capturing, slot);
    if (st != ULTIMA_HSAMP_OK) return st;
    if (capturing) h->captured = true;

    RunBuffers buf;
    buf.cand = h->cand;
    buf.cand_n = h->cand_n;
    buf.cand_slots = h->cand_slots;
    buf.ovf = h->ovf;
    buf.gtab = h->gtab;
    buf.fullv = h->fullv;
    buf.fullp = h->fullp;
    buf.fs_tab = h->fs_tab;
    buf.fin_idx = h->fin_idx;
    buf.fin_n = h->fin_n;
    buf.blob = slot->dev;
    buf.commit = commit;
    st = launch_run(rp, bl, b, buf, stream, h->phase_ev);
    if (st != ULTIMA_HSAMP_OK) return st;
    if (!capturing) HIP_TRY(hipEventRecord(slot->ev, stream));
    return ULTIMA_HSAMP_OK;
}
}  // namespace

int ultima_hsamp_query_kernels(ultima_hsamp* h, const ultima_hsamp_batch* b, uint32_t* kernels) {
    if (h == nullptr || kernels == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    int st = validate_batch(b, h->max_rows, h->max_vocab);
    if (st != ULTIMA_HSAMP_OK) return st;
    Built bl;
    st = build_blob(h->hs, b, bl);
    if (st != ULTIMA_HSAMP_OK) return st;
    RunPlan rp;
    st = plan_run(h->caps, b, bl, rp);
    if (st != ULTIMA_HSAMP_OK) return st;
    uint32_t k = 0;
    if (rp.exact) k |= ULTIMA_HSAMP_KERNELS_EXACT;
    else if (bl.any_topk) k |= ULTIMA_HSAMP_KERNELS_GENERAL;
    if (bl.any_full) k |= ULTIMA_HSAMP_KERNELS_FULL;
    if (rp.wb) k |= ULTIMA_HSAMP_KERNELS_WRITEBACK;
    *kernels = k;
    return ULTIMA_HSAMP_OK;
}

int ultima_hsamp_read_probe(ultima_hsamp* h, const ultima_hsamp_batch* b, float* out, void* hip_stream) {
    if (h == nullptr || out == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    int st = validate_batch(b, h->max_rows, h->max_vocab);
    if (st != ULTIMA_HSAMP_OK) return st;
    HIP_TRY(hipSetDevice(h->device));
    Built bl;
    st = build_blob(h->hs, b, bl);
    if (st != ULTIMA_HSAMP_OK) return st;
    RunPlan rp;
    st = plan_run(h->caps, b, bl, rp);
    if (st != ULTIMA_HSAMP_OK) return st;
    const int tiles = (rp.slice_len + kTile - 1) / kTile;
    if (!rp.vec || tiles > 2) return ULTIMA_HSAMP_ERR_UNSUPPORTED;
    StreamArgs a{};
    a.logits = b->logits;
    a.logits_stride = b->logits_stride;
    a.rows = rp.B;
    a.vocab = rp.V;
    a.nslices = rp.S;
    a.slice_len = rp.slice_len;
    a.blocks_per_xcd = rp.grid / kXcds;
    a.ns_magic = rp.S > 1 ? (uint32_t)((1ull << 32) / (uint64_t)rp.S + 1) : 0u;
    a.vec_tail = rp.V % (16 / (b->dtype == ULTIMA_HSAMP_F32 ? 4 : 2));
    HIP_TRY(launch_read_probe(a, b->dtype, tiles, rp.grid, out, static_cast<hipStream_t>(hip_stream)));
    return ULTIMA_HSAMP_OK;
}

int ultima_hsamp_sample_host(ultima_hsamp* h, float* logits, int32_t vocab,
                             const ultima_hsamp_params* params, const int32_t* hist,
                             const int32_t* bias_ids, const float* bias_vals, double u,
                             int writeback, int32_t* token_out) {
    if (h == nullptr || logits == nullptr || params == nullptr || token_out == nullptr)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (vocab < 1) return ULTIMA_HSAMP_ERR_INVALID;
    if (vocab > h->max_vocab) return ULTIMA_HSAMP_ERR_CAPACITY;
    if (params->hist_len < 0 || (params->hist_len > 0 && hist == nullptr)) return ULTIMA_HSAMP_ERR_INVALID;
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t s = h->own_stream;
    const size_t L = (size_t)params->hist_len;
    if (L > h->hist_cap) {
        if (h->d_hist) HIP_TRY(hipFree(h->d_hist));
        if (h->h_hist) HIP_TRY(hipHostFree(h->h_hist));
        h->d_hist = nullptr;
        h->h_hist = nullptr;
        h->hist_cap = 0;
        const size_t cap = std::max<size_t>(L, 1024);
        HIP_TRY(hipMalloc(reinterpret_cast<void**>(&h->d_hist), cap * 4));
        HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&h->h_hist), cap * 4, hipHostMallocDefault));
        h->hist_cap = cap;
    }
    std::memcpy(h->h_row, logits, (size_t)vocab * 4);
    HIP_TRY(hipMemcpyAsync(h->d_row, h->h_row, (size_t)vocab * 4, hipMemcpyHostToDevice, s));
    if (L > 0) {
        std::memcpy(h->h_hist, hist, L * 4);
        HIP_TRY(hipMemcpyAsync(h->d_hist, h->h_hist, L * 4, hipMemcpyHostToDevice, s));
    }
    *h->h_u = u;
    HIP_TRY(hipMemcpyAsync(h->d_u, h->h_u, 8, hipMemcpyHostToDevice, s));
    ultima_hsamp_params p = *params;
    p.bias_offset = 0;
    ultima_hsamp_batch b{};
    b.rows = 1;
    b.vocab = vocab;
    b.dtype = ULTIMA_HSAMP_F32;
    b.flags = writeback ? ULTIMA_HSAMP_WRITEBACK : 0u;
    b.logits = h->d_row;
    b.logits_stride = ((int64_t)vocab + 3) & ~int64_t(3);
    b.hist = L > 0 ? h->d_hist : nullptr;
    b.hist_stride = (int64_t)L;
    b.u = h->d_u;
    b.params = &p;
    b.bias_ids = params->bias_count > 0 ? bias_ids + params->bias_offset : nullptr;
    b.bias_vals = params->bias_count > 0 ? bias_vals + params->bias_offset : nullptr;
    b.token = h->d_tok;
    int st = ultima_hsamp_run(h, &b, s);
    if (st != ULTIMA_HSAMP_OK) {
        (void)hipStreamSynchronize(s);
        return st;
    }
    HIP_TRY(hipMemcpyAsync(h->h_tok, h->d_tok, 4, hipMemcpyDeviceToHost, s));
    if (writeback) HIP_TRY(hipMemcpyAsync(h->h_row, h->d_row, (size_t)vocab * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (writeback) std::memcpy(logits, h->h_row, (size_t)vocab * 4);
    *token_out = *h->h_tok;
    return ULTIMA_HSAMP_OK;
}

}  // extern "C"
