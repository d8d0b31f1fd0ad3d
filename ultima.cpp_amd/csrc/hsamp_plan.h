// Per-row plan and launch arguments shared by the host API and the kernels.
#pragma once

#include <stdint.h>

#include "ultima_hsamp.h"

namespace hsamp {

// Row outcome bits (ultima_hsamp.h).
constexpr uint32_t ROWF_GREEDY = ULTIMA_HSAMP_ROW_GREEDY;
constexpr uint32_t ROWF_U_USED = ULTIMA_HSAMP_ROW_U_USED;
constexpr uint32_t ROWF_CDF_NEAR = ULTIMA_HSAMP_ROW_CDF_NEAR;
constexpr uint32_t ROWF_NAN = ULTIMA_HSAMP_ROW_NAN;
constexpr uint32_t ROWF_UNIFORM = ULTIMA_HSAMP_ROW_UNIFORM;
constexpr uint32_t ROWF_TOPP_NEAR = ULTIMA_HSAMP_ROW_TOPP_NEAR;
constexpr uint32_t ROWF_REREAD = ULTIMA_HSAMP_ROW_REREAD;

// RowPlan::flags -- which stages run for the row. Each follows the reference's
// own predicate (src/sampler/sampler.cpp line in brackets), evaluated on the host.
enum : uint32_t {
    RF_GREEDY = 1u << 0,  // temperature <= 0: argmax after penalties       [261]
    RF_TEMP = 1u << 1,    // temperature != 1: multiply by fl(1/T)          [101-106]
    RF_REP = 1u << 2,     // rep != 1, repeat_last_n > 0, window non-empty  [44, 239]
    RF_DRY = 1u << 3,     // mult > 0, dry_last_n > 0, window >= 2 ids       [69, 246]
    RF_FP = 1u << 4,      // freq != 0 or presence != 0, window non-empty   [89, 254]
    RF_TOPK = 1u << 5,    // 0 < top_k < V                                  [110, 267]
    RF_TOPP = 1u << 6,    // top_p < 1 and not top_p <= 0                   [147, 270]
    RF_MINP = 1u << 7,    // min_p > 0                                      [168, 273]
    RF_MASK = 1u << 8,    // allowed-token mask given for the batch
    RF_BIAS = 1u << 9,    // logit bias entries present                     [30]
    RF_SINGLE = 1u << 10, // V == 1: one id, top-k off, no uniform drawn   [110, random.tcc:2660]
    RF_FULL = 1u << 11,   // sampling row over the whole vocabulary: top-k off or above kLimitK (k_full)
    RF_DEVWIN = 1u << 12, // the row's history length is read on the device: the windows are taken
                          // there, min(cap, length), from the caps in RowPlan::win_caps
    RF_FPRE = 1u << 13,   // a k_full row with a plain transform (no penalties, no logit bias, no
                          // top-k): its whole-row passes run over many blocks first (k_fs_*)
};

// k_fs_* per-row tables, nW entries each (nW = full_stride / (512 * full_g)):
// window maxima m_w, NaN seen, approximate window sums of exp(x - m_w) (the
// binade predictions' input), the windows' predicted binades / integer
// increments for the exact sum, their
// numerators' sums in double (two entries' space: FS_SD and the one after),
// their counts of ids left in (transformed logit above -inf) and their
// smallest numerator above 0 (float bits; all ones when none). An even number
// of tables keeps the doubles 8-byte aligned.
enum : int {
    FS_MAX = 0, FS_NAN = 1, FS_A = 2, FS_EF = 3, FS_D0 = 4, FS_D1 = 5, FS_SD = 6, FS_CNT = 8, FS_EMIN = 9, FS_TABLES = 10
};

// Hash-table value bits for one token of a slice (penalty bookkeeping).
enum : uint32_t {
    HV_FP_MASK = 0x7fffu,    // occurrences in the frequency/presence window
    HV_DRY_SHIFT = 15,       // occurrences in the DRY window, bits 15..29
    HV_DRY_MASK = 0x7fffu,
    HV_BIAS = 1u << 30,      // a logit-bias entry exists
    HV_REP = 1u << 31,       // id is in the repetition window
};

// Exact lists: per-slice history counts, one 16-bit entry per slice id
// (occurrences in the count window, a logit-bias bit, a repetition-window bit).
enum : uint32_t {
    XC_CNT_MASK = 0x3fffu,
    XC_BIAS = 0x4000u,
    XC_REP = 0x8000u,
};

struct alignas(16) RowPlan {
    float inv_temp;     // fl(1.0f / T) when RF_TEMP, else 1.0f
    float rep;          // repetition penalty
    float freq;         // frequency penalty
    float pres;         // presence penalty
    float top_p;
    float min_p;
    int32_t top_k;      // 0 < k < V when RF_TOPK
    int32_t hist_len;   // L: ids in the row's history
    int32_t rep_win;    // effective windows (suffix lengths), 0 when the stage is off
    int32_t dry_win;
    int32_t fp_win;
    int32_t scan_len;   // max of the three: history suffix each block scans
    int32_t dry_allowed;
    int32_t dry_tab;    // offset of this row's DRY penalty table (dry_win + 1 floats)
    int32_t bias_off;   // offset of this row's sorted bias ids/values in the plan blob
    int32_t bias_cnt;
    uint32_t flags;
    float temp;         // T (sampling rows): a first guess when inverting the temperature
    // RF_DEVWIN: the windows' caps (0: the stage is off): repetition | DRY << 16,
    // then frequency/presence; the window fields above hold the caps too
    uint32_t win_caps[2];
};
static_assert(sizeof(RowPlan) == 80, "RowPlan layout");

// Everything one launch of the stream kernel needs, passed by value.
struct StreamArgs {
    const void* logits;
    int64_t logits_stride;      // elements
    const int32_t* hist;
    int64_t hist_stride;
    const int32_t* hist_len_dev;  // [rows] device history lengths, or NULL: the plans' hist_len
    const uint32_t* mask;
    int64_t mask_stride;        // words
    const double* u;
    const RowPlan* plans;
    const float* dry_tab;
    const int32_t* bias_ids;
    const float* bias_vals;
    int32_t* token;
    uint32_t* row_flags;
    int32_t* topk_idx;
    int32_t* topk_count;
    int32_t* kept_idx;
    float* kept_prob;
    int32_t* kept_count;
    int32_t set_cap;
    int32_t rows;
    int32_t vocab;
    int32_t nslices;            // S slices per row
    int32_t slice_len;          // elements per slice (multiple of 32)
    int32_t kmax;               // max top_k over sampling rows (<= K_LIMIT)
    int32_t cand_cap;           // candidates one slice may leave in global scratch
    int32_t buf_cap;            // LDS candidate buffer entries
    int32_t mhash_slots;        // row penalty table slots in k_merge (power of two)
    int32_t bitmap_words;       // slice_len / 32
    int32_t blocks_per_xcd;     // grid / 8
    int32_t fin_cap;            // entries per row in fin_idx
    unsigned long long* cand;   // [rows * S * cand_cap]
    int32_t* cand_n;            // [rows * S]
    int32_t* cand_th;           // [rows * S] a sampling slice's final survival bound (key)
    int32_t* fin_idx;           // [rows * fin_cap] final kept ids (for writeback)
    int32_t* fin_n;             // [rows]
    unsigned long long* ovf;    // [blocks * ovf_cap] per-block overflow of the LDS buffer
    int32_t ovf_cap;            // one tile of candidates
    int32_t win;                // entries of each slice's list k_merge loads up front
    uint32_t win_magic;         // floor(2^32 / win) + 1: umulhi(g, win_magic) == g / win for g < 2^16
    uint32_t ns_magic;          // floor(2^32 / nslices) + 1: umulhi(g, ns_magic) == g / nslices
                                // for g < 2^32 / nslices (block and row indices)
    int32_t dtype;              // logits element type (0 f32, 1 bf16)
    int32_t fast;               // every row fits k_merge's fast path
    int32_t pen_flag;           // penalties only lower logits: k_stream hands penalised ids over as
                                // flagged candidates (pre-penalty key) instead of leaving them out
    int32_t vec_tail;           // the row's last ids k_merge reads itself (V % chunk with vector loads)
    int32_t uniform;            // bit 0: every row is greedy, bit 1: every row is top-k sampling
    int32_t exact;              // exact lists: k_stream leaves every candidate with its final logit
                                // before temperature (penalties applied), k_pick merges them
    int32_t mbm_off;            // exact lists: words from the LDS base to the slice's mask words
    int32_t stage_off;          // exact lists: bytes from the LDS base to the staged chunks
    int32_t hist_direct;        // exact lists: every history row fits 8 * kBlock ids; k_stream
                                // loads whole rows before the tile, without waiting for the plan
    float* fullv;               // [rows * full_stride] k_full: transformed logits (-inf once removed)
    float* fullp;               // [rows * full_stride] k_full: softmax numerators
    int32_t full_stride;        // k_full: floats per row of fullv / fullp (whole windows of 512 * full_g)
    int32_t full_g;             // k_full: 512-id steps per index-order window
    uint32_t* fs_tab;           // [rows * FS_TABLES * nW] k_fs_* results for k_full's RF_FPRE rows, then
                                // (16-byte aligned) [rows * nW * 64] uint4 lane tables
    uint32_t* gtab;             // [rows * 2 * mhash_slots] penalty tables, or NULL: tables in LDS
    uint32_t merge_lds;         // dynamic LDS of k_merge
    uint32_t lds_bytes;         // dynamic LDS size of the launch
    // ultima_hsamp_run_commit: the decode loop's per-token rules applied
    // where each row's token is decided (c_hist NULL: none)
    int32_t* c_hist;
    int64_t c_stride;
    int32_t* c_len;
    int32_t* c_active;
    int32_t* c_budget;          // NULL: no budgets
    int32_t c_keep;
    int32_t c_nstop;
    int32_t c_stop[8];
};

constexpr int kBlock = 256;        // threads per block (4 wave64)
constexpr int kLimitK = 1024;      // largest top_k the top-k path takes
constexpr int kCntCap = 9 * kBlock;  // k_merge flag mode: distinct penalised ids (fast-path window + bias list)
constexpr int kXcds = 8;           // MI355X: workgroups round-robin over 8 XCDs

}  // namespace hsamp
