// Host-side pieces of one sampler run shared by the two entry points that
// launch kernels: ultima_hsamp_run() (scratch owned by a handle, grown on
// demand) and ultima_hsamp_run_noalloc() (scratch carved from a fixed device
// array). Planning is pure host arithmetic; launching takes the buffers as
// arguments, so the two entry points differ only in where the buffers live.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <tuple>
#include <vector>

#include "hsamp_plan.h"
#include "ultima_hsamp.h"

namespace hsamp {

// What a device offers the kernels, and the diagnostics overrides of the
// kernel choice (read from the environment once, when a handle is created).
struct DevCaps {
    size_t lds_limit = 0;   // LDS bytes one block may use
    int cus = 256;          // compute units
    bool exact_off = false; // ULTIMA_HSAMP_EXACT=0: the general kernels take every batch
    int forced_tiles = 0;   // ULTIMA_HSAMP_EXACT_TILES: 1, 2 or 4 tiles per exact slice (0: the library's choice)
    int forced_slices = 0;  // ULTIMA_HSAMP_SLICES: slices per row (0: the library's choice)
};

// The ULTIMA_HSAMP_EXACT / _EXACT_TILES / _SLICES overrides into dc.
void read_overrides(DevCaps& dc);

// Host buffers one run fills (kept between runs so that their capacity is reused).
struct HostScratch {
    std::vector<char> blob;
    std::vector<RowPlan> plans;
    std::vector<float> dry;
    std::vector<int32_t> bias_ids;
    std::vector<float> bias_vals;
    std::vector<std::pair<int32_t, float>> tmp;
    std::vector<std::pair<std::tuple<uint32_t, uint32_t, int32_t, int32_t>, int32_t>> dry_seen;
};

// What the batch's rows ask for, from the reference's stage predicates.
struct Built {
    size_t off_dry = 0, off_bias_ids = 0, off_bias_vals = 0, total = 0;
    int kmax = 0;              // max top_k over rows that select
    int max_pen = 0;           // max over penalty rows of (scan_len + bias entries)
    bool any_pen = false;
    int max_scan = 0;          // max history window over penalty rows
    int max_bias = 0;          // max logit-bias entries over rows
    bool pen_lowers = true;    // every penalty stage can only lower a logit
    bool pen_lowers_nb = true; // every stage but the logit bias can only lower a logit
    bool any_dry = false;      // a row with the DRY stage
    bool inv_ok = true;        // every sampling row has 0 < fl(1/T) < inf
    bool any_mask = false;     // the batch carries an allowed-token mask
    bool any_full = false;     // a sampling row over the whole vocabulary (k_full)
    bool any_topk = false;     // a greedy or top-k row (k_stream + k_merge)
    bool any_greedy = false;   // a greedy row (k_stream's greedy kernel)
    bool any_sample = false;   // a top-k sampling row (k_stream's sampling kernel)
    bool dry_split = false;    // a row whose DRY and frequency/presence windows differ
    bool two_windows = false;  // a row whose repetition and count windows are both on and differ
    bool any_fpre = false;     // a k_full row with a plain transform (RF_FPRE)
    bool any_full_gen = false; // a k_full row without RF_FPRE
    bool any_fpre_plain = false;  // an RF_FPRE row without top-p and min-p
    bool any_fpre_tp = false;     // an RF_FPRE row with top-p or min-p
};

// Kernel choice, slicing, LDS sizes and scratch sizes (in elements) of one run.
struct RunPlan {
    int B = 0, V = 0, S = 1, slice_len = 0, kmax = 1;
    int cand_cap = 0, buf_cap = 0, bitmap_words = 0, mhash = 16, win = 1, pick_nw = 16;
    int ex_tiles = 1, grid = 0, full_stride = 0, full_g = 1;
    bool exact = false, vec = false, gtab = false, fast = false, pen_flag = false, wb = false;
    bool cnt_ranked = false;  // exact lists: history counts by rank (a bitmap over the slice)
    size_t lds = 0, lds_ex = 0, merge_lds = 0, full_lds = 0, wb_lds = 0, cnt_bytes = 0, stage_off = 0;
    // scratch the kernels use
    size_t cand_elems = 0;    // u64 candidate lists, B * S * cand_cap
    size_t cand_slots = 0;    // per-slice counts, then as many bounds (int32 each)
    size_t ovf_elems = 0;     // u64 per-row overflow of k_merge's / k_pick's LDS buffer
    size_t gtab_words = 0;    // uint32 per-row penalty tables (0 when in LDS)
    size_t full_elems = 0;    // f32 fullv and fullp, B * V each (k_full rows)
    size_t fin_elems = 0;     // int32 kept ids for write-back, B * kLimitK (and B counts)
    size_t fs_elems = 0;      // uint32 k_fs_* per-window tables, B * FS_TABLES * windows, then B * windows * 256 lane words
};

// Device scratch of one run.
struct RunBuffers {
    unsigned long long* cand = nullptr;
    int32_t* cand_n = nullptr;    // cand_slots counts, then cand_slots bounds
    size_t cand_slots = 0;
    unsigned long long* ovf = nullptr;
    uint32_t* gtab = nullptr;
    float* fullv = nullptr;
    float* fullp = nullptr;
    uint32_t* fs_tab = nullptr;
    int32_t* fin_idx = nullptr;
    int32_t* fin_n = nullptr;
    const char* blob = nullptr;   // device copy of HostScratch::blob
    const ultima_hsamp_commit* commit = nullptr;   // ultima_hsamp_run_commit's rules, or none
};

// Argument checks of ultima_hsamp_run (limits: max_rows / max_vocab).
int validate_batch(const ultima_hsamp_batch* b, int32_t max_rows, int32_t max_vocab);
// RowPlans + DRY tables + bias entries into hs.blob.
int build_blob(HostScratch& hs, const ultima_hsamp_batch* b, Built& out);
// Kernel choice and sizes (dc carries the diagnostics overrides).
int plan_run(const DevCaps& dc, const ultima_hsamp_batch* b, const Built& bl, RunPlan& rp);
// Launches the run's kernels on `stream` (nothing is allocated or copied).
int launch_run(const RunPlan& rp, const Built& bl, const ultima_hsamp_batch* b, const RunBuffers& buf,
               hipStream_t stream, hipEvent_t phase_ev);
// HIP error -> status (ULTIMA_HSAMP_DEBUG=1 prints the failing call).
int hip_fail(hipError_t e, const char* what, int line);

}  // namespace hsamp
