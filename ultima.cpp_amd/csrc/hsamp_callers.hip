// Batched callers of the sampler: the server's decode loop over many KV slots
// at once, and verification of a drafted block of tokens.
//
// Multi-slot decode (ultima_hsamp_decode_commit). The reference serves one
// sequence at a time: per token, sample(), stop on -1, eos or im_end, else
// push_recent(next) and continue until max_tokens
// (src/server/http_server.cpp:174-201). Here a step samples every slot's row
// in one ultima_hsamp_run (each row its own knobs and its device history) and
// k_decode_commit then applies the loop's rules to every row at once: a row
// that is no longer active gets token -1 and is left alone; a stop token ends
// the row (not pushed, as the reference breaks before push_recent); any other
// token is appended to the row's history, and the row's budget, when given,
// counts it and ends the row at zero. The shapes stay fixed from step to
// step, so a step can be captured into a graph and replayed.
//
// Block verification (ultima_hsamp_verify_block). A drafter proposes a block
// of tokens and the target model's logits for every position of the block
// come back at once ([block_size][vocab], include/ultima/model/dspark.hpp:
// 76-91; the reference's host loop for it is still open, plan.md:196-197).
// The emitted tokens are exactly those of the reference's one-token-at-a-time
// loop on the target logits with the same uniforms: position i is sampled
// with the history extended by the drafts before it (which the loop would
// have pushed had they been accepted) and its own uniform, all positions in
// one batch; the block is accepted up to the first position whose sample
// differs from its draft, and that sample (or, when every draft matches, the
// last position's) is emitted after them. Drafts stored right after the
// sequence's ids are read in place: every position's history is a prefix of
// that one array.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "ultima_hsamp.h"

namespace hsamp {
namespace {

constexpr int kMaxStop = 8;

struct StopIds {
    int32_t id[kMaxStop];
};

__global__ __launch_bounds__(64) void k_decode_commit(int32_t* __restrict__ hist, int64_t stride,
                                                      int32_t* __restrict__ len, int32_t* __restrict__ tokens,
                                                      int32_t* __restrict__ active, int32_t* __restrict__ budget,
                                                      int rows, int keep, StopIds stop, int n_stop) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    // the row's token, state, length and budget go out together: one memory
    // round trip before any decision
    const int32_t tok = tokens[r];
    const int32_t act = active[r];
    int L = len[r];
    const int32_t bud = budget != nullptr ? budget[r] : 0;
    if (act == 0) {
        if (threadIdx.x == 0) tokens[r] = -1;
        return;
    }
    // a slot whose budget is spent emits nothing (max_tokens 0: the reference's
    // loop body never runs)
    if (budget != nullptr && bud <= 0) {
        if (threadIdx.x == 0) {
            tokens[r] = -1;
            active[r] = 0;
        }
        return;
    }
    bool end = tok < 0;
    for (int i = 0; i < n_stop; ++i) end = end || tok == stop.id[i];
    if (end) {
        if (threadIdx.x == 0) active[r] = 0;
        return;
    }
    int32_t* h = hist + (int64_t)r * stride;
    L = L < 0 ? 0 : L;
    if (L >= stride) {
        // [stride - keep, stride) -> [0, keep); keep <= stride / 2, so the
        // ranges overlap at most in h[keep], which thread 0 reads (i = 0)
        // before it writes it below
        const int64_t from = stride - keep;
        // eight ids per thread in flight, then their stores (the ranges do not
        // overlap: from >= keep)
        for (int i0 = 0; i0 < keep; i0 += 8 * 64) {
            int32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * 64 + (int)threadIdx.x;
                v[j] = h[from + min(i, keep - 1)];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * 64 + (int)threadIdx.x;
                if (i < keep) h[i] = v[j];
            }
        }
        L = keep;
    }
    if (threadIdx.x == 0) {
        h[L] = tok;
        len[r] = L + 1;
        if (budget != nullptr) {
            const int32_t b = bud - 1;
            budget[r] = b;
            if (b <= 0) active[r] = 0;
        }
    }
}

// Row i of the prefix histories: the sequence's ids, then drafts 0 .. i-1.
__global__ __launch_bounds__(256) void k_verify_prefix(const int32_t* __restrict__ hist, int hist_len,
                                                       const int32_t* __restrict__ draft, int32_t* __restrict__ work,
                                                       int64_t stride) {
    const int i = blockIdx.x;
    int32_t* row = work + (int64_t)i * stride;
    for (int j = threadIdx.x; j < hist_len + i; j += 256) row[j] = j < hist_len ? hist[j] : draft[j - hist_len];
}

// The first position whose sample differs from its draft (or the last
// position), then the emitted tokens: the drafts before it and its sample.
__global__ __launch_bounds__(64) void k_verify_accept(const int32_t* __restrict__ draft,
                                                      const int32_t* __restrict__ sampled, int n_pos,
                                                      int32_t* __restrict__ out_tokens, int32_t* __restrict__ out_count) {
    const int lane = threadIdx.x;
    int m = n_pos - 1;
    for (int b = 0; b < n_pos - 1; b += 64) {
        const int i = b + lane;
        const bool miss = i < n_pos - 1 && sampled[i] != draft[i];
        const unsigned long long bal = __ballot(miss);
        if (bal != 0ull) {
            m = b + __ffsll((long long)bal) - 1;
            break;
        }
    }
    for (int j = lane; j < n_pos; j += 64) out_tokens[j] = j < m ? draft[j] : (j == m ? sampled[m] : -1);
    if (lane == 0) *out_count = m + 1;
}

}  // namespace
}  // namespace hsamp

extern "C" int ultima_hsamp_decode_commit(int32_t* hist, int64_t hist_stride, int32_t* hist_len_dev, int32_t* tokens,
                                          int32_t* active, int32_t* budget, int32_t rows, int32_t keep,
                                          const int32_t* stop_ids, int32_t n_stop, void* hip_stream) {
    if (hist == nullptr || hist_len_dev == nullptr || tokens == nullptr || active == nullptr)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (rows < 1 || hist_stride < 2 || keep < 1 || (int64_t)keep > hist_stride / 2 || hist_stride > INT32_MAX)
        return ULTIMA_HSAMP_ERR_INVALID;
    if (n_stop < 0 || n_stop > hsamp::kMaxStop || (n_stop > 0 && stop_ids == nullptr)) return ULTIMA_HSAMP_ERR_INVALID;
    hsamp::StopIds s{};
    for (int i = 0; i < n_stop; ++i) s.id[i] = stop_ids[i];
    hipLaunchKernelGGL(hsamp::k_decode_commit, dim3(rows), dim3(64), 0, static_cast<hipStream_t>(hip_stream), hist,
                       hist_stride, hist_len_dev, tokens, active, budget, (int)rows, (int)keep, s, (int)n_stop);
    return hipGetLastError() == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}

extern "C" int64_t ultima_hsamp_verify_work_ints(int32_t n_pos, int32_t hist_len) {
    if (n_pos < 1 || hist_len < 0) return -1;
    const int64_t stride = std::max<int64_t>(1, (int64_t)hist_len + n_pos - 1);
    return (int64_t)n_pos * stride + n_pos;
}

extern "C" int ultima_hsamp_verify_block(ultima_hsamp* h, const ultima_hsamp_verify* v, void* hip_stream) {
    if (h == nullptr || v == nullptr || v->params == nullptr) return ULTIMA_HSAMP_ERR_INVALID;
    if (v->n_pos < 1 || v->hist_len < 0 || v->vocab < 1) return ULTIMA_HSAMP_ERR_INVALID;
    if (v->logits == nullptr || v->u == nullptr || v->work == nullptr || v->out_tokens == nullptr ||
        v->out_count == nullptr)
        return ULTIMA_HSAMP_ERR_INVALID;
    if ((v->n_pos > 1 && v->draft == nullptr) || (v->hist_len > 0 && v->hist == nullptr))
        return ULTIMA_HSAMP_ERR_INVALID;
    const int n = v->n_pos;
    const int64_t stride = std::max<int64_t>(1, (int64_t)v->hist_len + n - 1);
    if (stride > INT32_MAX) return ULTIMA_HSAMP_ERR_INVALID;
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    int32_t* sampled = v->work + (int64_t)n * stride;
    // Drafts that follow the history in memory (or no history): row i's
    // history is the first hist_len + i ids of that one array, which every
    // row reads in place (batch hist_stride 0); else the prefix rows are built
    // in the workspace.
    const bool in_place = v->hist_len == 0 || n == 1 || v->draft == v->hist + v->hist_len;
    const int32_t* shared = v->hist_len > 0 ? v->hist : v->draft;   // (NULL when both are empty)
    if (!in_place) {
        hipLaunchKernelGGL(hsamp::k_verify_prefix, dim3(n), dim3(256), 0, stream, v->hist, (int)v->hist_len, v->draft,
                           v->work, stride);
        if (hipGetLastError() != hipSuccess) return ULTIMA_HSAMP_ERR_HIP;
    }
    std::vector<ultima_hsamp_params> ps((size_t)n, *v->params);
    for (int i = 0; i < n; ++i) ps[(size_t)i].hist_len = (int64_t)v->hist_len + i;
    ultima_hsamp_batch b{};
    b.rows = n;
    b.vocab = v->vocab;
    b.dtype = v->dtype;
    b.flags = 0;
    b.logits = v->logits;
    b.logits_stride = v->logits_stride;
    b.hist = in_place ? shared : v->work;
    b.hist_stride = in_place ? 0 : stride;
    b.mask = v->mask;
    b.mask_stride = v->mask_stride;
    b.u = v->u;
    b.params = ps.data();
    b.bias_ids = v->bias_ids;
    b.bias_vals = v->bias_vals;
    b.token = sampled;
    b.row_flags = v->row_flags;
    const int st = ultima_hsamp_run(h, &b, hip_stream);
    if (st != ULTIMA_HSAMP_OK) return st;
    hipLaunchKernelGGL(hsamp::k_verify_accept, dim3(1), dim3(64), 0, stream, v->draft, sampled, n, v->out_tokens,
                       v->out_count);
    return hipGetLastError() == hipSuccess ? ULTIMA_HSAMP_OK : ULTIMA_HSAMP_ERR_HIP;
}
