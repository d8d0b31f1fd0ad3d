/*
 * ultima_hsamp -- C ABI of the MI355X (gfx950) token sampler.
 *
 * This is the boundary a foreign caller binds (ctypes, cgo, JNI, N-API). It
 * replaces the reference's C++ entry points, which have no C ABI of their own:
 *   - ultima::sampler::sample(std::span<float>, const SamplerParams&, SamplerContext&)
 *       /root/reference/include/ultima/sampler/sampler.hpp:83-85,
 *       /root/reference/src/sampler/sampler.cpp:230-277
 *     -> ultima_hsamp_run() for [B, V] batches resident in device memory, and
 *        ultima_hsamp_sample_host() for one row in host memory (B = 1).
 *   - ultima::sampler::argmax(std::span<const float>)
 *       sampler.hpp:88, sampler.cpp:220-228
 *     -> ultima_hsamp_sample_host() with temperature <= 0 and identity knobs.
 *   - SamplerParams and SamplerParams::identity()
 *       sampler.hpp:16-52, sampler.cpp:192-205
 *     -> ultima_hsamp_params, ultima_hsamp_params_default(), ultima_hsamp_params_identity().
 *
 * Semantics per row are the reference's transform ladder, in its order:
 * allowed-token mask (extension) -> logit bias -> repetition penalty -> DRY ->
 * frequency/presence -> (temperature <= 0: argmax, no uniform used) ->
 * temperature -> top-k -> top-p -> min-p -> softmax -> categorical draw.
 * Ties in top-k go to the lower index; ties in top-p go to the lower index.
 * The draw takes a caller-supplied uniform u in [0, 1): the token is the first
 * index whose double-precision running sum of normalised probabilities
 * (index order) is >= u, which is what std::discrete_distribution does with
 * the u it draws from SamplerContext::rng().
 *
 * Errors are returned as negative status codes; nothing throws, nothing aborts.
 * All entry points are thread-safe across handles; one handle must not be used
 * by two threads at once.
 */
#ifndef ULTIMA_HSAMP_H
#define ULTIMA_HSAMP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ULTIMA_HSAMP_VERSION 1

/* Status codes. */
#define ULTIMA_HSAMP_OK 0
#define ULTIMA_HSAMP_ERR_INVALID (-1)     /* bad argument (NULL, size, alignment, NaN knob) */
#define ULTIMA_HSAMP_ERR_HIP (-2)         /* a HIP runtime call failed */
#define ULTIMA_HSAMP_ERR_UNSUPPORTED (-3) /* valid request this build does not implement */
#define ULTIMA_HSAMP_ERR_NOMEM (-4)       /* device or pinned allocation failed */
#define ULTIMA_HSAMP_ERR_CAPACITY (-5)    /* exceeds the limits the handle was created with */
#define ULTIMA_HSAMP_ERR_NO_DEVICE (-6)   /* no usable gfx950 device */

/* Logit element types. */
#define ULTIMA_HSAMP_F32 0
#define ULTIMA_HSAMP_BF16 1

/* ultima_hsamp_batch.flags */
#define ULTIMA_HSAMP_WRITEBACK 1u /* leave logits in the state sample() leaves them (F32 only) */
#define ULTIMA_HSAMP_STREAM_ONLY 0x100u /* diagnostics, no counterpart in the reference: run only the
                                           pass over the logits (no token is written), so that a
                                           caller can time that kernel apart */

/* Per-row outcome bits written to row_flags (when given). */
#define ULTIMA_HSAMP_ROW_GREEDY 1u        /* temperature <= 0: argmax, u unused */
#define ULTIMA_HSAMP_ROW_U_USED 2u        /* the draw read u (T > 0 and V >= 2) */
#define ULTIMA_HSAMP_ROW_CDF_NEAR 4u      /* |cp - u| <= 1e-6 at the chosen boundary */
#define ULTIMA_HSAMP_ROW_NAN 8u           /* a NaN logit was seen (outside the contract) */
#define ULTIMA_HSAMP_ROW_UNIFORM 16u      /* nothing finite was left: uniform draw over V */
#define ULTIMA_HSAMP_ROW_TOPP_NEAR 32u    /* top-p cumulative within 1e-6 of top_p at the cutoff */
#define ULTIMA_HSAMP_ROW_REREAD 64u       /* diagnostics: penalties pushed the top-k below the first
                                             pass's bounds and the row was read again in full */

/* Hard limits of this build. */
#define ULTIMA_HSAMP_MAX_VOCAB (1 << 24)      /* token ids and V below 2^24 */
#define ULTIMA_HSAMP_MAX_WINDOW 32767         /* effective penalty window per row */
#define ULTIMA_HSAMP_MAX_BIAS 4096            /* logit-bias entries per row */

/* One row's knobs: ultima::sampler::SamplerParams (sampler.hpp:16-52) with the
 * logit_bias map given as a slice of the batch's bias arrays and the
 * context's history length given explicitly. size_t knobs are uint64_t. */
typedef struct ultima_hsamp_params {
    float rep_penalty;          /* sampler.hpp:22 */
    float dry_multiplier;       /* sampler.hpp:26 */
    float dry_base;             /* sampler.hpp:27 */
    float frequency_penalty;    /* sampler.hpp:32 */
    float presence_penalty;     /* sampler.hpp:33 */
    float temperature;          /* sampler.hpp:36 */
    float top_p;                /* sampler.hpp:42 */
    float min_p;                /* sampler.hpp:45 */
    uint64_t repeat_last_n;     /* sampler.hpp:23 */
    uint64_t dry_allowed_len;   /* sampler.hpp:28 */
    uint64_t dry_last_n;        /* sampler.hpp:29 */
    uint64_t top_k;             /* sampler.hpp:39 */
    int64_t hist_len;           /* ids in this row's history (SamplerContext::recent()) */
    int64_t bias_offset;        /* first entry of this row in bias_ids/bias_vals */
    int64_t bias_count;         /* entries (unique ids) for this row; 0 = no bias */
} ultima_hsamp_params;

/* One batch. Device pointers are caller-owned device memory on the handle's
 * device; host pointers are read during ultima_hsamp_run() only. */
typedef struct ultima_hsamp_batch {
    int32_t rows;               /* B >= 1 */
    int32_t vocab;              /* V >= 1 */
    int32_t dtype;              /* ULTIMA_HSAMP_F32 or ULTIMA_HSAMP_BF16 */
    uint32_t flags;             /* ULTIMA_HSAMP_WRITEBACK, ULTIMA_HSAMP_STREAM_ONLY */
    void* logits;               /* device [rows, logits_stride] elements of dtype */
    int64_t logits_stride;      /* elements between rows, >= vocab */
    const int32_t* hist;        /* device [rows, hist_stride] ids, oldest first; NULL if unused */
    int64_t hist_stride;        /* >= max hist_len; or 0: one history shared by every row,
                                   row r its first hist_len ids (not with hist_len_dev) */
    const uint32_t* mask;       /* device [rows, mask_stride] words or NULL: bit t of word t>>5 */
    int64_t mask_stride;        /* >= ceil(vocab / 32) */
    const double* u;            /* device [rows] uniforms in [0, 1) */
    const ultima_hsamp_params* params; /* HOST [rows] */
    const int32_t* bias_ids;    /* HOST, indexed by params[r].bias_offset; NULL if no bias */
    const float* bias_vals;     /* HOST, same indexing */
    int32_t* token;             /* device [rows] out: sampled id */
    uint32_t* row_flags;        /* device [rows] out or NULL: ULTIMA_HSAMP_ROW_* bits */
    int32_t* topk_idx;          /* device [rows, set_cap] out or NULL: finite top-k members, index order */
    int32_t* topk_count;        /* device [rows] out or NULL (-1 when top-k is off) */
    int32_t* kept_idx;          /* device [rows, set_cap] out or NULL: ids left before the draw */
    float* kept_prob;           /* device [rows, set_cap] out or NULL: their final probabilities */
    int32_t* kept_count;        /* device [rows] out or NULL */
    int32_t set_cap;            /* capacity of the set outputs per row */
    const int32_t* hist_len_dev; /* device [rows] or NULL: each row's history length, read on the
                                  * device in place of params[r].hist_len (ignored then; a history
                                  * kept on the GPU by ultima_hsamp_history_push): every penalty
                                  * window is taken there, min(its last_n, hist_len_dev[r]) as
                                  * window_slice does, so one plan (and one captured graph) serves
                                  * every step from the first token on. last_n values are capped
                                  * at hist_stride. */
} ultima_hsamp_batch;

typedef struct ultima_hsamp ultima_hsamp;

/* Create a handle on `device` able to run batches of up to max_rows rows of
 * up to max_vocab logits. Allocates the device workspace and pinned staging. */
int ultima_hsamp_create(int device, int32_t max_rows, int32_t max_vocab, ultima_hsamp** out);

/* Release a handle (waits for its outstanding work). NULL is a no-op. */
int ultima_hsamp_destroy(ultima_hsamp* h);

/* Sample every row of `batch`, asynchronously on `hip_stream` (a hipStream_t,
 * NULL = the null stream). Inputs must stay valid and unchanged until the work
 * completes; outputs are valid once it has. Work from one handle must not
 * overlap on two streams. The call may be captured into a HIP graph once the
 * same batch (same knobs, rows and vocab) has run uncaptured on the handle;
 * under capture it allocates and uploads nothing and returns
 * ULTIMA_HSAMP_ERR_UNSUPPORTED if it would have to. A captured graph holds the
 * handle's scratch: once a graph has been captured, a later uncaptured run that
 * needs more scratch allocates a larger area and keeps the old one until
 * ultima_hsamp_destroy(), so earlier graphs stay valid to replay (they must not
 * be replayed after destroy, nor overlap other work of the handle). */
int ultima_hsamp_run(ultima_hsamp* h, const ultima_hsamp_batch* batch, void* hip_stream);

/* One row in HOST memory, synchronously -- sample() of sampler.cpp:230-277 with
 * an explicit uniform. logits (V floats) are staged to the device; with
 * writeback != 0 they are copied back in the state sample() leaves them in.
 * hist: hist_len ids; bias_ids/bias_vals: params->bias_count entries from
 * params->bias_offset (may be NULL when bias_count == 0). */
int ultima_hsamp_sample_host(ultima_hsamp* h, float* logits, int32_t vocab,
                             const ultima_hsamp_params* params, const int32_t* hist,
                             const int32_t* bias_ids, const float* bias_vals, double u,
                             int writeback, int32_t* token_out);

/* SamplerParams{} defaults (sampler.hpp:16-52) and SamplerParams::identity()
 * (sampler.cpp:192-205); history and bias fields are zeroed. */
void ultima_hsamp_params_default(ultima_hsamp_params* p);
void ultima_hsamp_params_identity(ultima_hsamp_params* p);

/* The uniform std::discrete_distribution derives from one mt19937_64 output x:
 * generate_canonical<double, 53> = double(x) / 2^64, clamped below 1. */
double ultima_hsamp_uniform_from_u64(uint64_t x);

/* Text for a status code. */
const char* ultima_hsamp_status_str(int status);

/* ULTIMA_HSAMP_VERSION of the loaded library. */
int ultima_hsamp_version(void);

/* The allocation-free variant of ultima_hsamp_run, ultima_hsamp_run_noalloc, is
 * declared in ultima_hsamp_noalloc.h and exported by its own library. */

/* Diagnostics, no counterpart in the reference: which kernels
 * ultima_hsamp_run() would launch for the batch (nothing is launched), as
 * ULTIMA_HSAMP_KERNELS_* bits: the exact-list pair (k_stream over exact
 * lists + k_pick), the general pair (k_stream + k_merge), the
 * full-vocabulary kernel (k_full), the write-back pass (k_writeback). */
#define ULTIMA_HSAMP_KERNELS_EXACT 1u
#define ULTIMA_HSAMP_KERNELS_GENERAL 2u
#define ULTIMA_HSAMP_KERNELS_FULL 4u
#define ULTIMA_HSAMP_KERNELS_WRITEBACK 8u
int ultima_hsamp_query_kernels(ultima_hsamp* h, const ultima_hsamp_batch* batch, uint32_t* kernels);

/* Diagnostics, no counterpart in the reference: a plain read of the batch's
 * logits with the launch shape ultima_hsamp_run() would use for it (same grid,
 * slices, block order and 16-byte loads; aligned rows only, else
 * ULTIMA_HSAMP_ERR_UNSUPPORTED). Each block writes its slice's maximum to
 * out (device, rows * 256 floats). Its duration is the floor for a pass over
 * these bytes with this launch shape; the benchmark times it beside the
 * stream kernel. Asynchronous on hip_stream. */
int ultima_hsamp_read_probe(ultima_hsamp* h, const ultima_hsamp_batch* batch, float* out, void* hip_stream);

/* Diagnostics, no counterpart in the reference: while set (non-NULL), every
 * ultima_hsamp_run() also records this hipEvent_t on its stream between the
 * stream pass (reads the logits) and the per-row merge, so a caller can time
 * the two kernels apart with its own events. NULL stops it. */
int ultima_hsamp_set_phase_event(ultima_hsamp* h, void* hip_event);

/* ---- Device-side history ------------------------------------------------------
 * The penalties' recent-token window kept on the GPU, one row per sequence,
 * appended with each step's sampled token where it already is (the token
 * output of ultima_hsamp_run), so that a decode loop uploads no history.
 * Replaces, per row, SamplerContext::push_recent(next) after each sample()
 *   /root/reference/src/sampler/sampler.cpp:213 (push_recent),
 *   /root/reference/src/server/http_server.cpp:183, apps/ultima-cli/main.cpp:679 (its callers),
 * for the window the reference intends the KV slot to supply
 * (/root/reference/include/ultima/sampler/sampler.hpp:54-56,
 *  /root/reference/include/ultima/kv_cache/kv_cache.hpp:108-111).
 * Row r holds hist_len_dev[r] ids, oldest first, in hist[r * hist_stride ...].
 * For every row: if it is full (hist_len_dev[r] >= hist_stride) its last `keep`
 * ids are first moved to its front; then tokens[r] is appended and
 * hist_len_dev[r] advanced. Penalties look at most max(repeat_last_n,
 * dry_last_n) ids back, so keep >= that window leaves every result as the
 * reference's unbounded recent_ gives it. 0 < keep <= hist_stride / 2.
 * Pass hist and hist_len_dev to ultima_hsamp_run (batch.hist, batch.hist_len_dev).
 * All pointers are device memory; asynchronous on hip_stream; allocates
 * nothing (it may be captured into a graph with the sampler). */
int ultima_hsamp_history_push(int32_t* hist, int64_t hist_stride, int32_t* hist_len_dev, const int32_t* tokens,
                              int32_t rows, int32_t keep, void* hip_stream);

/* ---- Batched callers ----------------------------------------------------------
 * Multi-slot decode: the server's per-token loop over one sequence
 *   next = sample(logits, params, sctx); if (next < 0) break;
 *   if (next == eos || next == im_end) break; sctx.push_recent(next); ...
 *   if (i + 1 == max_tokens) break;
 *     /root/reference/src/server/http_server.cpp:174-201
 * applied to every slot of a batch at once, after an ultima_hsamp_run over the
 * slots' rows (their device histories: batch.hist, batch.hist_len_dev). For row
 * r: if active[r] == 0, or budget is not NULL and budget[r] <= 0 (a slot started
 * with max_tokens 0 emits nothing), the row has ended: tokens[r] becomes -1,
 * active[r] 0, and nothing else changes; else if tokens[r] < 0 or is one of stop_ids[0 .. n_stop) the row ends
 * (active[r] = 0; the token is not pushed and tokens[r] is left as sampled);
 * else tokens[r] is appended to the row's history as ultima_hsamp_history_push
 * does (same hist_stride / keep rules) and, when budget is not NULL,
 * budget[r] is decremented and the row ends when it reaches 0 (max_tokens).
 * hist, hist_len_dev, tokens, active, budget: device memory; stop_ids: HOST, at
 * most 8. Asynchronous on hip_stream, allocates nothing (graph-capturable). */
int ultima_hsamp_decode_commit(int32_t* hist, int64_t hist_stride, int32_t* hist_len_dev, int32_t* tokens,
                               int32_t* active, int32_t* budget, int32_t rows, int32_t keep,
                               const int32_t* stop_ids, int32_t n_stop, void* hip_stream);

/* The same step as ultima_hsamp_run followed by ultima_hsamp_decode_commit,
 * with the commit's rules applied where each row's token is decided (no
 * kernel of its own): for decode loops whose every step samples and commits.
 * The fields mean what ultima_hsamp_decode_commit's arguments mean; the batch
 * must not ask for write-back (ULTIMA_HSAMP_ERR_UNSUPPORTED). hist and
 * hist_len_dev are normally the batch's own (batch.hist, batch.hist_len_dev):
 * the rows' histories the step samples from are the ones it appends to. */
/* ultima_hsamp_run_commit returns ULTIMA_HSAMP_ERR_INVALID when keep is below
 * the batch's longest penalty window (a compaction would drop ids that window
 * holds in the reference's unbounded history). */
typedef struct ultima_hsamp_commit {
    int32_t* hist;              /* device [rows, hist_stride] */
    int64_t hist_stride;        /* >= 2 */
    int32_t* hist_len_dev;      /* device [rows] */
    int32_t* active;            /* device [rows]: 0 = the row has ended */
    int32_t* budget;            /* device [rows] or NULL: tokens a row may still emit */
    int32_t keep;               /* 1 <= keep <= hist_stride / 2 */
    int32_t n_stop;             /* 0 .. 8 */
    const int32_t* stop_ids;    /* HOST [n_stop] */
} ultima_hsamp_commit;

int ultima_hsamp_run_commit(ultima_hsamp* h, const ultima_hsamp_batch* batch, const ultima_hsamp_commit* commit,
                            void* hip_stream);

/* Block verification: the target model's logits for every position of a
 * drafted block ([block_size][vocab] as a drafter proposes it,
 * /root/reference/include/ultima/model/dspark.hpp:76-91; the reference's host
 * loop for it is open, /root/reference/plan.md:196-197) turned into the tokens
 * that the one-token-at-a-time loop above (sample(), push_recent) would emit
 * on those logits with the same uniforms. Position i (0 <= i < n_pos) is
 * sampled with the sequence's history extended by draft[0 .. i) and uniform
 * u[i]; m is the first i < n_pos - 1 whose sample differs from draft[i], else
 * n_pos - 1. out_tokens[0 .. m] = draft[0 .. m) then position m's sample (the
 * rest -1), *out_count = m + 1. Stop tokens among them are the caller's to
 * act on, as in the loop. */
typedef struct ultima_hsamp_verify {
    int32_t n_pos;              /* positions: drafted tokens + 1; 1 <= n_pos <= the handle's max_rows */
    int32_t vocab;              /* V >= 1 */
    int32_t dtype;              /* ULTIMA_HSAMP_F32 or ULTIMA_HSAMP_BF16 */
    void* logits;               /* device [n_pos, logits_stride]: position i's logits */
    int64_t logits_stride;      /* elements between positions, >= vocab */
    const int32_t* draft;       /* device [n_pos - 1] drafted tokens (may be NULL when n_pos == 1);
                                   at hist + hist_len (the drafts appended to the sequence's ids)
                                   the rows read that one array in place: no prefix rows built */
    const int32_t* hist;        /* device [hist_len]: the sequence's recent ids before the block, oldest first */
    int32_t hist_len;           /* >= 0 */
    const uint32_t* mask;       /* device [n_pos, mask_stride] allowed-token words or NULL */
    int64_t mask_stride;
    const double* u;            /* device [n_pos]: the uniform each position's draw takes */
    const ultima_hsamp_params* params; /* HOST: the sequence's knobs (their hist_len is ignored) */
    const int32_t* bias_ids;    /* HOST, as in ultima_hsamp_batch */
    const float* bias_vals;
    int32_t* work;              /* device, ultima_hsamp_verify_work_ints(n_pos, hist_len) int32s */
    int32_t* out_tokens;        /* device [n_pos] out */
    int32_t* out_count;         /* device [1] out */
    uint32_t* row_flags;        /* device [n_pos] out or NULL: each position's ULTIMA_HSAMP_ROW_* bits */
} ultima_hsamp_verify;

/* int32s of workspace ultima_hsamp_verify_block needs (-1 for invalid sizes). */
int64_t ultima_hsamp_verify_work_ints(int32_t n_pos, int32_t hist_len);

/* Verify one block, asynchronously on hip_stream: one ultima_hsamp_run over the
 * n_pos positions (its capture rules apply) between two small kernels. */
int ultima_hsamp_verify_block(ultima_hsamp* h, const ultima_hsamp_verify* v, void* hip_stream);

/* ---- The logits producer ----------------------------------------------------
 * The model's last step before sampling, on the device: each row's final
 * hidden state through the output rmsnorm, the Hadamard fold when the head is
 * folded, and the lm-head matvec, written as the [rows, vocab] f32 logits that
 * ultima_hsamp_run() samples, with no host round trip. Replaces, per token row,
 * the reference's
 *   kernels::rmsnorm_f32(last, output_norm, x_norm, hidden, rms_eps)
 *   if (head.hadamard_folded && fold)
 *     kernels::hadamard_fold_f32(x_norm, fold_buf, hidden, fold.block, fold.signs_for(hidden))
 *   matvec_dispatch_threaded(pool, head.dtype, head.data, head_in, out_logits, vocab, hidden)
 *   out_logits[i] *= 1 / logit_scale            (when logit_scale is neither 1 nor 0)
 *     /root/reference/src/model/qwen_model.cpp:182-207,
 *     /root/reference/src/model/weight_dispatch.cpp:106-146 (every head type it
 *     dispatches: F32, BF16, Q4_K, Q5_K, Q6_K, Q8_0, Q4_1, Q5_0, PQ2_0),
 *     /root/reference/src/kernels/rmsnorm.cpp:21-52, hadamard.cpp:9-44,
 *     matvec_f32_f32.cpp:22-50, matvec_bf16_f32.cpp:48-68,
 *     matvec_q4k_f32.cpp:108-160, matvec_q5k_f32.cpp:48-80,
 *     matvec_q6k_f32.cpp:99-169, matvec_q8_0_f32.cpp:83-117,
 *     matvec_q4_1_f32.cpp:47-75, matvec_q5_0_f32.cpp:108-150,
 *     matvec_pq2_0_f32.cpp:111-184.
 * The results are the reference's bits: every sum runs in the order of its
 * AVX2 kernels (the F32 / BF16 heads: eight fused multiply-add partials, their
 * horizontal sum, the n % 8 tail; each quantised type: its kernel's own
 * partial-sum layout and dequantisation roundings). Quantised rows are the
 * GGUF blocks back to back (row bytes = H / block values * block bytes); as in
 * the reference, a hidden size that is not a whole number of the type's blocks
 * gives logits of 0. PQ2_0 follows the vectorised path matvec_pq2_0_f32 takes
 * for a call of at least 8 rows (every thread's share of a vocabulary head).
 * All pointers are device memory. */
#define ULTIMA_HSAMP_HEAD_Q4_K 2     /* 256 values in 144 bytes */
#define ULTIMA_HSAMP_HEAD_Q5_K 3     /* 256 values in 176 bytes */
#define ULTIMA_HSAMP_HEAD_Q6_K 4     /* 256 values in 210 bytes */
#define ULTIMA_HSAMP_HEAD_Q8_0 5     /* 32 values in 34 bytes */
#define ULTIMA_HSAMP_HEAD_Q4_1 6     /* 32 values in 20 bytes */
#define ULTIMA_HSAMP_HEAD_Q5_0 7     /* 32 values in 22 bytes */
#define ULTIMA_HSAMP_HEAD_PQ2_0 8    /* 128 values in 34 bytes */
#define ULTIMA_HSAMP_MAX_FOLD_BLOCK 8192
typedef struct ultima_hsamp_head {
    const float* hidden;        /* [rows, hidden_stride] final hidden states */
    int64_t hidden_stride;      /* elements between rows, >= hidden_dim */
    int32_t rows;               /* >= 1 */
    int32_t hidden_dim;         /* H >= 1 */
    int32_t vocab;              /* V >= 1 */
    int32_t weight_dtype;       /* ULTIMA_HSAMP_F32, ULTIMA_HSAMP_BF16 or ULTIMA_HSAMP_HEAD_* */
    const float* norm_scale;    /* [H] output-norm weights */
    float eps;                  /* rms epsilon */
    float logit_scale;          /* logits are multiplied by 1 / logit_scale unless it is 1 or 0 */
    const void* weight;         /* [V, H] row-major head weights (f32, bf16 bit patterns, or GGUF blocks) */
    float* normed;              /* [rows, H] scratch, left holding the head's input: the normed rows,
                                   folded when the head is */
    float* logits;              /* [rows, logits_stride] output */
    int64_t logits_stride;      /* elements between rows, >= V */
    int32_t fold_block;         /* 0: no fold; else the fold's block (a power of two up to
                                   ULTIMA_HSAMP_MAX_FOLD_BLOCK; one that does not divide H leaves
                                   the rows unfolded, as the reference does) */
    const float* fold_signs;    /* [H] +-1 signs applied before the rotation, or NULL */
} ultima_hsamp_head;

/* Runs the head for every row on hip_stream (NULL = the default stream).
 * Allocates nothing. */
int ultima_hsamp_lm_head(const ultima_hsamp_head* head, void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif
