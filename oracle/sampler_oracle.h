/*
 * CPU restatement of the reference token sampler -- TEST INFRASTRUCTURE ONLY.
 *
 * This is the checker the HIP sampler is compared against. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product library never links or calls it.
 *
 * It restates /root/reference/src/sampler/sampler.cpp stage by stage (the
 * function-level citations are in sampler_oracle.cpp) with two additions the
 * reference does not have:
 *   - an allowed-token bitmask (bit t of word t>>5, LSB first); a clear bit
 *     means the token's logit becomes -inf before the logit bias, which is
 *     the same as a -INFINITY logit_bias entry for that token;
 *   - an explicit uniform `u` per row. The reference draws it inside
 *     std::discrete_distribution from SamplerContext::rng(); orc_u_from_seed()
 *     reproduces that draw for a context seeded with `seed`.
 * Tie order is explicit: (value desc, index asc) for top-k and
 * (probability desc, index asc) for top-p. The reference leaves both
 * unspecified (std::partial_sort / std::sort, sampler.cpp:113-114,151-152).
 *
 * Parity pins: see tests/test_oracle_*.py. Every stage has a closed-form,
 * brute-force or library-semantics check, plus a comparison against the
 * reference compiled from its own sources (oracle/_ref) on tie-free inputs.
 */
#ifndef ULTIMA_SAMPLER_ORACLE_H
#define ULTIMA_SAMPLER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors ultima::sampler::SamplerParams (include/ultima/sampler/sampler.hpp:16-52)
 * minus logit_bias (passed as id/value arrays) and seed (replaced by u). */
typedef struct orc_params {
    float    rep_penalty;        /* sampler.hpp:22 */
    uint64_t repeat_last_n;      /* sampler.hpp:23 */
    float    dry_multiplier;     /* sampler.hpp:26 */
    float    dry_base;           /* sampler.hpp:27 */
    uint64_t dry_allowed_len;    /* sampler.hpp:28 */
    uint64_t dry_last_n;         /* sampler.hpp:29 */
    float    frequency_penalty;  /* sampler.hpp:32 */
    float    presence_penalty;   /* sampler.hpp:33 */
    float    temperature;        /* sampler.hpp:36 */
    uint64_t top_k;              /* sampler.hpp:39 */
    float    top_p;              /* sampler.hpp:42 */
    float    min_p;              /* sampler.hpp:45 */
} orc_params;

/* What one row's draw left behind, for comparisons. Arrays are caller-owned
 * with capacity `cap`; counts are the full counts even when they exceed cap. */
typedef struct orc_trace {
    int32_t  cap;
    int32_t  topk_count;   /* finite members of the top-k set, index order */
    int32_t* topk_idx;
    int32_t  kept_count;   /* finite logits left before the draw, index order */
    int32_t* kept_idx;
    float*   kept_prob;    /* final softmax probability of each kept id */
    int32_t  u_consumed;   /* 1 iff the draw read u (T > 0 and V >= 2) */
    int32_t  greedy;       /* 1 iff T <= 0 short-circuited to argmax */
    double   cdf_margin;   /* min |cp - u| over the chosen id and its predecessor */
    double   topp_margin;  /* |cum - top_p| at the top-p cutoff (+inf if unused) */
} orc_trace;

/* One row, in place. `logits` holds V floats and ends in the state the
 * reference leaves it in. hist/hist_len: the context's recent ids (oldest
 * first). mask_words: NULL or ceil(V/32) words. bias ids must be unique.
 * Returns the token id (-1 when V == 0). trace may be NULL. */
int32_t orc_sample_row(float* logits, int64_t V, const orc_params* p,
                       const int32_t* hist, int64_t hist_len,
                       const uint32_t* mask_words,
                       const int32_t* bias_ids, const float* bias_vals, int64_t n_bias,
                       double u, orc_trace* trace);

/* The CPU baseline's per-stage breakdown: rows in order on the calling thread,
 * stage_ns[7] = nanoseconds summed over the rows of [penalties (mask, bias,
 * repetition, DRY, frequency/presence), temperature, top-k, top-p, min-p,
 * softmax, draw]. Same arguments and results as orc_sample_batch. */
void orc_sample_batch_stages(float* logits, int64_t rows, int64_t V, int64_t stride,
                             const orc_params* params, const int32_t* hist, int64_t hist_stride,
                             const int64_t* hist_len, const uint32_t* mask, int64_t mask_stride,
                             const double* u, int32_t* tokens, double* stage_ns);

/* argmax of sampler.cpp:220-228 (first maximum, -1 when empty). */
int32_t orc_argmax(const float* logits, int64_t V);

/* Batch of rows for the CPU baseline: rows split statically over nthreads
 * std::threads. Row r reads logits + r*stride (mutated in place), hist +
 * r*hist_stride (hist_len[r] ids), params[r], mask + r*mask_stride (or none),
 * u[r], and writes tokens[r]. No bias. */
void orc_sample_batch(float* logits, int64_t rows, int64_t V, int64_t stride,
                      const orc_params* params,
                      const int32_t* hist, int64_t hist_stride, const int64_t* hist_len,
                      const uint32_t* mask, int64_t mask_stride,
                      const double* u, int32_t* tokens, int32_t nthreads);

/* u that std::discrete_distribution draws from a fresh std::mt19937_64(seed):
 * generate_canonical<double,53> over one engine call. */
double orc_u_from_seed(uint64_t seed);
/* n-th output (1-based) of std::mt19937_64(seed). */
uint64_t orc_mt19937_64_nth(uint64_t seed, uint64_t n);
/* glibc expf, called through the same std::exp(float) the reference uses. */
float orc_expf(float x);
/* glibc powf, as std::pow(float, float). */
float orc_powf(float x, float y);
/* Fill out[i] = expf(x[i]) for n inputs with nthreads threads. */
void orc_expf_many(const float* x, float* out, int64_t n, int32_t nthreads);

#ifdef __cplusplus
}
#endif
#endif
