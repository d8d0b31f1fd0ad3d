// CPU restatement of the reference token sampler -- TEST INFRASTRUCTURE ONLY.
// See sampler_oracle.h for what it is and who may use it.
//
// Every function cites the reference line range it restates
// (paths relative to the reference root, /root/reference). Build flags matter:
// C++20, -O3, default x86-64 ISA, -ffp-contract=off, no fast-math, so each
// float expression rounds exactly where the reference's does.

#include "sampler_oracle.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <numeric>
#include <random>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

constexpr float kNegInf = -std::numeric_limits<float>::infinity();

struct Ids {
    const int32_t* p;
    std::size_t n;
};

// src/sampler/sampler.cpp:19-24 -- suffix of length last_n (all if shorter, empty if 0).
Ids window_slice(Ids recent, uint64_t last_n) {
    if (last_n == 0 || recent.n == 0) return {nullptr, 0};
    if (last_n >= recent.n) return recent;
    return {recent.p + (recent.n - last_n), static_cast<std::size_t>(last_n)};
}

// Extension (no reference counterpart): a clear mask bit sets the logit to -inf.
void apply_mask(float* l, std::size_t V, const uint32_t* mask) {
    if (mask == nullptr) return;
    for (std::size_t i = 0; i < V; ++i)
        if (((mask[i >> 5] >> (i & 31)) & 1u) == 0u) l[i] = kNegInf;
}

// src/sampler/sampler.cpp:28-36
void apply_logit_bias(float* l, std::size_t V, const int32_t* ids, const float* vals, int64_t n) {
    for (int64_t j = 0; j < n; ++j) {
        const int32_t id = ids[j];
        if (id >= 0 && static_cast<std::size_t>(id) < V) l[id] += vals[j];
    }
}

// src/sampler/sampler.cpp:41-54 -- dedupe the window, then divide positive /
// multiply non-positive logits once per unique id.
void apply_rep_penalty(float* l, std::size_t V, Ids recent, float penalty) {
    if (penalty == 1.0f || recent.n == 0) return;
    std::vector<int32_t> uniq(recent.p, recent.p + recent.n);
    std::sort(uniq.begin(), uniq.end());
    uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
    for (int32_t t : uniq) {
        if (t < 0 || static_cast<std::size_t>(t) >= V) continue;
        float& x = l[t];
        x = (x > 0.0f) ? (x / penalty) : (x * penalty);
    }
}

// src/sampler/sampler.cpp:65-83 -- count ids in the window; ids seen more than
// allowed_len times lose multiplier * powf(base, n - allowed_len).
void apply_dry(float* l, std::size_t V, Ids recent, float multiplier, float base,
               uint64_t allowed_len) {
    if (multiplier <= 0.0f || recent.n < 2) return;
    std::unordered_map<int32_t, std::size_t> counts;
    counts.reserve(recent.n);
    for (std::size_t i = 0; i < recent.n; ++i) counts[recent.p[i]]++;
    for (const auto& [id, n] : counts) {
        if (n <= allowed_len) continue;
        if (id < 0 || static_cast<std::size_t>(id) >= V) continue;
        const float pen = multiplier * std::pow(base, static_cast<float>(n - allowed_len));
        l[id] -= pen;
    }
}

// src/sampler/sampler.cpp:86-99 -- two separately rounded subtractions.
void apply_freq_presence(float* l, std::size_t V, Ids recent, float freq_pen, float presence_pen) {
    if (freq_pen == 0.0f && presence_pen == 0.0f) return;
    std::unordered_map<int32_t, std::size_t> counts;
    counts.reserve(recent.n);
    for (std::size_t i = 0; i < recent.n; ++i) counts[recent.p[i]]++;
    for (const auto& [id, n] : counts) {
        if (id < 0 || static_cast<std::size_t>(id) >= V) continue;
        float& x = l[id];
        x -= static_cast<float>(n) * freq_pen;
        x -= presence_pen;
    }
}

// src/sampler/sampler.cpp:101-106
void apply_temperature(float* l, std::size_t V, float temp) {
    if (temp == 1.0f) return;
    if (temp <= 0.0f) return;
    const float inv = 1.0f / temp;
    for (std::size_t i = 0; i < V; ++i) l[i] *= inv;
}

// src/sampler/sampler.cpp:109-121 -- keep the k largest; ties go to the lower
// index (the reference's partial_sort order among equal logits is unspecified).
bool apply_top_k(float* l, std::size_t V, uint64_t k) {
    if (k == 0 || k >= V) return false;
    std::vector<std::size_t> idx(V);
    std::iota(idx.begin(), idx.end(), 0);
    std::partial_sort(idx.begin(), idx.begin() + static_cast<std::ptrdiff_t>(k), idx.end(),
                      [&](std::size_t a, std::size_t b) {
                          return l[a] > l[b] || (l[a] == l[b] && a < b);
                      });
    std::vector<bool> keep(V, false);
    for (std::size_t i = 0; i < k; ++i) keep[idx[i]] = true;
    for (std::size_t i = 0; i < V; ++i)
        if (!keep[i]) l[i] = kNegInf;
    return true;
}

// src/sampler/sampler.cpp:124-142 -- max-subtracted softmax; -inf entries are
// skipped; the denominator is a float sum in index order.
std::vector<float> softmax_probs(const float* l, std::size_t V) {
    float m = kNegInf;
    for (std::size_t i = 0; i < V; ++i)
        if (l[i] > m) m = l[i];
    if (m == kNegInf) return std::vector<float>(V, 1.0f / static_cast<float>(V));
    std::vector<float> p(V, 0.0f);
    float sum = 0.0f;
    for (std::size_t i = 0; i < V; ++i) {
        if (l[i] == kNegInf) {
            p[i] = 0.0f;
            continue;
        }
        p[i] = std::exp(l[i] - m);
        sum += p[i];
    }
    if (sum <= 0.0f) return p;
    const float inv = 1.0f / sum;
    for (auto& x : p) x *= inv;
    return p;
}

// src/sampler/sampler.cpp:146-164 -- nucleus: sort by probability (ties to
// the lower index), float running sum, keep the shortest prefix with sum >= p.
void apply_top_p(float* l, std::size_t V, float p, double* margin) {
    if (p >= 1.0f || p <= 0.0f) return;
    auto probs = softmax_probs(l, V);
    std::vector<std::size_t> idx(V);
    std::iota(idx.begin(), idx.end(), 0);
    std::sort(idx.begin(), idx.end(), [&](std::size_t a, std::size_t b) {
        return probs[a] > probs[b] || (probs[a] == probs[b] && a < b);
    });
    float cum = 0.0f;
    std::size_t cutoff = idx.size();
    for (std::size_t i = 0; i < idx.size(); ++i) {
        cum += probs[idx[i]];
        if (cum >= p) {
            cutoff = i + 1;
            break;
        }
    }
    if (margin != nullptr) *margin = std::fabs(static_cast<double>(cum) - static_cast<double>(p));
    std::vector<bool> keep(V, false);
    for (std::size_t i = 0; i < cutoff; ++i) keep[idx[i]] = true;
    for (std::size_t i = 0; i < V; ++i)
        if (!keep[i]) l[i] = kNegInf;
}

// src/sampler/sampler.cpp:167-176
void apply_min_p(float* l, std::size_t V, float min_p) {
    if (min_p <= 0.0f) return;
    auto probs = softmax_probs(l, V);
    float max_p = 0.0f;
    for (float x : probs)
        if (x > max_p) max_p = x;
    const float threshold = min_p * max_p;
    for (std::size_t i = 0; i < V; ++i)
        if (probs[i] < threshold) l[i] = kNegInf;
}

// src/sampler/sampler.cpp:178-182 with std::discrete_distribution<int> spelled
// out from libstdc++ 11 (bits/random.tcc:83-89 __normalize, 2656-2677
// _M_initialize, 2695-2713 operator()): probabilities widened to double,
// double sum in index order, each divided by it, double partial sums, last one
// forced to 1.0, then the first index whose partial sum is >= u. Fewer than two
// probabilities: index 0 without drawing.
int32_t draw(const std::vector<float>& probs, double u, orc_trace* tr) {
    const std::size_t V = probs.size();
    if (V < 2) return 0;
    if (tr) tr->u_consumed = 1;
    std::vector<double> q(probs.begin(), probs.end());
    const double sum = std::accumulate(q.begin(), q.end(), 0.0);
    for (auto& x : q) x = x / sum;
    std::vector<double> cp;
    cp.reserve(V);
    std::partial_sum(q.begin(), q.end(), std::back_inserter(cp));
    cp[V - 1] = 1.0;
    const auto pos = std::lower_bound(cp.begin(), cp.end(), u);
    const std::size_t i = static_cast<std::size_t>(pos - cp.begin());
    if (tr) {
        double m = std::numeric_limits<double>::infinity();
        if (i < V) m = std::fabs(cp[i] - u);
        if (i > 0 && i - 1 < V) m = std::min(m, std::fabs(cp[i - 1] - u));
        tr->cdf_margin = m;
    }
    return static_cast<int32_t>(i);
}

void record_kept(const float* l, std::size_t V, orc_trace* tr) {
    if (tr == nullptr) return;
    const auto probs = softmax_probs(l, V);
    int32_t n = 0;
    for (std::size_t i = 0; i < V; ++i) {
        if (l[i] == kNegInf) continue;
        if (n < tr->cap) {
            tr->kept_idx[n] = static_cast<int32_t>(i);
            tr->kept_prob[n] = probs[i];
        }
        ++n;
    }
    tr->kept_count = n;
}

}  // namespace

extern "C" {

// src/sampler/sampler.cpp:220-228
int32_t orc_argmax(const float* logits, int64_t V) {
    if (V <= 0) return -1;
    std::size_t best = 0;
    float best_v = logits[0];
    for (std::size_t i = 1; i < static_cast<std::size_t>(V); ++i) {
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    }
    return static_cast<int32_t>(best);
}

}  // extern "C"

namespace {

// Stage clock for the CPU baseline's breakdown: adds the time since the last
// mark to slot i (nothing when no accumulator is given).
struct StageClock {
    double* acc;
    std::chrono::steady_clock::time_point t;
    explicit StageClock(double* a) : acc(a) {
        if (acc) t = std::chrono::steady_clock::now();
    }
    void mark(int i) {
        if (!acc) return;
        const auto n = std::chrono::steady_clock::now();
        acc[i] += std::chrono::duration<double, std::nano>(n - t).count();
        t = n;
    }
};

// src/sampler/sampler.cpp:230-277 -- the fixed stage order. stage_ns (optional):
// nanoseconds per stage, added to [penalties, temperature, top-k, top-p,
// min-p, softmax, draw]; the kept-set trace is taken outside the clock.
int32_t sample_row_impl(float* logits, int64_t V_, const orc_params* p, const int32_t* hist,
                        int64_t hist_len, const uint32_t* mask_words, const int32_t* bias_ids,
                        const float* bias_vals, int64_t n_bias, double u, orc_trace* tr,
                        double* stage_ns) {
    if (tr) {
        tr->topk_count = -1;
        tr->kept_count = 0;
        tr->u_consumed = 0;
        tr->greedy = 0;
        tr->cdf_margin = std::numeric_limits<double>::infinity();
        tr->topp_margin = std::numeric_limits<double>::infinity();
    }
    if (V_ <= 0) return -1;
    const std::size_t V = static_cast<std::size_t>(V_);
    const Ids recent{hist, static_cast<std::size_t>(hist_len > 0 ? hist_len : 0)};
    StageClock clk(stage_ns);

    apply_mask(logits, V, mask_words);
    apply_logit_bias(logits, V, bias_ids, bias_vals, n_bias);
    if (p->rep_penalty != 1.0f && p->repeat_last_n > 0)
        apply_rep_penalty(logits, V, window_slice(recent, p->repeat_last_n), p->rep_penalty);
    if (p->dry_multiplier > 0.0f && p->dry_last_n > 0)
        apply_dry(logits, V, window_slice(recent, p->dry_last_n), p->dry_multiplier, p->dry_base,
                  p->dry_allowed_len);
    if (p->frequency_penalty != 0.0f || p->presence_penalty != 0.0f) {
        const uint64_t win = std::max(p->repeat_last_n, p->dry_last_n);
        apply_freq_presence(logits, V, window_slice(recent, win), p->frequency_penalty,
                            p->presence_penalty);
    }
    clk.mark(0);
    if (p->temperature <= 0.0f) {
        if (tr) tr->greedy = 1;
        const int32_t t = orc_argmax(logits, V_);
        clk.mark(6);
        return t;
    }
    apply_temperature(logits, V, p->temperature);
    clk.mark(1);
    const bool topk = p->top_k > 0 && apply_top_k(logits, V, p->top_k);
    clk.mark(2);
    if (topk && tr) {
        int32_t n = 0;
        for (std::size_t i = 0; i < V; ++i) {
            if (logits[i] == kNegInf) continue;
            if (n < tr->cap) tr->topk_idx[n] = static_cast<int32_t>(i);
            ++n;
        }
        tr->topk_count = n;
    }
    if (p->top_p < 1.0f) apply_top_p(logits, V, p->top_p, tr ? &tr->topp_margin : nullptr);
    clk.mark(3);
    if (p->min_p > 0.0f) apply_min_p(logits, V, p->min_p);
    clk.mark(4);
    record_kept(logits, V, tr);
    StageClock clk2(stage_ns);
    const auto probs = softmax_probs(logits, V);
    clk2.mark(5);
    const int32_t t = draw(probs, u, tr);
    clk2.mark(6);
    return t;
}

}  // namespace

extern "C" {

int32_t orc_sample_row(float* logits, int64_t V_, const orc_params* p, const int32_t* hist,
                       int64_t hist_len, const uint32_t* mask_words, const int32_t* bias_ids,
                       const float* bias_vals, int64_t n_bias, double u, orc_trace* tr) {
    return sample_row_impl(logits, V_, p, hist, hist_len, mask_words, bias_ids, bias_vals, n_bias, u, tr,
                           nullptr);
}

// One thread, rows in order, with the per-stage clock: stage_ns[7] gets the
// nanoseconds of [penalties, temperature, top-k, top-p, min-p, softmax, draw]
// summed over the rows (mask and bias count as penalties).
void orc_sample_batch_stages(float* logits, int64_t rows, int64_t V, int64_t stride,
                             const orc_params* params, const int32_t* hist, int64_t hist_stride,
                             const int64_t* hist_len, const uint32_t* mask, int64_t mask_stride,
                             const double* u, int32_t* tokens, double* stage_ns) {
    for (int i = 0; i < 7; ++i) stage_ns[i] = 0.0;
    for (int64_t r = 0; r < rows; ++r)
        tokens[r] = sample_row_impl(logits + r * stride, V, &params[r], hist ? hist + r * hist_stride : nullptr,
                                    hist ? hist_len[r] : 0, mask ? mask + r * mask_stride : nullptr, nullptr,
                                    nullptr, 0, u[r], nullptr, stage_ns);
}

void orc_sample_batch(float* logits, int64_t rows, int64_t V, int64_t stride,
                      const orc_params* params, const int32_t* hist, int64_t hist_stride,
                      const int64_t* hist_len, const uint32_t* mask, int64_t mask_stride,
                      const double* u, int32_t* tokens, int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            tokens[r] = orc_sample_row(logits + r * stride, V, &params[r],
                                       hist ? hist + r * hist_stride : nullptr,
                                       hist ? hist_len[r] : 0,
                                       mask ? mask + r * mask_stride : nullptr, nullptr, nullptr,
                                       0, u[r], nullptr);
        }
    };
    if (nthreads == 1 || rows <= 1) {
        work(0, rows);
        return;
    }
    std::vector<std::thread> th;
    const int64_t per = (rows + nthreads - 1) / nthreads;
    for (int32_t t = 0; t < nthreads; ++t) {
        const int64_t r0 = t * per, r1 = std::min<int64_t>(rows, r0 + per);
        if (r0 >= r1) break;
        th.emplace_back(work, r0, r1);
    }
    for (auto& x : th) x.join();
}

// libstdc++ 11 bits/random.tcc:3346-3376 (generate_canonical<double, 53>) on one
// mt19937_64 output, as discrete_distribution::operator() draws it through
// __detail::_Adaptor (bits/random.h:164-196).
double orc_u_from_seed(uint64_t seed) {
    std::mt19937_64 rng(seed);
    std::__detail::_Adaptor<std::mt19937_64, double> aurng(rng);
    return aurng();
}

uint64_t orc_mt19937_64_nth(uint64_t seed, uint64_t n) {
    std::mt19937_64 rng(seed);
    uint64_t x = 0;
    for (uint64_t i = 0; i < n; ++i) x = rng();
    return x;
}

float orc_expf(float x) { return std::exp(x); }
float orc_powf(float x, float y) { return std::pow(x, y); }

void orc_expf_many(const float* x, float* out, int64_t n, int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    std::vector<std::thread> th;
    const int64_t per = (n + nthreads - 1) / nthreads;
    for (int32_t t = 0; t < nthreads; ++t) {
        const int64_t a = t * per, b = std::min<int64_t>(n, a + per);
        if (a >= b) break;
        th.emplace_back([=] {
            for (int64_t i = a; i < b; ++i) out[i] = std::exp(x[i]);
        });
    }
    for (auto& t : th) t.join();
}

}  // extern "C"
