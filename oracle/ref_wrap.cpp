// C ABI over the reference's own sampler, for validating the restatement and
// for timing the reference on the host -- TEST INFRASTRUCTURE ONLY.
//
// Compiled together with /root/reference/src/sampler/sampler.cpp, which is
// read where it lies (never copied) by oracle/Makefile into oracle/_ref/.
// Each entry builds a SamplerParams (include/ultima/sampler/sampler.hpp:16-52)
// and a SamplerContext seeded with `seed` holding the history as its recent
// ids (sampler.hpp:57-78), then calls ultima::sampler::sample()
// (src/sampler/sampler.cpp:230-277), so the uniform is the context's own
// mt19937_64 draw.
#include "ultima/sampler/sampler.hpp"

#include <algorithm>
#include <cstdint>
#include <span>
#include <thread>
#include <vector>

#include "sampler_oracle.h"

#define REF_API extern "C" __attribute__((visibility("default")))

namespace {

ultima::sampler::SamplerParams to_params(const orc_params* p, const int32_t* bias_ids,
                                         const float* bias_vals, int64_t n_bias) {
    ultima::sampler::SamplerParams s = ultima::sampler::SamplerParams::identity();
    s.rep_penalty = p->rep_penalty;
    s.repeat_last_n = static_cast<std::size_t>(p->repeat_last_n);
    s.dry_multiplier = p->dry_multiplier;
    s.dry_base = p->dry_base;
    s.dry_allowed_len = static_cast<std::size_t>(p->dry_allowed_len);
    s.dry_last_n = static_cast<std::size_t>(p->dry_last_n);
    s.frequency_penalty = p->frequency_penalty;
    s.presence_penalty = p->presence_penalty;
    s.temperature = p->temperature;
    s.top_k = static_cast<std::size_t>(p->top_k);
    s.top_p = p->top_p;
    s.min_p = p->min_p;
    for (int64_t j = 0; j < n_bias; ++j) s.logit_bias[bias_ids[j]] = bias_vals[j];
    return s;
}

int32_t run_row(float* logits, int64_t V, const ultima::sampler::SamplerParams& s,
                const int32_t* hist, int64_t hist_len, uint64_t seed) {
    ultima::sampler::SamplerContext ctx(seed);
    if (hist != nullptr && hist_len > 0)
        ctx.set_recent(std::span<const int32_t>(hist, static_cast<std::size_t>(hist_len)));
    return ultima::sampler::sample(std::span<float>(logits, static_cast<std::size_t>(V)), s, ctx);
}

}  // namespace

REF_API int32_t ref_sample_row(float* logits, int64_t V, const orc_params* p, const int32_t* hist,
                               int64_t hist_len, const int32_t* bias_ids, const float* bias_vals,
                               int64_t n_bias, uint64_t seed) {
    return run_row(logits, V, to_params(p, bias_ids, bias_vals, n_bias), hist, hist_len, seed);
}

REF_API int32_t ref_argmax(const float* logits, int64_t V) {
    return ultima::sampler::argmax(std::span<const float>(logits, static_cast<std::size_t>(V)));
}

// Rows split statically over nthreads threads; row r uses seeds[r].
REF_API void ref_sample_batch(float* logits, int64_t rows, int64_t V, int64_t stride,
                              const orc_params* params, const int32_t* hist, int64_t hist_stride,
                              const int64_t* hist_len, const uint64_t* seeds, int32_t* tokens,
                              int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const auto s = to_params(&params[r], nullptr, nullptr, 0);
            tokens[r] = run_row(logits + r * stride, V, s, hist ? hist + r * hist_stride : nullptr,
                                hist ? hist_len[r] : 0, seeds[r]);
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
