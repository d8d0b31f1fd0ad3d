// ultima::sampler on the HIP backend: the drop-in for the reference's
// src/sampler/sampler.cpp behind the same header. Host code only; every
// sampling decision is made by libultima_hsamp's kernels.
#include "ultima/sampler/sampler.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <random>
#include <vector>

#include "ultima_hsamp.h"

namespace ultima::sampler {

namespace {

constexpr std::int32_t kBatchRows = 1024;  // largest sample_batch()

// One process-wide handle on the device named by ULTIMA_HSAMP_DEVICE (default
// 0), created on first use. sample() serialises on it, which matches the
// reference's callers (one generation loop per model mutex).
struct Backend {
    std::mutex mu;
    ultima_hsamp* h = nullptr;
    int status = ULTIMA_HSAMP_OK;
    bool writeback = true;    // sample() leaves logits as the reference does (in place)
    std::vector<float> scratch;
};

Backend& backend() {
    static Backend b;
    static std::once_flag once;
    std::call_once(once, [] {
        const char* dev = std::getenv("ULTIMA_HSAMP_DEVICE");
        b.status = ultima_hsamp_create(dev ? std::atoi(dev) : 0, kBatchRows, ULTIMA_HSAMP_MAX_VOCAB, &b.h);
    });
    return b;
}

// SamplerContext's seed when none is given (reference sampler.cpp:184-187).
std::uint64_t seed_from_device() {
    std::random_device rd;
    return (static_cast<std::uint64_t>(rd()) << 32) | rd();
}

ultima_hsamp_params to_abi(const SamplerParams& p, std::size_t hist_len, std::size_t n_bias) {
    ultima_hsamp_params q{};
    q.rep_penalty = p.rep_penalty;
    q.repeat_last_n = p.repeat_last_n;
    q.dry_multiplier = p.dry_multiplier;
    q.dry_base = p.dry_base;
    q.dry_allowed_len = p.dry_allowed_len;
    q.dry_last_n = p.dry_last_n;
    q.frequency_penalty = p.frequency_penalty;
    q.presence_penalty = p.presence_penalty;
    q.temperature = p.temperature;
    q.top_k = p.top_k;
    q.top_p = p.top_p;
    q.min_p = p.min_p;
    q.hist_len = static_cast<std::int64_t>(hist_len);
    q.bias_offset = 0;
    q.bias_count = static_cast<std::int64_t>(n_bias);
    return q;
}

}  // namespace

// Reference sampler.cpp:192-205.
SamplerParams SamplerParams::identity() {
    SamplerParams p;
    p.rep_penalty = 1.0f;
    p.repeat_last_n = 0;
    p.dry_multiplier = 0.0f;
    p.dry_last_n = 0;
    p.frequency_penalty = 0.0f;
    p.presence_penalty = 0.0f;
    p.temperature = 1.0f;
    p.top_k = 0;
    p.top_p = 1.0f;
    p.min_p = 0.0f;
    return p;
}

// Reference sampler.cpp:208-217.
SamplerContext::SamplerContext(std::uint64_t s) : seed_{s}, rng_{s} {}
SamplerContext::SamplerContext() : SamplerContext(seed_from_device()) {}
void SamplerContext::push_recent(TokenId t) { recent_.push_back(t); }
void SamplerContext::set_recent(std::span<const TokenId> tokens) {
    recent_.assign(tokens.begin(), tokens.end());
}

void set_inplace_writeback(bool on) noexcept {
    Backend& b = backend();
    std::lock_guard<std::mutex> lk(b.mu);
    b.writeback = on;
}

bool gpu_available() noexcept { return backend().status == ULTIMA_HSAMP_OK; }

// Reference sampler.cpp:230-277. The uniform is drawn from ctx.rng() exactly
// where std::discrete_distribution would draw it: only when the ladder reaches
// the draw (T > 0) and there are at least two logits.
TokenId sample(std::span<float> logits, const SamplerParams& params, SamplerContext& ctx) {
    if (logits.empty()) return -1;
    Backend& b = backend();
    if (b.status != ULTIMA_HSAMP_OK || logits.size() > ULTIMA_HSAMP_MAX_VOCAB) return -1;
    double u = 0.0;
    if (!(params.temperature <= 0.0f) && logits.size() >= 2)
        u = std::generate_canonical<double, 53>(ctx.rng());
    std::vector<std::int32_t> ids;
    std::vector<float> vals;
    ids.reserve(params.logit_bias.size());
    vals.reserve(params.logit_bias.size());
    for (const auto& [id, v] : params.logit_bias) {
        ids.push_back(id);
        vals.push_back(v);
    }
    const auto recent = ctx.recent();
    const ultima_hsamp_params q = to_abi(params, recent.size(), ids.size());
    std::lock_guard<std::mutex> lk(b.mu);
    std::int32_t tok = -1;
    const int st = ultima_hsamp_sample_host(b.h, logits.data(), static_cast<std::int32_t>(logits.size()),
                                            &q, recent.data(), ids.data(), vals.data(), u,
                                            b.writeback ? 1 : 0, &tok);
    return st == ULTIMA_HSAMP_OK ? tok : -1;
}

// Reference sampler.cpp:220-228: the greedy path of the ladder with every knob
// at identity is exactly the first-maximum argmax.
TokenId argmax(std::span<const float> logits) noexcept {
    if (logits.empty()) return -1;
    Backend& b = backend();
    if (b.status != ULTIMA_HSAMP_OK || logits.size() > ULTIMA_HSAMP_MAX_VOCAB) return -1;
    ultima_hsamp_params q;
    ultima_hsamp_params_identity(&q);
    q.temperature = 0.0f;
    std::lock_guard<std::mutex> lk(b.mu);
    b.scratch.assign(logits.begin(), logits.end());
    std::int32_t tok = -1;
    const int st = ultima_hsamp_sample_host(b.h, b.scratch.data(), static_cast<std::int32_t>(logits.size()),
                                            &q, nullptr, nullptr, nullptr, 0.0, 0, &tok);
    return st == ULTIMA_HSAMP_OK ? tok : -1;
}

int sample_batch(const float* logits_dev, std::int32_t rows, std::int32_t vocab, std::int64_t stride,
                 std::span<const SamplerParams> params, const TokenId* hist_dev,
                 std::int64_t hist_stride, std::span<const std::int64_t> hist_len,
                 const double* u_dev, TokenId* tokens_dev, void* hip_stream) {
    if (rows < 1 || params.size() != static_cast<std::size_t>(rows) ||
        hist_len.size() != static_cast<std::size_t>(rows))
        return ULTIMA_HSAMP_ERR_INVALID;
    Backend& b = backend();
    if (b.status != ULTIMA_HSAMP_OK) return b.status;
    std::vector<ultima_hsamp_params> q(static_cast<std::size_t>(rows));
    std::vector<std::int32_t> ids;
    std::vector<float> vals;
    for (std::int32_t r = 0; r < rows; ++r) {
        const SamplerParams& p = params[static_cast<std::size_t>(r)];
        q[static_cast<std::size_t>(r)] = to_abi(p, static_cast<std::size_t>(hist_len[static_cast<std::size_t>(r)]),
                                                p.logit_bias.size());
        q[static_cast<std::size_t>(r)].bias_offset = static_cast<std::int64_t>(ids.size());
        for (const auto& [id, v] : p.logit_bias) {
            ids.push_back(id);
            vals.push_back(v);
        }
    }
    ultima_hsamp_batch bt{};
    bt.rows = rows;
    bt.vocab = vocab;
    bt.dtype = ULTIMA_HSAMP_F32;
    bt.logits = const_cast<float*>(logits_dev);
    bt.logits_stride = stride;
    bt.hist = hist_dev;
    bt.hist_stride = hist_stride;
    bt.u = u_dev;
    bt.params = q.data();
    bt.bias_ids = ids.empty() ? nullptr : ids.data();
    bt.bias_vals = vals.empty() ? nullptr : vals.data();
    bt.token = tokens_dev;
    std::lock_guard<std::mutex> lk(b.mu);
    return ultima_hsamp_run(b.h, &bt, hip_stream);
}

}  // namespace ultima::sampler
