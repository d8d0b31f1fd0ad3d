#pragma once
// ultima::sampler -- drop-in replacement for the reference's sampler interface
// (/root/reference/include/ultima/sampler/sampler.hpp:1-90). The declarations
// in the first part of this header keep the reference's names, member order,
// defaults and signatures exactly, so existing callers
// (src/server/http_server.cpp:159-183, apps/ultima-cli/main.cpp:661-679,
// tests/unit/test_sampler.cpp) compile unchanged. Every sampling decision is
// made by the HIP kernels of libultima_hsamp (include/ultima_hsamp.h).

#include <cstdint>
#include <optional>
#include <random>
#include <span>
#include <unordered_map>
#include <vector>

namespace ultima::sampler {

using TokenId = std::int32_t;

// Knobs of one request, applied in member order (reference sampler.hpp:16-52).
struct SamplerParams {
    std::unordered_map<TokenId, float> logit_bias;

    float       rep_penalty      = 1.1f;
    std::size_t repeat_last_n    = 64;

    float       dry_multiplier   = 0.8f;
    float       dry_base         = 1.75f;
    std::size_t dry_allowed_len  = 2;
    std::size_t dry_last_n       = 512;

    float       frequency_penalty = 0.0f;
    float       presence_penalty  = 0.0f;

    float       temperature      = 0.2f;

    std::size_t top_k            = 40;

    float       top_p            = 0.95f;

    float       min_p            = 0.05f;

    std::optional<std::uint64_t> seed;

    // Every knob at its no-op value: the ladder reduces to a plain draw at T = 1.
    static SamplerParams identity();
};

// Per-request state: the RNG that supplies the draw's uniform and the recent
// ids the penalties read (reference sampler.hpp:57-78).
class SamplerContext {
public:
    explicit SamplerContext(std::uint64_t seed);
    SamplerContext();   // seeded from std::random_device

    void push_recent(TokenId t);

    std::span<const TokenId> recent() const noexcept { return recent_; }
    void set_recent(std::span<const TokenId> tokens);

    std::uint64_t   seed() const noexcept { return seed_; }
    std::mt19937_64& rng() noexcept       { return rng_; }

private:
    std::uint64_t         seed_;
    std::mt19937_64       rng_;
    std::vector<TokenId>  recent_;
};

// Apply the transform ladder to `logits` and return the sampled id; -1 when
// `logits` is empty or the GPU backend fails (reference sampler.hpp:83-85).
// Draws the uniform from ctx.rng() exactly when the reference does (T > 0 and
// at least two logits). Like the reference, `logits` is transformed in place:
// it ends in the state the reference's sample() leaves it in (penalised and
// scaled, ids outside the kept set at -inf). set_inplace_writeback(false)
// leaves it unchanged instead, for callers that never read it afterwards.
TokenId sample(std::span<float> logits,
               const SamplerParams& params,
               SamplerContext&      ctx);

// First index of the maximum logit; -1 when empty (reference sampler.hpp:88).
TokenId argmax(std::span<const float> logits) noexcept;

// ---- Additions of this build (no reference counterpart) --------------------

// Whether sample() copies the transformed logits back into the caller's
// buffer. On by default, as the reference's sample() works in place; no
// reference caller reads them after the call, and turning it off saves a
// device-to-host copy of the row and a write-back kernel per call.
void set_inplace_writeback(bool on) noexcept;

// True when a gfx950 device and libultima_hsamp are usable.
bool gpu_available() noexcept;

// Device-resident batch on the sampler's device: `rows` rows of `vocab` fp32
// logits (row stride `stride` elements), one SamplerParams per row, row r's
// history in hist_dev[r * hist_stride ..] (hist_len[r] ids, oldest first),
// one uniform per row in u_dev. Token ids land in tokens_dev. Asynchronous on
// `hip_stream` (a hipStream_t); the device buffers must stay valid until the
// work completes. Returns 0 or a negative ultima_hsamp status.
int sample_batch(const float* logits_dev, std::int32_t rows, std::int32_t vocab,
                 std::int64_t stride, std::span<const SamplerParams> params,
                 const TokenId* hist_dev, std::int64_t hist_stride,
                 std::span<const std::int64_t> hist_len, const double* u_dev,
                 TokenId* tokens_dev, void* hip_stream);

} // namespace ultima::sampler
