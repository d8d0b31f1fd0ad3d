// Test driver for the ultima::sampler drop-in (libultima_sampler.so).
//
//   dropin_driver refcases          the reference's own cases
//                                   (/root/reference/tests/unit/test_sampler.cpp:21-117),
//                                   compiled unchanged against the drop-in header;
//                                   exit status = number of failed checks
//   dropin_driver replay IN OUT     run sample() with in-place writeback on every
//                                   case of IN and write token + logits to OUT
//                                   (tests/test_gpu_dropin.py compares them with
//                                   the CPU oracle)
//   dropin_driver cli IN OUT        the reference CLI's generation loop
//                                   (apps/ultima-cli/main.cpp:661-679): identity()
//                                   + temperature, one SamplerContext pushing each
//                                   sampled id; writes token + logits per step
//   dropin_driver batch IN OUT      sample_batch() over device copies of a batch
//                                   (rows, per-row knobs, histories, uniforms)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ultima/sampler/sampler.hpp"

using ultima::sampler::argmax;
using ultima::sampler::sample;
using ultima::sampler::sample_batch;
using ultima::sampler::SamplerContext;
using ultima::sampler::SamplerParams;
using ultima::sampler::TokenId;

static int failures = 0;
#define CHECK(x)                                                        \
    do {                                                                \
        if (!(x)) {                                                     \
            std::fprintf(stderr, "CHECK failed line %d: %s\n", __LINE__, #x); \
            ++failures;                                                 \
        }                                                               \
    } while (0)

static int refcases() {
    {   // test_sampler.cpp:21-24
        std::vector<float> l{0.1f, 0.3f, 0.2f, 0.9f, 0.5f};
        CHECK(argmax(l) == 3);
    }
    {   // :26-32
        std::vector<float> l{1.0f, 5.0f, 2.0f, 3.0f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 0.0f;
        SamplerContext ctx(42);
        CHECK(sample(l, p, ctx) == 1);
    }
    {   // :34-42
        std::vector<float> l{1.0f, 2.0f, 3.0f, 4.0f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 1.0f;
        SamplerContext ctx(7);
        const TokenId t = sample(l, p, ctx);
        CHECK(t >= 0);
        CHECK(t < 4);
    }
    {   // :44-55
        SamplerParams p = SamplerParams::identity();
        p.temperature = 1.0f;
        std::vector<float> l1{0.5f, 0.7f, 0.3f, 0.9f, 0.6f, 0.4f, 0.8f, 0.2f};
        auto l2 = l1;
        SamplerContext c1(123456ull), c2(123456ull);
        CHECK(sample(l1, p, c1) == sample(l2, p, c2));
    }
    {   // :57-64
        std::vector<float> l{0.1f, 0.4f, 0.3f, 0.9f, 0.2f};
        SamplerParams p = SamplerParams::identity();
        p.top_k = 1;
        p.temperature = 1.0f;
        SamplerContext ctx(1);
        CHECK(sample(l, p, ctx) == 3);
    }
    {   // :66-78
        std::vector<float> l{0.1f, 2.0f, 2.5f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 0.0f;
        p.rep_penalty = 2.0f;
        p.repeat_last_n = 8;
        SamplerContext ctx(1);
        ctx.push_recent(2);
        CHECK(sample(l, p, ctx) == 1);
    }
    {   // :80-88
        std::vector<float> l{10.0f, -5.0f, -6.0f, -7.0f, -8.0f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 1.0f;
        p.min_p = 0.5f;
        SamplerContext ctx(42);
        CHECK(sample(l, p, ctx) == 0);
    }
    {   // :90-100 (only token 0 can survive: p0 = 0.731 >= 0.5)
        std::vector<float> l{10.0f, 9.0f, 0.0f, 0.0f, 0.0f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 1.0f;
        p.top_p = 0.5f;
        SamplerContext ctx(5);
        CHECK(sample(l, p, ctx) == 0);
    }
    {   // :102-109
        std::vector<float> l{0.1f, 0.2f, 0.3f};
        SamplerParams p = SamplerParams::identity();
        p.temperature = 0.0f;
        p.logit_bias[0] = 100.0f;
        SamplerContext ctx(1);
        CHECK(sample(l, p, ctx) == 0);
    }
    {   // :111-117
        std::vector<float> l{0.1f, 0.5f, 0.9f, 0.3f, 0.7f, 0.2f, 0.4f, 0.6f, 0.8f, 0.15f};
        SamplerParams p;
        SamplerContext ctx(99);
        const TokenId t = sample(l, p, ctx);
        CHECK(t >= 0);
        CHECK(t < 10);
    }
    CHECK(argmax(std::vector<float>{}) == -1);
    std::vector<float> empty;
    SamplerContext c0(3);
    CHECK(sample(empty, SamplerParams::identity(), c0) == -1);
    std::printf("refcases: %d failure(s)\n", failures);
    return failures;
}

// Case file: int32 count, then per case
//   int32 V, float logits[V], int32 H, int32 hist[H], int32 NB, (int32 id, float v)[NB],
//   float rep, u64 rep_n, float dry_mult, float dry_base, u64 dry_allowed, u64 dry_n,
//   float freq, float pres, float temp, u64 top_k, float top_p, float min_p, u64 seed
template <class T>
static bool rd(std::FILE* f, T& x) { return std::fread(&x, sizeof(T), 1, f) == 1; }

// The knob record both case formats share.
static bool read_params(std::FILE* f, SamplerParams& p, uint64_t& seed) {
    uint64_t rep_n, dry_allowed, dry_n, top_k;
    bool ok = rd(f, p.rep_penalty) && rd(f, rep_n) && rd(f, p.dry_multiplier) && rd(f, p.dry_base) &&
              rd(f, dry_allowed) && rd(f, dry_n) && rd(f, p.frequency_penalty) && rd(f, p.presence_penalty) &&
              rd(f, p.temperature) && rd(f, top_k) && rd(f, p.top_p) && rd(f, p.min_p) && rd(f, seed);
    p.repeat_last_n = rep_n;
    p.dry_allowed_len = dry_allowed;
    p.dry_last_n = dry_n;
    p.top_k = top_k;
    return ok;
}


static int replay(const char* in, const char* out) {
    std::FILE* f = std::fopen(in, "rb");
    std::FILE* g = std::fopen(out, "wb");
    if (!f || !g) return 100;
    int32_t n = 0;
    if (!rd(f, n)) return 101;
    for (int32_t c = 0; c < n; ++c) {
        int32_t V, H, NB;
        if (!rd(f, V)) return 102;
        std::vector<float> l(static_cast<size_t>(V));
        if (std::fread(l.data(), 4, l.size(), f) != l.size()) return 103;
        rd(f, H);
        std::vector<TokenId> h(static_cast<size_t>(H));
        if (H && std::fread(h.data(), 4, h.size(), f) != h.size()) return 104;
        rd(f, NB);
        SamplerParams p = SamplerParams::identity();
        for (int32_t j = 0; j < NB; ++j) {
            int32_t id;
            float v;
            rd(f, id);
            rd(f, v);
            p.logit_bias[id] = v;
        }
        uint64_t seed;
        if (!read_params(f, p, seed)) return 105;
        SamplerContext ctx(seed);
        ctx.set_recent(h);
        const TokenId t = sample(l, p, ctx);
        std::fwrite(&t, 4, 1, g);
        std::fwrite(l.data(), 4, l.size(), g);
    }
    std::fclose(f);
    std::fclose(g);
    return 0;
}

// CLI file: int32 V, int32 steps, float temperature, u64 seed, int32 P, int32 prompt[P],
// then steps x float logits[V]. Out: per step int32 token, float logits[V] after sample().
static int cli(const char* in, const char* out) {
    std::FILE* f = std::fopen(in, "rb");
    std::FILE* g = std::fopen(out, "wb");
    if (!f || !g) return 100;
    int32_t V, steps, P;
    float temperature;
    uint64_t seed;
    if (!rd(f, V) || !rd(f, steps) || !rd(f, temperature) || !rd(f, seed) || !rd(f, P)) return 101;
    std::vector<TokenId> prompt(static_cast<size_t>(P));
    if (P && std::fread(prompt.data(), 4, prompt.size(), f) != prompt.size()) return 102;
    // apps/ultima-cli/main.cpp:661-664
    SamplerParams sp = SamplerParams::identity();
    sp.temperature = temperature;
    SamplerContext sctx{seed};
    for (auto t : prompt) sctx.push_recent(t);
    std::vector<float> logits(static_cast<size_t>(V));
    for (int32_t i = 0; i < steps; ++i) {
        if (std::fread(logits.data(), 4, logits.size(), f) != logits.size()) return 103;
        // main.cpp:669-672
        const TokenId next = (temperature <= 0.0f) ? argmax(logits) : sample(logits, sp, sctx);
        sctx.push_recent(next);
        std::fwrite(&next, 4, 1, g);
        std::fwrite(logits.data(), 4, logits.size(), g);
    }
    std::fclose(f);
    std::fclose(g);
    return 0;
}

// Batch file: int32 B, int32 V, int32 H, float logits[B][V], int32 hist[B][H],
// int64 hist_len[B], double u[B], then B knob records. Out: int32 token[B].
static int batch(const char* in, const char* out) {
    std::FILE* f = std::fopen(in, "rb");
    std::FILE* g = std::fopen(out, "wb");
    if (!f || !g) return 100;
    int32_t B, V, H;
    if (!rd(f, B) || !rd(f, V) || !rd(f, H)) return 101;
    const size_t nl = static_cast<size_t>(B) * static_cast<size_t>(V), nh = static_cast<size_t>(B) * static_cast<size_t>(H);
    std::vector<float> logits(nl);
    std::vector<TokenId> hist(nh);
    std::vector<int64_t> hist_len(static_cast<size_t>(B));
    std::vector<double> u(static_cast<size_t>(B));
    if (std::fread(logits.data(), 4, nl, f) != nl || std::fread(hist.data(), 4, nh, f) != nh ||
        std::fread(hist_len.data(), 8, hist_len.size(), f) != hist_len.size() ||
        std::fread(u.data(), 8, u.size(), f) != u.size())
        return 102;
    std::vector<SamplerParams> params(static_cast<size_t>(B));
    for (auto& p : params) {
        uint64_t seed;
        p = SamplerParams::identity();
        if (!read_params(f, p, seed)) return 103;
    }
    float* d_logits = nullptr;
    TokenId* d_hist = nullptr;
    double* d_u = nullptr;
    TokenId* d_tok = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d_logits), nl * 4) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&d_hist), std::max<size_t>(nh, 1) * 4) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&d_u), u.size() * 8) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&d_tok), static_cast<size_t>(B) * 4) != hipSuccess)
        return 104;
    if (hipMemcpy(d_logits, logits.data(), nl * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (nh && hipMemcpy(d_hist, hist.data(), nh * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(d_u, u.data(), u.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
        return 105;
    const int st = sample_batch(d_logits, B, V, V, params, d_hist, H, hist_len, d_u, d_tok, nullptr);
    if (st != 0) {
        std::fprintf(stderr, "sample_batch: status %d\n", st);
        return 106;
    }
    std::vector<TokenId> tok(static_cast<size_t>(B));
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(tok.data(), d_tok, tok.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return 107;
    std::fwrite(tok.data(), 4, tok.size(), g);
    (void)hipFree(d_logits);
    (void)hipFree(d_hist);
    (void)hipFree(d_u);
    (void)hipFree(d_tok);
    std::fclose(f);
    std::fclose(g);
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "refcases") == 0) return refcases();
    if (argc >= 4 && std::strcmp(argv[1], "replay") == 0) return replay(argv[2], argv[3]);
    if (argc >= 4 && std::strcmp(argv[1], "cli") == 0) return cli(argv[2], argv[3]);
    if (argc >= 4 && std::strcmp(argv[1], "batch") == 0) return batch(argv[2], argv[3]);
    std::fprintf(stderr, "usage: %s refcases | replay IN OUT | cli IN OUT | batch IN OUT\n", argv[0]);
    return 2;
}
