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
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ultima/sampler/sampler.hpp"

using ultima::sampler::argmax;
using ultima::sampler::sample;
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

static int replay(const char* in, const char* out) {
    std::FILE* f = std::fopen(in, "rb");
    std::FILE* g = std::fopen(out, "wb");
    if (!f || !g) return 100;
    ultima::sampler::set_inplace_writeback(true);
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
        uint64_t rep_n, dry_allowed, dry_n, top_k, seed;
        rd(f, p.rep_penalty); rd(f, rep_n); rd(f, p.dry_multiplier); rd(f, p.dry_base);
        rd(f, dry_allowed); rd(f, dry_n); rd(f, p.frequency_penalty); rd(f, p.presence_penalty);
        rd(f, p.temperature); rd(f, top_k); rd(f, p.top_p); rd(f, p.min_p); rd(f, seed);
        p.repeat_last_n = rep_n;
        p.dry_allowed_len = dry_allowed;
        p.dry_last_n = dry_n;
        p.top_k = top_k;
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

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "refcases") == 0) return refcases();
    if (argc >= 4 && std::strcmp(argv[1], "replay") == 0) return replay(argv[2], argv[3]);
    std::fprintf(stderr, "usage: %s refcases | replay IN OUT\n", argv[0]);
    return 2;
}
