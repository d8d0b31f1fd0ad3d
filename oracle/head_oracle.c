/* CPU restatement of the reference's logits producer: the final rmsnorm and
 * the lm-head matvec of one token's hidden state (reference
 * src/model/qwen_model.cpp:182-207). TEST INFRASTRUCTURE ONLY: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it as the
 * checker; the product never links it.
 *
 * The reference computes these with its AVX2 + FMA kernels (the kernels
 * target is built with -mavx2 -mfma, src/kernels/CMakeLists.txt:42-47), so
 * their results follow that evaluation order, restated here in plain C:
 *   - eight partial sums, partial l taking elements l, l + 8, ... with a
 *     fused multiply-add each;
 *   - the horizontal sum of the eight: s_i = p_i + p_{i+4}, then
 *     (s_0 + s_1) + (s_2 + s_3);
 *   - the scalar tail (t = n % 8 elements) as GCC compiles it for the
 *     reference's flags (GCC 11, -O3 -mavx2 -mfma; C++ contracts by
 *     default): fused multiply-adds, except that in the f32 loops (rmsnorm,
 *     f32 matvec), which GCC vectorises, the first four products are rounded
 *     on their own and added in order when t >= 4. Every real model
 *     dimension is a multiple of 8, where the tail is empty.
 * Build with -ffp-contract=off: every fused operation here is an explicit
 * fmaf and nothing else may be fused.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* _mm256_add/hadd order of src/kernels/rmsnorm.cpp:30-36 and
 * matvec_f32_f32.cpp:37-42 / matvec_bf16_f32.cpp:39-46 */
static float hsum8(const float p[8]) {
    const float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
    return (s0 + s1) + (s2 + s3);
}

/* acc + a[0] b[0] + ... + a[t-1] b[t-1], t < 8, as the vectorised f32 tail. */
static float tail_acc(float acc, const float* a, const float* b, int t) {
    int i = 0;
    if (t >= 4)
        for (; i < 4; ++i) acc = acc + a[i] * b[i];
    for (; i < t; ++i) acc = fmaf(a[i], b[i], acc);
    return acc;
}

/* src/kernels/rmsnorm.cpp:21-52 (rmsnorm_f32_avx2, which rmsnorm_f32 calls):
 * sum of squares, mean, 1 / sqrt(mean + eps), y = (x * scale) * inv. */
void orc_rmsnorm(const float* x, const float* scale, float* y, int64_t n, float eps) {
    const int64_t n8 = n / 8 * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = 0; i < n8; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    const float ss = tail_acc(hsum8(acc), x + n8, x + n8, (int)(n - n8));
    const float mean_sq = ss / (float)n;
    const float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = (x[i] * scale[i]) * inv_rms;
}

/* src/kernels/matvec_f32_f32.cpp:22-50 (matvec_f32_f32_avx2): the tail adds
 * onto the horizontal sum. */
void orc_matvec_f32(const float* w, const float* x, float* y, int64_t M, int64_t K) {
    const int64_t k8 = K / 8 * 8;
    for (int64_t m = 0; m < M; ++m) {
        const float* row = w + m * K;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t k = 0; k < k8; k += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(row[k + l], x[k + l], acc[l]);
        y[m] = tail_acc(hsum8(acc), row + k8, x + k8, (int)(K - k8));
    }
}

/* src/kernels/matvec_bf16_f32.cpp:48-68 (matvec_bf16_f32_avx2): bf16 widened
 * exactly; the tail is summed on its own and added last. */
void orc_matvec_bf16(const uint16_t* w, const float* x, float* y, int64_t M, int64_t K) {
    const int64_t k8 = K / 8 * 8;
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* row = w + m * K;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t k = 0; k < k8; k += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(bf16_to_f32(row[k + l]), x[k + l], acc[l]);
        float tail = 0.0f;   /* (not vectorised: every product fused) */
        for (int64_t k = k8; k < K; ++k) tail = fmaf(bf16_to_f32(row[k]), x[k], tail);
        y[m] = hsum8(acc) + tail;
    }
}

/* src/model/qwen_model.cpp:182-207 for `rows` hidden states: rmsnorm with the
 * output norm, the head matvec (dtype 0 f32, 1 bf16), then the logit scale
 * (1 / logit_scale, when it is neither 1 nor 0). normed: [rows * H] scratch. */
void orc_lm_head(const float* hidden, int64_t rows, int64_t H, const float* norm_scale, float eps,
                 const void* weight, int dtype, int64_t V, float logit_scale, float* logits, float* normed) {
    for (int64_t r = 0; r < rows; ++r) {
        float* xn = normed + r * H;
        orc_rmsnorm(hidden + r * H, norm_scale, xn, H, eps);
        float* y = logits + r * V;
        if (dtype == 0)
            orc_matvec_f32((const float*)weight, xn, y, V, H);
        else
            orc_matvec_bf16((const uint16_t*)weight, xn, y, V, H);
        if (logit_scale != 1.0f && logit_scale != 0.0f) {
            const float inv = 1.0f / logit_scale;
            for (int64_t i = 0; i < V; ++i) y[i] *= inv;
        }
    }
}
