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
 * The quantised heads (weight_dispatch.cpp:106-146: Q8_0, Q6_K, Q4_K, Q5_K,
 * Q4_1, Q5_0, PQ2_0) follow their kernels' own partial-sum layouts, restated
 * per format below; where those kernels leave scalar C++ (the dequantisation
 * into a scratch row of Q5_K and Q4_1, PQ2_0's per-block fold), GCC contracts
 * a * b + c into one fused multiply-add under the reference's flags, and so
 * does this restatement. The Hadamard fold (hadamard.cpp:26-44) has no
 * multiply-add to fuse.
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

/* ---- quantised heads ----------------------------------------------------- */

/* IEEE half -> float, exact (subnormals normalised, Inf/NaN kept with their
 * payload), as the kernels' fp16_to_float (e.g. matvec_q8_0_f32.cpp:13-36). */
static float fp16_to_f32(const uint8_t* p) {
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            unsigned shift = 0;
            while ((mant & 0x400u) == 0) { mant <<= 1; ++shift; }
            bits = sign | ((127u - 14u - shift) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* (a0 + a1) + (a2 + a3) per lane, then the horizontal sum: the reduction of
 * four eight-lane accumulators (matvec_q5k_f32.cpp:78-79 and the Q4_1 / Q5_0
 * kernels). */
static float hsum4x8(float a[4][8]) {
    float t[8];
    for (int l = 0; l < 8; ++l) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    return hsum8(t);
}

/* ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)) per lane, then the
 * horizontal sum: eight accumulators (matvec_q6k_f32.cpp:164-166,
 * matvec_q4k_f32.cpp:155-157). */
static float hsum8x8(float a[8][8]) {
    float t[8];
    for (int l = 0; l < 8; ++l)
        t[l] = ((a[0][l] + a[1][l]) + (a[2][l] + a[3][l])) + ((a[4][l] + a[5][l]) + (a[6][l] + a[7][l]));
    return hsum8(t);
}

static int zero_rows(float* y, int64_t M, int64_t K, int64_t blk) {
    if (K == 0 || K % blk != 0) {
        for (int64_t m = 0; m < M; ++m) y[m] = 0.0f;
        return 1;
    }
    return 0;
}

/* src/kernels/matvec_q8_0_f32.cpp:83-117 (matvec_q8_0_f32_avx2). Block: fp16 d,
 * 32 int8. Lane l of the block accumulator takes elements c * 8 + l (c = 0..3)
 * from zero; then row lane l += d * block lane l (fused); horizontal sum. */
void orc_matvec_q8_0(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 32)) return;
    const int64_t nb = K / 32, rb = nb * 34;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float racc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 34;
            const float d = fp16_to_f32(blk);
            const int8_t* qs = (const int8_t*)(blk + 2);
            const float* xs = x + b * 32;
            float bacc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int c = 0; c < 4; ++c)
                for (int l = 0; l < 8; ++l) bacc[l] = fmaf((float)qs[c * 8 + l], xs[c * 8 + l], bacc[l]);
            for (int l = 0; l < 8; ++l) racc[l] = fmaf(d, bacc[l], racc[l]);
        }
        y[m] = hsum8(racc);
    }
}

/* src/kernels/matvec_q6k_f32.cpp:99-169 (matvec_q6k_f32_avx2). Super-block of
 * 256: ql[128], qh[64], int8 scales[16], fp16 d. Each half (128 values) forms
 * four runs of 32 six-bit values q - 32 (q1: low nibbles of ql[0..31] with qh
 * bits 0-1, q2: low nibbles of ql[32..63] with bits 2-3, q3: high nibbles of
 * ql[0..31] with bits 4-5, q4: high nibbles of ql[32..63] with bits 6-7);
 * run r's value l is scaled by fl(d * scale[2r + l / 16]) (rounded on its
 * own) and fused into accumulator (r % 2) * 4 + l / 8, lane l % 8, in the
 * order q1, q2, q3, q4. */
void orc_matvec_q6k(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 256)) return;
    const int64_t nb = K / 256, rb = nb * 210;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float a[8][8];
        memset(a, 0, sizeof a);
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 210;
            const float d = fp16_to_f32(blk + 208);
            for (int half = 0; half < 2; ++half) {
                const uint8_t* ql = blk + half * 64;
                const uint8_t* qh = blk + 128 + half * 32;
                const int8_t* sc = (const int8_t*)(blk + 192 + half * 8);
                const float* xh = x + b * 256 + half * 128;
                float s[8];
                for (int i = 0; i < 8; ++i) s[i] = d * (float)sc[i];
                for (int r = 0; r < 4; ++r) {
                    for (int l = 0; l < 32; ++l) {
                        const unsigned lo = (r & 1) ? ql[32 + l] : ql[l];
                        const unsigned nib = (r < 2) ? (lo & 0x0Fu) : (lo >> 4);
                        const int q = (int)(nib | (((qh[l] >> (2 * r)) & 3u) << 4)) - 32;
                        const float v = (float)q * s[2 * r + l / 16];
                        float* acc = &a[(r & 1) * 4 + l / 8][l % 8];
                        *acc = fmaf(v, xh[32 * r + l], *acc);
                    }
                }
            }
        }
        y[m] = hsum8x8(a);
    }
}

/* Q4_K / Q5_K six-bit scale and min j of the 12-byte table
 * (matvec_q4k_f32.cpp:45-55, dequant_q5k.cpp:42-52). */
static void scale_min_k4(const uint8_t* sm, int j, unsigned* sc, unsigned* mn) {
    if (j < 4) {
        *sc = sm[j] & 0x3Fu;
        *mn = sm[j + 4] & 0x3Fu;
    } else {
        *sc = (sm[j + 4] & 0x0Fu) | ((sm[j - 4] >> 6) << 4);
        *mn = (sm[j + 4] >> 4) | ((sm[j] >> 6) << 4);
    }
}

/* src/kernels/matvec_q4k_f32.cpp:108-160 (matvec_q4k_f32_avx2). Super-block of
 * 256: fp16 d, fp16 dmin, 12 bytes of scales/mins, qs[128]. Pair j (j = 0..3)
 * shares qs[32j .. 32j+31]: low nibbles are values 64j + l with
 * (d1, m1) = (fl(d * sc(2j)), fl(dmin * mn(2j))), high nibbles values
 * 64j + 32 + l with pair 2j + 1; each value fl(nib * d1 - m1) (fused) is fused
 * into accumulator l / 8 (low) or 4 + l / 8 (high), lane l % 8. */
void orc_matvec_q4k(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 256)) return;
    const int64_t nb = K / 256, rb = nb * 144;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float a[8][8];
        memset(a, 0, sizeof a);
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 144;
            const float d = fp16_to_f32(blk), dmin = fp16_to_f32(blk + 2);
            const uint8_t* sm = blk + 4;
            const uint8_t* qs = blk + 16;
            const float* xb = x + b * 256;
            for (int j = 0; j < 4; ++j) {
                unsigned sc0, mn0, sc1, mn1;
                scale_min_k4(sm, 2 * j, &sc0, &mn0);
                scale_min_k4(sm, 2 * j + 1, &sc1, &mn1);
                const float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
                const float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
                for (int l = 0; l < 32; ++l) {
                    const float v = fmaf((float)(qs[32 * j + l] & 0x0Fu), d1, -m1);
                    a[l / 8][l % 8] = fmaf(v, xb[64 * j + l], a[l / 8][l % 8]);
                }
                for (int l = 0; l < 32; ++l) {
                    const float v = fmaf((float)(qs[32 * j + l] >> 4), d2, -m2);
                    a[4 + l / 8][l % 8] = fmaf(v, xb[64 * j + 32 + l], a[4 + l / 8][l % 8]);
                }
            }
        }
        y[m] = hsum8x8(a);
    }
}

/* src/kernels/matvec_q5k_f32.cpp:48-80 (matvec_q5k_f32_avx2) over
 * dequant_q5k_block (dequant_q5k.cpp:57-93): super-block of 256, fp16 d, fp16
 * dmin, 12 bytes of scales/mins, qh[32], ql[128]; value 64j + l (low nibble of
 * ql[32j + l], fifth bit qh[l] bit 2j) and 64j + 32 + l (high nibble, bit
 * 2j + 1) dequantised as fl(d1 * q - m1) (GCC fuses it); value e of the
 * super-block fused into accumulator (e % 32) / 8, lane e % 8. */
void orc_matvec_q5k(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 256)) return;
    const int64_t nb = K / 256, rb = nb * 176;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float a[4][8];
        memset(a, 0, sizeof a);
        float scr[256];
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 176;
            const float d = fp16_to_f32(blk), dmin = fp16_to_f32(blk + 2);
            const uint8_t* sm = blk + 4;
            const uint8_t* qh = blk + 16;
            const uint8_t* ql = blk + 48;
            for (int j = 0; j < 4; ++j) {
                unsigned sc0, mn0, sc1, mn1;
                scale_min_k4(sm, 2 * j, &sc0, &mn0);
                scale_min_k4(sm, 2 * j + 1, &sc1, &mn1);
                const float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
                const float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
                for (int l = 0; l < 32; ++l) {
                    const unsigned lo = (ql[32 * j + l] & 0x0Fu) | ((qh[l] >> (2 * j)) & 1u) << 4;
                    const unsigned hi = (ql[32 * j + l] >> 4) | ((qh[l] >> (2 * j + 1)) & 1u) << 4;
                    scr[64 * j + l] = fmaf(d1, (float)lo, -m1);
                    scr[64 * j + 32 + l] = fmaf(d2, (float)hi, -m2);
                }
            }
            const float* xs = x + b * 256;
            for (int i = 0; i < 256; ++i) a[(i % 32) / 8][i % 8] = fmaf(scr[i], xs[i], a[(i % 32) / 8][i % 8]);
        }
        y[m] = hsum4x8(a);
    }
}

/* src/kernels/matvec_q4_1_f32.cpp:47-75 (matvec_q4_1_f32_avx2) over
 * dequant_q4_1_block (dequant_q4_1.cpp:46-54): block of 32, fp16 d, fp16 m,
 * qs[16]; value j = fl(nib(qs[j]) * d + m) (GCC fuses it), value j + 16 the
 * high nibble; value i fused into accumulator i / 8, lane i % 8. */
void orc_matvec_q4_1(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 32)) return;
    const int64_t nb = K / 32, rb = nb * 20;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float a[4][8];
        memset(a, 0, sizeof a);
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 20;
            const float d = fp16_to_f32(blk), mn = fp16_to_f32(blk + 2);
            const uint8_t* qs = blk + 4;
            float v[32];
            for (int j = 0; j < 16; ++j) {
                v[j] = fmaf((float)(qs[j] & 0x0Fu), d, mn);
                v[j + 16] = fmaf((float)(qs[j] >> 4), d, mn);
            }
            const float* xs = x + b * 32;
            for (int i = 0; i < 32; ++i) a[i / 8][i % 8] = fmaf(v[i], xs[i], a[i / 8][i % 8]);
        }
        y[m] = hsum4x8(a);
    }
}

/* src/kernels/matvec_q5_0_f32.cpp:108-150 (matvec_q5_0_f32_avx2): block of 32,
 * fp16 d, 32 fifth bits (qh, little-endian), qs[16]; value i (low nibble of
 * qs[i] for i < 16, high nibble of qs[i - 16] after) with bit i of qh is the
 * signed q = (nib | bit << 4) - 16, scaled fl(q * d) on its own and fused into
 * accumulator i / 8, lane i % 8. */
void orc_matvec_q5_0(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 32)) return;
    const int64_t nb = K / 32, rb = nb * 22;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float a[4][8];
        memset(a, 0, sizeof a);
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 22;
            const float d = fp16_to_f32(blk);
            const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                                ((uint32_t)blk[5] << 24);
            const uint8_t* qs = blk + 6;
            const float* xs = x + b * 32;
            for (int i = 0; i < 32; ++i) {
                const unsigned nib = i < 16 ? (qs[i] & 0x0Fu) : (qs[i - 16] >> 4);
                const int q = (int)(nib | ((qh >> i) & 1u) << 4) - 16;
                const float v = (float)q * d;
                a[i / 8][i % 8] = fmaf(v, xs[i], a[i / 8][i % 8]);
            }
        }
        y[m] = hsum4x8(a);
    }
}

/* src/kernels/matvec_pq2_0_f32.cpp:111-184, the vectorised path
 * matvec_pq2_0_f32 takes for calls of at least 8 rows (every thread's share
 * of a vocabulary head): block of 128, fp16 d, 32 bytes of four 2-bit codes
 * (low pair first). The activation's block sums are plain sequential float
 * sums; per block, lane l of one accumulator takes, for code position
 * j = 0..3 and byte group g = 0..3, byte i = 8g + l's code j times
 * x[128b + 4i + j] (fused, from zero); the row sum += d * (horizontal sum -
 * block sum) (GCC fuses it). */
void orc_matvec_pq2_0(const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    if (zero_rows(y, M, K, 128)) return;
    const int64_t nb = K / 128, rb = nb * 34;
    for (int64_t m = 0; m < M; ++m) {
        const uint8_t* row = w + m * rb;
        float acc = 0.0f;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * 34;
            const float d = fp16_to_f32(blk);
            const uint8_t* codes = blk + 2;
            const float* xs = x + b * 128;
            float bsum = 0.0f;
            for (int i = 0; i < 128; ++i) bsum += xs[i];
            float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < 4; ++j)
                for (int g = 0; g < 4; ++g)
                    for (int l = 0; l < 8; ++l) {
                        const int i = 8 * g + l;
                        a[l] = fmaf((float)((codes[i] >> (2 * j)) & 3u), xs[4 * i + j], a[l]);
                    }
            acc = fmaf(d, hsum8(a) - bsum, acc);
        }
        y[m] = acc;
    }
}

/* src/kernels/hadamard.cpp:9-44 (hadamard_fold_f32): y = x * signs (or x),
 * then each `block` of y through the unnormalised fast Walsh-Hadamard
 * butterflies (len 1, 2, 4, ...: a + b, a - b) and * fl(1 / sqrt(block)).
 * A block of 0 or one that does not divide the width leaves x as it is
 * (signs not applied). */
void orc_hadamard_fold(const float* x, float* y, int64_t width, int64_t block, const float* signs) {
    if (block == 0 || width % block != 0) {
        if (y != x) memmove(y, x, (size_t)width * sizeof(float));
        return;
    }
    for (int64_t i = 0; i < width; ++i) y[i] = signs ? x[i] * signs[i] : x[i];
    if (block < 2) return;
    for (int64_t off = 0; off < width; off += block) {
        float* v = y + off;
        for (int64_t len = 1; len < block; len <<= 1)
            for (int64_t i = 0; i < block; i += 2 * len)
                for (int64_t j = i; j < i + len; ++j) {
                    const float a = v[j], b = v[j + len];
                    v[j] = a + b;
                    v[j + len] = a - b;
                }
        const float inv = 1.0f / sqrtf((float)block);
        for (int64_t i = 0; i < block; ++i) v[i] *= inv;
    }
}

/* Bytes of one head row of H values for a weight type (0 when H does not
 * split into the type's blocks). Types: 0 f32, 1 bf16, 2 Q4_K, 3 Q5_K,
 * 4 Q6_K, 5 Q8_0, 6 Q4_1, 7 Q5_0, 8 PQ2_0. */
int64_t orc_head_row_bytes(int dtype, int64_t H) {
    static const int64_t be[9] = {1, 1, 256, 256, 256, 32, 32, 32, 128};
    static const int64_t bb[9] = {4, 2, 144, 176, 210, 34, 20, 22, 34};
    if (dtype < 0 || dtype > 8 || H % be[dtype] != 0) return 0;
    return H / be[dtype] * bb[dtype];
}

void orc_matvec(const void* w, int dtype, const float* x, float* y, int64_t M, int64_t K) {
    switch (dtype) {
        case 0: orc_matvec_f32((const float*)w, x, y, M, K); break;
        case 1: orc_matvec_bf16((const uint16_t*)w, x, y, M, K); break;
        case 2: orc_matvec_q4k((const uint8_t*)w, x, y, M, K); break;
        case 3: orc_matvec_q5k((const uint8_t*)w, x, y, M, K); break;
        case 4: orc_matvec_q6k((const uint8_t*)w, x, y, M, K); break;
        case 5: orc_matvec_q8_0((const uint8_t*)w, x, y, M, K); break;
        case 6: orc_matvec_q4_1((const uint8_t*)w, x, y, M, K); break;
        case 7: orc_matvec_q5_0((const uint8_t*)w, x, y, M, K); break;
        case 8: orc_matvec_pq2_0((const uint8_t*)w, x, y, M, K); break;
        default: for (int64_t m = 0; m < M; ++m) y[m] = 0.0f;
    }
}

/* src/model/qwen_model.cpp:182-207 for `rows` hidden states: rmsnorm with the
 * output norm, the Hadamard fold when the head is folded (fold_block > 0;
 * fold_signs may be NULL), the head matvec of weight type `dtype` (as
 * orc_matvec), then the logit scale (1 / logit_scale, when it is neither 1
 * nor 0). normed: [rows * H] scratch, left holding the head's input (the
 * normed rows, folded when the head is). */
void orc_lm_head(const float* hidden, int64_t rows, int64_t H, const float* norm_scale, float eps,
                 const void* weight, int dtype, int64_t V, float logit_scale, float* logits, float* normed,
                 int64_t fold_block, const float* fold_signs) {
    for (int64_t r = 0; r < rows; ++r) {
        float* xn = normed + r * H;
        orc_rmsnorm(hidden + r * H, norm_scale, xn, H, eps);
        if (fold_block > 0) orc_hadamard_fold(xn, xn, H, fold_block, fold_signs);
        float* y = logits + r * V;
        orc_matvec(weight, dtype, xn, y, V, H);
        if (logit_scale != 1.0f && logit_scale != 0.0f) {
            const float inv = 1.0f / logit_scale;
            for (int64_t i = 0; i < V; ++i) y[i] *= inv;
        }
    }
}
