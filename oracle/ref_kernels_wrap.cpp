// C ABI over the reference's own rmsnorm, matvec and Hadamard kernels
// (src/kernels/rmsnorm.cpp, matvec_*.cpp, dequant_*.cpp, hadamard.cpp, compiled
// where they lie by oracle/Makefile into oracle/_ref/libref_kernels.so). Test
// infrastructure only: it pins oracle/head_oracle.c.
#include <cstddef>
#include <cstdint>

#include "ultima/kernels/hadamard.hpp"
#include "ultima/kernels/matvec.hpp"
#include "ultima/kernels/norms.hpp"

namespace k = ultima::kernels;

extern "C" {
void ref_rmsnorm(const float* x, const float* scale, float* y, int64_t n, float eps) {
    k::rmsnorm_f32(x, scale, y, (std::size_t)n, eps);
}
void ref_matvec_f32(const float* w, const float* x, float* y, int64_t M, int64_t K) {
    k::matvec_f32_f32(w, x, y, (std::size_t)M, (std::size_t)K);
}
void ref_matvec_bf16(const uint16_t* w, const float* x, float* y, int64_t M, int64_t K) {
    k::matvec_bf16_f32(reinterpret_cast<const std::uint8_t*>(w), x, y, (std::size_t)M, (std::size_t)K);
}
// The quantised heads by the weight type numbers of head_oracle.c's
// orc_matvec (2 Q4_K, 3 Q5_K, 4 Q6_K, 5 Q8_0, 6 Q4_1, 7 Q5_0, 8 PQ2_0): the
// per-range kernels matvec_dispatch_threaded's workers run
// (src/kernels/matvec_threaded.cpp:36-136).
void ref_matvec_q(int dtype, const uint8_t* w, const float* x, float* y, int64_t M, int64_t K) {
    const std::size_t m = (std::size_t)M, kk = (std::size_t)K;
    switch (dtype) {
        case 2: k::matvec_q4k_f32(w, x, y, m, kk); break;
        case 3: k::matvec_q5k_f32(w, x, y, m, kk); break;
        case 4: k::matvec_q6k_f32(w, x, y, m, kk); break;
        case 5: k::matvec_q8_0_f32(w, x, y, m, kk); break;
        case 6: k::matvec_q4_1_f32(w, x, y, m, kk); break;
        case 7: k::matvec_q5_0_f32(w, x, y, m, kk); break;
        case 8: k::matvec_pq2_0_f32(w, x, y, m, kk); break;
        default: break;
    }
}
void ref_hadamard_fold(const float* x, float* y, int64_t width, int64_t block, const float* signs) {
    k::hadamard_fold_f32(x, y, (std::size_t)width, (std::size_t)block, signs);
}
}
