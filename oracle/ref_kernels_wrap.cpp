// C ABI over the reference's own rmsnorm and matvec kernels (src/kernels/
// rmsnorm.cpp, matvec_f32_f32.cpp, matvec_bf16_f32.cpp, compiled where they
// lie by oracle/Makefile into oracle/_ref/libref_kernels.so). Test
// infrastructure only: it pins oracle/head_oracle.c.
#include <cstddef>
#include <cstdint>

#include "ultima/kernels/matvec.hpp"
#include "ultima/kernels/norms.hpp"

extern "C" {
void ref_rmsnorm(const float* x, const float* scale, float* y, int64_t n, float eps) {
    ultima::kernels::rmsnorm_f32(x, scale, y, (std::size_t)n, eps);
}
void ref_matvec_f32(const float* w, const float* x, float* y, int64_t M, int64_t K) {
    ultima::kernels::matvec_f32_f32(w, x, y, (std::size_t)M, (std::size_t)K);
}
void ref_matvec_bf16(const uint16_t* w, const float* x, float* y, int64_t M, int64_t K) {
    ultima::kernels::matvec_bf16_f32(reinterpret_cast<const std::uint8_t*>(w), x, y, (std::size_t)M, (std::size_t)K);
}
}
