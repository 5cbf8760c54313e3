// ref_core_driver.cpp -- C ABI over the reference's own header-only C++ E8 kernels.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile against the reference
// header where it lies (/root/reference/ojasx2/math/csrc/ojasx_math_core.hpp);
// the output goes to oracle/_ref/ and is never linked by the product.  This file
// holds no reference code: it only instantiates the reference's templates.
//
//   ojr_ternary_lut        -> get_ternary_rank_to_coords   (ojasx_math_core.hpp:549-573)
//   ojr_ternary_fwd_f32    -> fused_ternary_e8_gemm_forward (ojasx_math_core.hpp:580-634),
//                             row loop as in ojasx_math_bindings.cpp:454-469
//   ojr_ternary_bwd_dx_f32 -> fused_ternary_e8_gemm_backward_dx (ojasx_math_core.hpp:641-702)
//   ojr_e8_fwd_f32         -> fused_e8_gemm_forward (2-bit, ojasx_math_core.hpp:440-483)
//   ojr_e8_bwd_dx_f32      -> fused_e8_gemm_backward_dx (2-bit, ojasx_math_core.hpp:490-534)
#include <cstdint>
#include "ojasx_math_core.hpp"

using namespace ojasx::math::lattice;

extern "C" {

__attribute__((visibility("default"))) const int8_t* ojr_ternary_lut() {
    return get_ternary_rank_to_coords();
}

__attribute__((visibility("default"))) void ojr_ternary_fwd_f32(
    const float* x, const uint8_t* packed, const float* scales, const float* bias, float* y,
    int64_t M, int64_t K, int64_t N, int64_t gs) {
#pragma omp parallel for schedule(static, 1)
    for (int64_t m = 0; m < M; ++m)
        fused_ternary_e8_gemm_forward<float>(x + m * K, packed, scales, bias, y + m * N, 1,
                                             (size_t)K, (size_t)N, (size_t)gs);
}

__attribute__((visibility("default"))) void ojr_ternary_bwd_dx_f32(
    const float* gy, const uint8_t* packed, const float* scales, float* gx, int64_t M,
    int64_t K, int64_t N, int64_t gs) {
#pragma omp parallel for schedule(static, 1)
    for (int64_t m = 0; m < M; ++m)
        fused_ternary_e8_gemm_backward_dx<float>(gy + m * N, packed, scales, gx + m * K, 1,
                                                 (size_t)K, (size_t)N, (size_t)gs);
}

__attribute__((visibility("default"))) void ojr_e8_fwd_f32(
    const float* x, const uint8_t* packed, const float* scales, const float* bias, float* y,
    int64_t M, int64_t K, int64_t N, int64_t gs) {
#pragma omp parallel for schedule(static, 1)
    for (int64_t m = 0; m < M; ++m)
        fused_e8_gemm_forward<float>(x + m * K, packed, scales, bias, y + m * N, 1, (size_t)K,
                                     (size_t)N, (size_t)gs);
}

__attribute__((visibility("default"))) void ojr_e8_bwd_dx_f32(
    const float* gy, const uint8_t* packed, const float* scales, float* gx, int64_t M,
    int64_t K, int64_t N, int64_t gs) {
#pragma omp parallel for schedule(static, 1)
    for (int64_t m = 0; m < M; ++m)
        fused_e8_gemm_backward_dx<float>(gy + m * N, packed, scales, gx + m * K, 1, (size_t)K,
                                         (size_t)N, (size_t)gs);
}

}  // extern "C"
