// qmm_launchers.hpp - C++-linkage shims with the exact signatures of the reference's
// quantized launchers (src/kernels/dequantize.h:25-132), implemented over the C ABI in qmm.h.
//
// A caller written against the reference (e.g. its device-resident layer pipeline,
// src/kernels/attention.hip:572-599, which calls launch_matmul_q*_device on the null
// stream) links against libqmm_gfx950.so and includes this header instead of dequantize.h.
// Like the reference, failures throw: std::invalid_argument for shapes the block format
// cannot represent, std::runtime_error for HIP errors.
#pragma once

#include <stdexcept>
#include <string>

#include "qmm.h"

namespace qmm_detail {
inline void throw_on_error(int rc) {
    if (rc == QMM_OK) return;
    if (rc == QMM_ERR_INVALID_ARGUMENT) throw std::invalid_argument(qmm_last_error());
    throw std::runtime_error(qmm_last_error());
}
}  // namespace qmm_detail

// Block geometry constants of the reference header (dequantize.h:6-22).
constexpr int QK4_0 = 32;
constexpr int BLOCK_Q4_0_BYTES = 18;
constexpr int QK8_0 = 32;
constexpr int BLOCK_Q8_0_BYTES = 34;
constexpr int QK_K = 256;
constexpr int K_SCALE_SIZE = 12;
constexpr int BLOCK_Q4_K_BYTES = 144;
constexpr int BLOCK_Q6_K_BYTES = 210;

inline void launch_dequantize_q4_0(const void* h_q4, void* h_fp16_out, int num_elements) {
    qmm_detail::throw_on_error(qmm_dequantize_q4_0_host(h_q4, h_fp16_out, num_elements));
}
inline void launch_dequantize_q8_0(const void* h_q8, void* h_fp16_out, int num_elements) {
    qmm_detail::throw_on_error(qmm_dequantize_q8_0_host(h_q8, h_fp16_out, num_elements));
}
inline void launch_dequantize_q4_k(const void* h_q4k, void* h_fp16_out, int num_elements) {
    qmm_detail::throw_on_error(qmm_dequantize_q4_k_host(h_q4k, h_fp16_out, num_elements));
}
inline void launch_dequantize_q6_k(const void* h_q6k, void* h_fp16_out, int num_elements) {
    qmm_detail::throw_on_error(qmm_dequantize_q6_k_host(h_q6k, h_fp16_out, num_elements));
}

inline void launch_matmul_q4_0(const void* h_A_fp16, const void* h_B_q4, void* h_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q4_0_host(h_A_fp16, h_B_q4, h_C_fp16, M, N, K));
}
inline void launch_matmul_q8_0(const void* h_A_fp16, const void* h_B_q8, void* h_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q8_0_host(h_A_fp16, h_B_q8, h_C_fp16, M, N, K));
}
inline void launch_matmul_q4_k(const void* h_A_fp16, const void* h_B_q4k, void* h_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q4_k_host(h_A_fp16, h_B_q4k, h_C_fp16, M, N, K));
}
inline void launch_matmul_q6_k(const void* h_A_fp16, const void* h_B_q6k, void* h_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q6_k_host(h_A_fp16, h_B_q6k, h_C_fp16, M, N, K));
}

// Device launchers: the reference launches on the null stream (dequantize.hip:790, 808).
inline void launch_matmul_q4_0_device(const void* d_A_fp16, const void* d_B_q4, void* d_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q4_0_device(d_A_fp16, d_B_q4, d_C_fp16, M, N, K, nullptr));
}
inline void launch_matmul_q8_0_device(const void* d_A_fp16, const void* d_B_q8, void* d_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q8_0_device(d_A_fp16, d_B_q8, d_C_fp16, M, N, K, nullptr));
}
inline void launch_matmul_q4_k_device(const void* d_A_fp16, const void* d_B_q4k, void* d_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q4_k_device(d_A_fp16, d_B_q4k, d_C_fp16, M, N, K, nullptr));
}
inline void launch_matmul_q6_k_device(const void* d_A_fp16, const void* d_B_q6k, void* d_C_fp16, int M, int N, int K) {
    qmm_detail::throw_on_error(qmm_matmul_q6_k_device(d_A_fp16, d_B_q6k, d_C_fp16, M, N, K, nullptr));
}
