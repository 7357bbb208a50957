// Internal entry points shared between the libweft_hip translation units.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace weft {

// Decode GEMV launchers (quantize X in-kernel, write Xq, any M).
void decode_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                size_t M);
void decode_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M);
void decode_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M);
void decode_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                    const int8_t* signs, float* Y, size_t N, size_t K, size_t M);

// Q4_K mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M);

// Q4_0 / MXFP4 mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                  size_t M);
void mul_mat_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* scale, float* Y, size_t N, size_t K, size_t M);

// IQ2_XXS mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                     const int8_t* signs, float* Y, size_t N, size_t K, size_t M);

// Activation quantizers over K contiguous values.
void quantize_q8_k(const float* X, uint8_t* Y, size_t K);
void quantize_q8_0(const float* X, uint8_t* Y, size_t K);

}  // namespace weft
