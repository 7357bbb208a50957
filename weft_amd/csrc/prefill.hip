// Prefill (many activation rows) production mul_mat entry points.
//
// production_mul_mat_{q4_0,q4_k,q4_k_staged,iq2_xxs,iq2_xxs_staged,mxfp4}
// (examples/kernels/mul_mat/*.py) compute the same Y = X . W^T as the decode
// kernels; the reference's variants differ only in CPU loop order.
// production_mul_mat_q4_k_persistent (mul_mat/q4_k_persistent.py:10-31)
// computes it from the persisted Q4K_I[16] interleave of W, with the
// artifact-phase _W_packed_size / _W_pack of that derived layout.  All four
// formats run int8-MFMA GEMMs for prefill shapes (prefill_q4k.hip,
// prefill_q80.hip, prefill_iq2.hip) and the decode GEMV kernels otherwise
// (small M, unaligned weights, K that does not fill the GEMM's staging unit).
#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

extern "C" {

void production_mul_mat_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                             size_t K, size_t M) {
  weft::mul_mat_q4_0(W, X, Xq, Y, N, K, M, weft::packed(K / 32 * weft::kQ4_0Bytes, K, N));
}

void production_mul_mat_q4_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                             size_t K, size_t M) {
  weft::mul_mat_q4k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ4_KBytes, K, N));
}

void production_mul_mat_q4_k_staged(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  weft::mul_mat_q4k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ4_KBytes, K, N));
}

size_t production_mul_mat_q4_k_persistent_W_packed_size(size_t N, size_t K) {
  return weft::q4k_i16_packed_size(N, K);
}

void production_mul_mat_q4_k_persistent_W_pack(const uint8_t* source, uint8_t* target, size_t N,
                                               size_t K) {
  weft::q4k_i16_pack(source, target, N, K);
}

void production_mul_mat_q4_k_persistent(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                        size_t M, size_t K, size_t N) {
  weft::mul_mat_q4k_persistent(W, X, Xq, Y, M, K, N);
}

void production_mul_mat_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                                const int8_t* signs, float* Y, size_t N, size_t K, size_t M) {
  weft::mul_mat_iq2_xxs(W, X, Xq, grid, signs, Y, N, K, M,
                        weft::packed(K / 256 * weft::kIq2xxsBytes, K, N));
}

void production_mul_mat_iq2_xxs_staged(const uint8_t* W, const float* X, uint8_t* Xq,
                                       const int8_t* grid, const int8_t* signs, float* Y, size_t N,
                                       size_t K, size_t M) {
  weft::mul_mat_iq2_xxs(W, X, Xq, grid, signs, Y, N, K, M,
                        weft::packed(K / 256 * weft::kIq2xxsBytes, K, N));
}

void production_mul_mat_q4_1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                             size_t K, size_t M) {
  weft::mul_mat_q4_1(W, X, Xq, Y, N, K, M, weft::packed(K / 32 * weft::kQ4_1Bytes, K, N));
}

void production_mul_mat_iq2_xs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                               const int8_t* signs, float* Y, size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::mul_mat_iq2_xs(W, X, Xq, grid, signs, Y, N, K, M, weft::packed(K / 256 * weft::kIq2xsBytes, K, N));
}

void production_mul_mat_iq2_xs_staged(const uint8_t* W, const float* X, uint8_t* Xq,
                                      const int8_t* grid, const int8_t* signs, float* Y, size_t N,
                                      size_t K, size_t M) {
  production_mul_mat_iq2_xs(W, X, Xq, grid, signs, Y, N, K, M);
}

void production_mul_mat_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                              const float* scale, float* Y, size_t N, size_t K, size_t M) {
  weft::mul_mat_mxfp4(W, X, Xq, codebook, scale, Y, N, K, M,
                      weft::packed(K / 32 * weft::kMxfp4Bytes, K, N));
}

}  // extern "C"
