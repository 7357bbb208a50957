// Internal entry points shared between the libweft_hip translation units.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "pairs.h"

namespace weft {

// Row strides of one mul_mat: bytes between weight rows (ldw), floats between
// activation rows (ldx) and floats between output rows (ldy).  The reference
// ABI's matrices are packed: {row bytes, K, N}.  GGML's MUL_MAT passes its
// tensors' nb01, nb11 / 4 and nb1 / 4 (ggml-cpu/ggml-cpu.c:1245-1443).
struct RowStrides {
  size_t ldw, ldx, ldy;
};

inline RowStrides packed(size_t row_bytes, size_t K, size_t N) { return RowStrides{row_bytes, K, N}; }

// Strides a launcher can take: rows at least as long as the packed ones
// (only checked when there is a second row), weight rows at the Encoding's
// alignment, and every byte offset representable.
inline bool strides_ok(const RowStrides& st, size_t row_bytes, size_t w_align, size_t K, size_t N,
                       size_t ny, size_t M) {
  if (N > 1 && (st.ldw < row_bytes || st.ldw % w_align != 0)) return false;
  if (M > 1 && (st.ldx < K || st.ldy < ny)) return false;
  return st.ldw < ((size_t)1 << 40) && st.ldx < ((size_t)1 << 38) && st.ldy < ((size_t)1 << 38);
}

// Decode GEMV launchers (quantize X in-kernel, write Xq, any M).
void decode_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                size_t M, const RowStrides& st);
// the same GEMV over an already quantized Q8_K activation (Xq read, not written)
void decode_q4k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                          size_t M, const RowStrides& st);
void decode_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
void decode_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
void decode_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                    const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                    const RowStrides& st);
void decode_q6_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
void decode_q5_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
void decode_nvfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);

// Batch-1 Q4_0 (fmt 0) / MXFP4 (1) / NVFP4 (5) / Q4_1 (6) GEMV with the records in VGPRs
// (decode_rec.hip); false, with nothing launched, when the call does not
// suit it (K > 4096, unaligned operands), for the caller's general kernel.
bool decode_rec_m1(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* scale, float* Y, size_t N, size_t K, const RowStrides& st);
// Batch-1 Q5_K GEMV with the records in VGPRs (decode_q5k.hip); false, with
// nothing launched, when the call does not suit it (K > 4096, W or its rows
// not 16-byte aligned).
bool decode_q5k_m1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                   const RowStrides& st);
// Batch-1 Q6_K GEMV with the records in VGPRs (decode_q6k.hip); false when
// the call does not suit it (K > 4096, an odd superblock count, unaligned).
bool decode_q6k_m1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                   const RowStrides& st);
// Batch-1 IQ2_XXS / IQ2_XS (xs) GEMV with the records in VGPRs (decode_iq2.hip);
// false, with nothing launched, when the call does not suit it (K > 4096,
// an odd superblock count, unaligned operands).
bool decode_iq2_m1(bool xs, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                   const int8_t* signs, float* Y, size_t N, size_t K, const RowStrides& st);

// MUL_MAT_ID: the GEMV over every (token, slot) pair of pr, each with the
// expert ids[t, s] selects (one activation row per pair; X quantized into
// xq_out, or the quantized xq_in read).  Q4_K, and Q4_0 (fmt 0), MXFP4 (1),
// IQ2_XXS (2), Q6_K (3), Q5_K (4), NVFP4 (5), Q4_1 (6), IQ2_XS (7).
void decode_q4k_pairs(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
                      float* Y, size_t N, size_t K, const RowStrides& st, const PairArgs& pr,
                      int n_pairs);
void decode_pairs(int fmt, const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
                  const int8_t* tab0, const void* tab1, float* Y, size_t N, size_t K,
                  const RowStrides& st, const PairArgs& pr, int n_pairs);
// MUL_MAT_ID grouping on the device (moe.hip): pairs grouped by expert and
// a table of tiles of at most kMoeTileRows pairs of one expert, written into
// ws (moe_group_bytes of it, 16-byte aligned).  The tile count stays on the
// device; tmax bounds it.
constexpr int kMaxExperts = 4096;
constexpr int kMoeTileRows = 64;
struct MoeGroups {
  int32_t* ntiles;
  int32_t* tiles;  // [tmax][3]: expert, first pair index, pairs
  int32_t* pairs;
  int tmax;
};
inline GroupTiles group_tiles(const MoeGroups& g, const PairArgs& pr) {
  return GroupTiles{g.tiles, g.ntiles, g.pairs, pr.n_ids, pr.ne11, g.tmax, pr.w_es, pr.y_s1, pr.y_s2};
}
int moe_tile_bound(int n_pairs, int n_as);
size_t moe_group_bytes(int n_pairs, int n_as);
MoeGroups moe_group(const PairArgs& pr, int n_pairs, void* ws);
// Q4_K MUL_MAT_ID on the grouped MFMA GEMM: Xq holds the quantized src1 rows
// (token * ne11 + row, xq_bytes in all), ws the grouping (moe_group_bytes).
// _ok: whether the shape suits the GEMM.
bool mul_mat_id_q4k_grouped_ok(const uint8_t* W, size_t xq_bytes, const float* Y, size_t N, size_t K,
                               const RowStrides& st, const PairArgs& pr, int n_pairs, const void* ws,
                               size_t ws_bytes);
void mul_mat_id_q4k_grouped(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                            const RowStrides& st, const PairArgs& pr, int n_pairs, void* ws);
// Q4_0 (fmt 0) / MXFP4 (fmt 1) / NVFP4 (fmt 2) / Q4_1 (fmt 3, Q8_1 activation)
// MUL_MAT_ID on the grouped MFMA GEMMs: src1
// rows (token t, row j) at t * pr.x_s2 + j * pr.x_s1 floats, quantized into
// Xq (planar for the GEMM, GGML's records at the end).
bool mul_mat_id_q80_grouped_ok(int fmt, const uint8_t* W, const float* X, const uint8_t* Xq, const float* Y,
                               size_t N, size_t K, const RowStrides& st, const PairArgs& pr, int n_pairs,
                               int n_tok, const void* ws, size_t ws_bytes, const int8_t* codebook,
                               const float* scale);
void mul_mat_id_q80_grouped(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                            size_t K, const RowStrides& st, const PairArgs& pr, int n_pairs, int n_tok,
                            void* ws, const int8_t* codebook, const float* scale);
// IQ2_XXS / IQ2_XS (xs) MUL_MAT_ID on the grouped MFMA GEMM over quantized Q8_K rows
bool mul_mat_id_iq2_grouped_ok(bool xs, const uint8_t* W, size_t xq_bytes, const float* Y, const int8_t* grid,
                               const int8_t* signs, size_t N, size_t K, const RowStrides& st,
                               const PairArgs& pr, int n_pairs, const void* ws, size_t ws_bytes);
void mul_mat_id_iq2_grouped(bool xs, const uint8_t* W, const uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                            float* Y, size_t N, size_t K, const RowStrides& st, const PairArgs& pr,
                            int n_pairs, void* ws);
// Q4_0 (fmt 0), MXFP4 (1), IQ2_XXS (2), Q6_K (3), Q5_K (4), NVFP4 (5), Q4_1 (6) or
// IQ2_XS (7) GEMV over an already quantized activation (Q8_0, Q8_1 or Q8_K
// records, read only)
// Whether a GEMV keeps one activation row of K values in LDS (the
// staged GEMV by format code as decode_quantized takes it; the Q4_K GEMV;
// the Q4K_I[16] GEMV).  Below 16 activation rows the prefill GEMMs take the
// rows these refuse.
bool staged_gemv_fits(int fmt, size_t K);
// The format's prefill GEMM on X (quantized into Xq) if it takes the call;
// false, with nothing launched, otherwise.  They never fall back to a GEMV,
// so a GEMV entry point can try them first for a row it cannot hold.
bool gemm_q80_try(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
bool gemm_kq_try(bool q6, const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
bool gemm_iq2_try(bool xs, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                  const int8_t* signs, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
bool gemm_q4k_try(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                  const RowStrides& st);
bool q4k_gemv_fits(size_t K);
bool q4k_i16_gemv_fits(size_t M, size_t K);  // M weight rows

void decode_quantized(int fmt, const uint8_t* W, const uint8_t* Xq, const int8_t* tab0,
                      const void* tab1, float* Y, size_t N, size_t K, size_t M,
                      const RowStrides& st);

// Q4_1 x Q8_1 and IQ2_XS x Q8_K decode GEMVs (quantize X in-kernel, write Xq, any M)
void decode_q4_1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
void decode_iq2_xs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                   const int8_t* signs, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);

// Q4_K mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st);
// the same over an already quantized Q8_K activation
void mul_mat_q4k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                           size_t M, const RowStrides& st);

// Q4_K mul_mat over the persisted 16-row interleave Q4K_I[16] (N a multiple
// of 16): GEMM on the cohort blocks for M >= 16, interleaved GEMV per row.
void mul_mat_q4k_persistent(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t M,
                            size_t K, size_t N);

// Q4K_I[16] layout: byte size, device repack from row-major Q4_K, and the
// GEMV of one Q8_K activation row (M weight rows); errors go to set_error.
size_t q4k_i16_packed_size(size_t M, size_t K);
void q4k_i16_pack(const uint8_t* source, uint8_t* target, size_t M, size_t K);
void q4k_i16_gemv(const uint8_t* W, const uint8_t* X, float* Y, size_t M, size_t K);

// Q4_0 / MXFP4 mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                  size_t M, const RowStrides& st);
void mul_mat_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
// Q4_1 x Q8_1: the Q4_0 GEMM body with each block's m * s term, GEMV otherwise
void mul_mat_q4_1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                  size_t M, const RowStrides& st);

// IQ2_XXS mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV otherwise.
void mul_mat_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                     const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                     const RowStrides& st);
// IQ2_XS mul_mat for any M: the IQ2 GEMM with per-16 scales for prefill shapes, GEMV otherwise.
void mul_mat_iq2_xs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                    float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
void mul_mat_iq2_xs_quantized(const uint8_t* W, const uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                              float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
void mul_mat_iq2_xxs_quantized(const uint8_t* W, const uint8_t* Xq, const int8_t* grid,
                               const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                               const RowStrides& st);

// NVFP4 mul_mat for any M: the Q8_0 int8-MFMA GEMM for prefill shapes, GEMV otherwise
void mul_mat_nvfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* ue4m3, float* Y, size_t N, size_t K, size_t M, const RowStrides& st);
// Q6_K / Q5_K mul_mat for any M: int8-MFMA GEMM for prefill shapes, GEMV
// otherwise; _quantized: over an already quantized Q8_K activation.
void mul_mat_q6k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                 const RowStrides& st);
void mul_mat_q5k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                 const RowStrides& st);
void mul_mat_q6k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                           const RowStrides& st);
void mul_mat_q5k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                           const RowStrides& st);
// Q6_K (q6) / Q5_K MUL_MAT_ID on the grouped MFMA GEMM over quantized Q8_K rows
bool mul_mat_id_kq_grouped_ok(bool q6, const uint8_t* W, size_t xq_bytes, const float* Y, size_t N, size_t K,
                              const RowStrides& st, const PairArgs& pr, int n_pairs, const void* ws,
                              size_t ws_bytes);
void mul_mat_id_kq_grouped(bool q6, const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                           const RowStrides& st, const PairArgs& pr, int n_pairs, void* ws);

// Activation quantizers over K contiguous values, and over M rows of K
// values ldx floats apart (records written contiguously).
void quantize_q8_k(const float* X, uint8_t* Y, size_t K);
void quantize_q8_0(const float* X, uint8_t* Y, size_t K);
void quantize_q8_k_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K);
void quantize_q8_0_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K);
void quantize_q8_1_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K);

}  // namespace weft
