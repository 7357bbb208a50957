/*
 * CPU oracle for the quantized mul_mat hot path (TEST INFRASTRUCTURE ONLY).
 *
 * A plain-C restatement of the GGML CPU functions that the reference Weft
 * repository uses as its numeric oracle (vendored GGML under
 * source/c/ggml/llama.cpp/ggml/src/).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker or the timed CPU baseline: the product path (libweft_hip) never
 * calls into it.
 *
 * Record layouts (bytes, little endian), ggml-common.h:
 *   Q4_0    18 B / 32  : f16 d | u8 qs[16]                       (:184-189)
 *   MXFP4   17 B / 32  : u8 e  | u8 qs[16]                       (:204-209)
 *   NVFP4   36 B / 64  : u8 d[4] (UE4M3) | u8 qs[32]            (:211-217)
 *   Q8_0    34 B / 32  : f16 d | i8 qs[32]                       (:241-246)
 *   Q4_K   144 B / 256 : f16 d | f16 dmin | u8 scales[12] | u8 qs[128]  (:317-328)
 *   Q8_K   292 B / 256 : f32 d | i8 qs[256] | i16 bsums[16]      (:361-366)
 *   IQ2_XXS 66 B / 256 : f16 d | u16 qs[32]                      (:371-375)
 */
#ifndef WEFT_ORACLE_H
#define WEFT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum wo_format {
  WO_Q4_0 = 0,
  WO_Q4_K = 1,
  WO_IQ2_XXS = 2,
  WO_MXFP4 = 3,
  WO_Q6_K = 4,
  WO_Q5_K = 5,
  WO_NVFP4 = 6,
  WO_Q4_1 = 7,
  WO_IQ2_XS = 8,
};

/* scalar conversions (ggml-impl.h:384-431, :477-495) */
float wo_fp16_to_fp32(uint16_t h);
uint16_t wo_fp32_to_fp16(float f);
float wo_e8m0_to_fp32_half(uint8_t e);
void wo_fp16_to_fp32_array(const uint16_t *h, float *out, int64_t n);
void wo_fp32_to_fp16_array(const float *f, uint16_t *out, int64_t n);

/* lookup tables, built from closed forms */
void wo_iq2xxs_grid(uint8_t out[2048]);  /* 256 x 8 magnitudes {8,25,43} */
void wo_ksigns_iq2xs(uint8_t out[128]);  /* i | parity(i) << 7 */
void wo_signs_i8x8(int8_t out[1024]);    /* 128 x 8 of +-1, the ABI's I8X8 sign table */
void wo_kvalues_mxfp4(int8_t out[16]);   /* doubled e2m1 */
void wo_iq2xs_grid(uint8_t out[4096]);   /* 512 x 8 magnitudes {8,25,43} */
void wo_e8m0_half_table(float out[256]);
float wo_ue4m3_to_fp32(uint8_t x);       /* ggml_ue4m3_to_fp32, incl. the 1/2 */
uint8_t wo_fp32_to_ue4m3(float x);
void wo_ue4m3_table(float out[256]);

/* weight quantizers (host-side input generators) */
void wo_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_q4_K(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_mxfp4(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_iq2_xxs(const float *x, uint8_t *y, int64_t k);
/* GGML's quantize_iq2_xxs / quantize_iq2_xs (ggml-quants.c:3580-3602):
 * quant_weights = the importance matrix (k values), NULL = all ones */
void wo_quantize_row_iq2_xxs_ggml(const float *x, uint8_t *y, int64_t k, const float *quant_weights);
void wo_quantize_row_iq2_xs_ggml(const float *x, uint8_t *y, int64_t k, const float *quant_weights);
/* the search tables of iq2xs_init_impl (xs: 0 = IQ2_XXS, 1 = IQ2_XS): the
 * grid index of 2-bit point u (-1: not on the grid), and its neighbour list
 * (returns the count written to out, 0 for a grid point) */
int wo_iq2_grid_index(int xs, int u);
int wo_iq2_neighbours(int xs, int u, uint16_t *out);
void wo_quantize_row_q6_K(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_q5_K(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_nvfp4(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_q4_1(const float *x, uint8_t *y, int64_t k);

/* activation quantizers (on the hot path) */
void wo_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_q8_K(const float *x, uint8_t *y, int64_t k);
void wo_quantize_row_q8_1(const float *x, uint8_t *y, int64_t k);

/* row dequantizers */
void wo_dequantize_row_q4_0(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_q4_K(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_iq2_xxs(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_mxfp4(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_q6_K(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_q5_K(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_nvfp4(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_q4_1(const uint8_t *x, float *y, int64_t k);
void wo_dequantize_row_iq2_xs(const uint8_t *x, float *y, int64_t k);

/* generic vec_dots: w row (k elements) . quantized activation row */
float wo_vec_dot_q4_0_q8_0(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_q4_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_iq2_xxs_q8_K(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_mxfp4_q8_0(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_q6_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_q5_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_nvfp4_q8_0(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_q4_1_q8_1(const uint8_t *w, const uint8_t *x, int64_t k);
float wo_vec_dot_iq2_xs_q8_K(const uint8_t *w, const uint8_t *x, int64_t k);

/* Bytes of one encoded row of k elements for a weight format, or of the
 * activation format that pairs with it (Q8_0 for Q4_0/MXFP4, Q8_K else). */
size_t wo_weight_row_bytes(int fmt, int64_t k);
size_t wo_act_row_bytes(int fmt, int64_t k);

/* GGML MUL_MAT semantics (ggml-cpu.c:1245-1443): quantize every row of
 * X (M x K) into Xq, then Y[m, n] = vec_dot(W[n], Xq[m]).  Rows of W are
 * split over nthreads threads (nthreads <= 0: all OpenMP threads). */
void wo_mul_mat(int fmt, const uint8_t *W, const float *X, uint8_t *Xq,
                float *Y, int64_t N, int64_t K, int64_t M, int nthreads);
/* Same loop over an already-quantized Xq (the vec_dot-only part). */
void wo_mul_mat_q(int fmt, const uint8_t *W, const uint8_t *Xq, float *Y,
                  int64_t N, int64_t K, int64_t M, int nthreads);

/* fp64 re-accumulation of the exact integer partials of every output:
 * E[m, n] = sum_b scale_b * P_b evaluated in double, and
 * A[m, n] = sum_b |scale_b * P_b| (the magnitude a tolerance is taken on),
 * b over the format's scale groups: 32-blocks, NVFP4's 16-sub-blocks, the
 * K-quants' sub-blocks (Q4_K / Q5_K: the scale and the min term of each),
 * IQ2_XXS's 32-groups and IQ2_XS's 16-halves. */
void wo_mul_mat_f64(int fmt, const uint8_t *W, const uint8_t *Xq, double *E,
                    double *A, int64_t N, int64_t K, int64_t M, int nthreads);

/* Integer partials of one row pair, for exactness checks on tiny inputs:
 * Q4_0 / MXFP4 : one int32 per 32-block (P)
 * Q4_K / Q5_K  : per superblock, 8 sub-block sums P_s then the min sum Mn
 * IQ2_XXS      : one int32 per 32-group (I_g * (2 s_g + 1))
 * IQ2_XS       : one int32 per 16-element half (its 4-bit scale's partial)
 * NVFP4        : one int32 per 16-element sub-block
 * Q6_K         : per superblock, the 16 group sums P_g (16 elements each)
 * returns the number of int32 written. */
int64_t wo_int_partials(int fmt, const uint8_t *w, const uint8_t *x, int64_t k,
                        int32_t *out);

/* GGML's threaded MUL_MAT as ggml_compute_forward_mul_mat schedules it
 * (ggml-cpu/ggml-cpu.c:1313-1443) for a 2-D F32 src1: thread ith quantizes
 * blocks [ith*nb/nth, (ith+1)*nb/nth) of every row, then all threads take
 * chunks of dr0 weight rows x dr1 activation rows (chunk size 16, 64 when
 * either side is a single row; one chunk per thread along the longer side
 * when there are fewer than 4 chunks per thread), the first at their own
 * index and the rest from a shared counter, and walk a chunk in 16 x 16
 * blocks.  nthreads <= 0: all OpenMP threads. */
void wo_mul_mat_ggml(int fmt, const uint8_t *W, const float *X, uint8_t *Xq,
                     float *Y, int64_t N, int64_t K, int64_t M, int nthreads);

/* Walk (read and write) `bytes` of `buf`: the reference timing protocol's
 * cache eviction between timed calls (doc/experiments/protocol.md:46-55). */
void wo_evict(uint8_t *buf, size_t bytes);

/* Threads OpenMP would use by default (for reporting the CPU baseline). */
int wo_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
