/*
 * libweft_hip -- MI355X (gfx950) implementation of Weft's quantized mul_mat
 * hot path behind Weft's generated-kernel C ABI.
 *
 * ABI rules kept from the reference (lib/Target/Emission/Emitter.h:465-512):
 *   void <symbol>(<one pointer per View parameter, in signature order>,
 *                 <one size_t per shape symbol, in first-appearance order>);
 *   record encodings travel as uint8_t*, dense views as their element type,
 *   read-only views are const.  The library allocates nothing, keeps no
 *   cross-call state, and never repacks or copies its arguments.
 *
 * HIP specifics:
 *   - every pointer is a DEVICE pointer (hipMalloc / torch device memory);
 *   - each call enqueues on the calling thread's current stream
 *     (weft_hip_set_stream; default: the null stream) and returns without
 *     waiting: results are visible to later work on that stream, or to the
 *     host after weft_hip_synchronize();
 *   - the kernels have no failure channel; shape/pointer errors found before
 *     the launch and launch errors are recorded per thread and returned (and
 *     cleared) by weft_hip_get_last_error(); nothing is launched for an
 *     invalid call.
 *
 * Record layouts are GGML's (source/c/ggml/llama.cpp/ggml/src/ggml-common.h):
 *   Q4_0 18 B/32, MXFP4 17 B/32, Q8_0 34 B/32, Q4_K 144 B/256,
 *   Q8_K 292 B/256, IQ2_XXS 66 B/256.
 * Table arguments: grid = I8X8[256x8] iq2xxs grid magnitudes (GGML's
 * tables hold 8, 25 and 43 only; the kernels negate grid bytes in place
 * and need every byte in [1, 127]), signs = I8X8[128x8] of +-1, codebook = int8[16] doubled E2M1, scale = fp32[256]
 * e8m0 "half" scales (examples/repro/weft/mul_mat_runtime.cpp:151-159).
 *
 * Reference citations are relative to the Weft repository root.
 */
#ifndef WEFT_HIP_H
#define WEFT_HIP_H

#include <stddef.h>
#include <stdint.h>

#define WEFT_HIP_VERSION_STRING "weft_hip 0.1 gfx950"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ control API */
/* No counterpart in the reference (its kernels are synchronous host C). */
int weft_hip_set_stream(void *stream);   /* hipStream_t; thread-local */
void *weft_hip_get_stream(void);
/* Source tile bindings of the calling thread (CompileOptions.meta; no
 * counterpart in the generated C, where they are compile-time constants):
 * "NC" = weight rows per workgroup and "MR" = activation rows per pass
 * (1..4) of the GEMV kernels; for the Q4_K prefill GEMM (M >= 16 of
 * production_mul_mat_q4_k_staged / production_mul_mat_q4_k) "NC" = weight
 * rows per tile (<= 64: 64, else 128) and "MC" = activation rows per tile
 * (<= 32: 32, else 64); 0 unsets.  Returns 1 when the name has a launch
 * knob here, 0 otherwise (KC, NR and the other MFMA GEMMs' fixed 64 x 128
 * tiles).  weft_hip_clear_tile_bindings unsets every binding. */
int weft_hip_set_tile_binding(const char *name, size_t value);
void weft_hip_clear_tile_bindings(void);
int weft_hip_get_last_error(void);       /* hipError_t, then cleared */
const char *weft_hip_error_string(int code);
int weft_hip_synchronize(void);          /* hipStreamSynchronize(current) */
const char *weft_hip_version(void);
/* Target discovery (stands in for weft-compile --query-native-target,
 * python/weft/runtime/driver.py:62-69): number of visible HIP devices, or a
 * negative hipError_t; the gcnArchName of device `dev` copied into `buf`. */
int weft_hip_device_count(void);
int weft_hip_device_arch(int dev, char *buf, size_t len);
/* ABI metadata of every exported kernel, as the JSON artifact weft-compile
 * emits (tools/weft-compile/weft-compile.cpp:116-147, kind
 * "weft-hip-artifact", gfx_arch / wavefront_size in place of march / abi /
 * vlen_bits). */
const char *weft_hip_artifact(void);
/* Launch log of the calling thread, a debugging and measurement aid that is
 * off by default: weft_hip_set_launch_log(1) turns it on (0 turns it off and
 * empties it) and returns the previous setting.  While on, the names of the
 * kernels this thread launches are appended, keeping at most the last 4096
 * bytes.  weft_hip_launch_log copies the names since the last read, comma
 * separated, into buf (len bytes with the NUL) and clears them; it returns
 * the log's length, and buf == NULL only returns the length. */
int weft_hip_set_launch_log(int enable);
size_t weft_hip_launch_log(char *buf, size_t len);
/* Measurement probes on the current stream: an empty launch, and one launch
 * that reads `bytes` (a multiple of 16, 16-byte aligned) of device memory
 * with `grid` x 512 threads and writes one word per wave into sink
 * (grid * 8 words). */
void weft_hip_probe_empty(void);
void weft_hip_probe_read(const void *src, size_t bytes, uint32_t *sink, int grid);
/* The same read in another shape: `threads` per workgroup (64..1024, a
 * multiple of 64), `unroll` 16-byte loads in flight per lane (1, 2, 4, 8,
 * 16), flags bit 0 = nontemporal loads, bit 1 = each workgroup reads one
 * contiguous chunk instead of the grid striding over the buffer; sink holds
 * grid * threads / 64 words.  weft_hip_probe_read is (512, 4, 0). */
void weft_hip_probe_read_shape(const void *src, size_t bytes, uint32_t *sink, int grid, int threads,
                               int unroll, int flags);
/* The write-side twin: writes `bytes` (a multiple of 16, 16-byte aligned) of
 * device memory with 16-byte stores, `threads` per workgroup as above,
 * `unroll` stores in flight per lane (1, 2 or 4), flags as above (bit 0:
 * nontemporal stores).  No counterpart in the reference: the floor a
 * write-bound kernel (row dequantize) is measured against. */
void weft_hip_probe_write_shape(void *dst, size_t bytes, int grid, int threads, int unroll, int flags);
/* Matrix-pipe probe: one workgroup per CU with `waves_per_simd` (1..4)
 * waves per SIMD, each running `iters` iterations of two
 * v_mfma_i32_32x32x32_i8 with `valu_per_mfma` (0, 4, 8, 12 or 16)
 * independent integer VALU instructions after each; sink holds
 * cu_count * 256 * waves_per_simd words.  Time per MFMA = elapsed /
 * (2 * iters * waves_per_simd). */
void weft_hip_probe_mfma(int valu_per_mfma, int waves_per_simd, int iters, uint32_t *sink);

/* ------------------------------------------------------ row dequantize */
/* examples/kernels/dequantize/q4_0.py:9-13; repro row_dequantize_runtime.cpp:177 */
void row_dequantize_q4_0(const uint8_t *W, float *Y, size_t K);
/* examples/kernels/dequantize/q4_k.py:9-20; row_dequantize_runtime.cpp:212 */
void row_dequantize_q4_k(const uint8_t *W, float *Y, size_t K);
/* examples/kernels/dequantize/iq2_xxs.py:9-53; row_dequantize_runtime.cpp:247 */
void row_dequantize_iq2_xxs(const uint8_t *W, const int8_t *grid, const int8_t *signs, float *Y,
                            size_t K);
/* examples/kernels/dequantize/mxfp4.py:9-20; row_dequantize_runtime.cpp:282 */
void row_dequantize_mxfp4(const uint8_t *W, const int8_t *codebook, const float *scale, float *Y,
                          size_t K);
/* examples/kernels/dequantize/q6_k.py:8-15; row_dequantize_runtime.cpp:222 */
void row_dequantize_q6_k(const uint8_t *W, float *Y, size_t K);
/* examples/kernels/dequantize/nvfp4.py:9-24; row_dequantize_runtime.cpp:287 */
void row_dequantize_nvfp4(const uint8_t *W, const int8_t *codebook, const float *scale, float *Y,
                          size_t K);
/* examples/kernels/dequantize/q5_k.py:9-15; row_dequantize_runtime.cpp:217 */
void row_dequantize_q5_k(const uint8_t *W, float *Y, size_t K);
/* examples/kernels/dequantize/q4_1.py:9-13; row_dequantize_runtime.cpp:182 */
void row_dequantize_q4_1(const uint8_t *W, float *Y, size_t K);
/* examples/kernels/dequantize/iq2_xs.py:9-75; row_dequantize_runtime.cpp:242 */
void row_dequantize_iq2_xs(const uint8_t *W, const int8_t *grid, const int8_t *signs, float *Y,
                           size_t K);

/* ------------------------------------------------ activation quantize */
/* examples/kernels/quantize/q8_0.py:26-28; repro q8_quantize_runtime.cpp:25 */
void q8_0_quantize(const float *X, uint8_t *Y, size_t K);
/* examples/kernels/quantize/q8_k.py:38-40; repro q8_quantize_runtime.cpp:26 */
void q8_K_quantize(const float *X, uint8_t *Y, size_t K);
/* examples/kernels/quantize/q8_1.py:28-30; repro q8_quantize_runtime.cpp:18, :43 */
void q8_1_quantize(const float *X, uint8_t *Y, size_t K);

/* ------------------------------------------------------------ vec_dot */
/* examples/kernels/vec_dot/q4_0_q8_0.py:8-23; repro vec_dot_runtime.cpp:191 */
void quantized_vec_dot_q4_0_q8_0(const uint8_t *W, const uint8_t *X, float *Y, size_t K);
/* examples/kernels/vec_dot/q4_k_q8_k.py:8-36; vec_dot_runtime.cpp:247 */
void quantized_vec_dot_q4_k_q8_k(const uint8_t *W, const uint8_t *X, float *Y, size_t K);
/* examples/kernels/vec_dot/iq2_xxs_q8_k.py:8-54; vec_dot_runtime.cpp:303 */
void quantized_vec_dot_iq2_xxs_q8_k(const uint8_t *W, const uint8_t *X, const int8_t *grid,
                                    const int8_t *signs, float *Y, size_t K);
/* examples/kernels/vec_dot/mxfp4_q8_0.py:9-33; vec_dot_runtime.cpp:359 */
void quantized_vec_dot_mxfp4_q8_0(const uint8_t *W, const uint8_t *X, const int8_t *codebook,
                                  const float *scale, float *Y, size_t K);
/* examples/kernels/vec_dot/q6_k_q8_k.py:8-44; vec_dot_runtime.cpp:263 */
void quantized_vec_dot_q6_k_q8_k(const uint8_t *W, const uint8_t *X, float *Y, size_t K);
/* examples/kernels/vec_dot/nvfp4_q8_0.py:9-38; vec_dot_runtime.cpp:367 */
void quantized_vec_dot_nvfp4_q8_0(const uint8_t *W, const uint8_t *X, const int8_t *codebook,
                                  const float *scale, float *Y, size_t K);
/* examples/kernels/vec_dot/q5_k_q8_k.py:8-38; vec_dot_runtime.cpp:255 */
void quantized_vec_dot_q5_k_q8_k(const uint8_t *W, const uint8_t *X, float *Y, size_t K);
/* examples/kernels/vec_dot/q4_1_q8_1.py:8-29; vec_dot_runtime.cpp:199 */
void quantized_vec_dot_q4_1_q8_1(const uint8_t *W, const uint8_t *X, float *Y, size_t K);
/* examples/kernels/vec_dot/iq2_xs_q8_k.py:9-45; vec_dot_runtime.cpp:295 */
void quantized_vec_dot_iq2_xs_q8_k(const uint8_t *W, const uint8_t *X, const int8_t *grid,
                                   const int8_t *signs, float *Y, size_t K);

/* --------------------------------------------------- production mul_mat */
/* W (N x K) encoded, X (M x K) fp32, Xq (M x K) written with the
 * activation quantization, Y (M x N) fp32 = X . W^T.  Shape order N, K, M. */

/* examples/kernels/mul_mat/q4_0.py:9-30; mul_mat_runtime.cpp:220 */
void production_mul_mat_q4_0(const uint8_t *W, const float *X, uint8_t *Xq, float *Y, size_t N,
                             size_t K, size_t M);
/* examples/kernels/mul_mat/q4_0_decode.py:10-20; mul_mat_runtime.cpp:217 */
void production_mul_mat_q4_0_decode(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/q4_k.py:10-20; mul_mat_runtime.cpp:356 */
void production_mul_mat_q4_k(const uint8_t *W, const float *X, uint8_t *Xq, float *Y, size_t N,
                             size_t K, size_t M);
/* examples/kernels/mul_mat/q4_k_decode.py:10-20; mul_mat_runtime.cpp:332-336 */
void production_mul_mat_q4_k_decode(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/q4_k_staged.py:9-37; mul_mat_runtime.cpp:350-354 */
void production_mul_mat_q4_k_staged(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/q4_k_persistent.py:10-31; mul_mat_runtime.cpp:338-347, :807-808.
 * W is the Q4K_I[16] interleave of an N x K Q4_K matrix (N a multiple of 16;
 * layout as for q4_k_q8_k_gemv below), made by _W_pack from row-major Q4_K
 * (device pointers, target 16-byte aligned).  The artifact-phase functions
 * take the derive builder's shape names (examples/formats/ggml.py:286-290):
 * their M is the weight's row count, the kernel's N.  The kernel's shape
 * parameters come in the artifact's order M, K, N (the builder's symbols
 * first), M being the activation's rows. */
size_t production_mul_mat_q4_k_persistent_W_packed_size(size_t M, size_t K);
void production_mul_mat_q4_k_persistent_W_pack(const uint8_t *source, uint8_t *target, size_t M,
                                               size_t K);
void production_mul_mat_q4_k_persistent(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                        size_t M, size_t K, size_t N);
/* examples/kernels/mul_mat/iq2_xxs.py; mul_mat_runtime.cpp:472 */
void production_mul_mat_iq2_xxs(const uint8_t *W, const float *X, uint8_t *Xq, const int8_t *grid,
                                const int8_t *signs, float *Y, size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/iq2_xxs_decode.py:10-23; mul_mat_runtime.cpp:458-463 */
void production_mul_mat_iq2_xxs_decode(const uint8_t *W, const float *X, uint8_t *Xq,
                                       const int8_t *grid, const int8_t *signs, float *Y, size_t N,
                                       size_t K, size_t M);
/* examples/kernels/mul_mat/iq2_xxs_staged.py:86-97; mul_mat_runtime.cpp:465-470 */
void production_mul_mat_iq2_xxs_staged(const uint8_t *W, const float *X, uint8_t *Xq,
                                       const int8_t *grid, const int8_t *signs, float *Y, size_t N,
                                       size_t K, size_t M);
/* examples/kernels/mul_mat/mxfp4.py:10-35; mul_mat_runtime.cpp:567 */
void production_mul_mat_mxfp4(const uint8_t *W, const float *X, uint8_t *Xq, const int8_t *codebook,
                              const float *scale, float *Y, size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/mxfp4_decode.py:10-23; mul_mat_runtime.cpp:564 */
void production_mul_mat_mxfp4_decode(const uint8_t *W, const float *X, uint8_t *Xq,
                                     const int8_t *codebook, const float *scale, float *Y,
                                     size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/q4_1.py:9-30; mul_mat_runtime.cpp:235-236 */
void production_mul_mat_q4_1(const uint8_t *W, const float *X, uint8_t *Xq, float *Y, size_t N,
                             size_t K, size_t M);
/* examples/kernels/mul_mat/q4_1_decode.py:10-20; mul_mat_runtime.cpp:232-233 */
void production_mul_mat_q4_1_decode(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/iq2_xs.py:26-56; mul_mat_runtime.cpp:446-447 */
void production_mul_mat_iq2_xs(const uint8_t *W, const float *X, uint8_t *Xq, const int8_t *grid,
                               const int8_t *signs, float *Y, size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/iq2_xs_staged.py:29-75; mul_mat_runtime.cpp:443-444 */
void production_mul_mat_iq2_xs_staged(const uint8_t *W, const float *X, uint8_t *Xq,
                                      const int8_t *grid, const int8_t *signs, float *Y, size_t N,
                                      size_t K, size_t M);
/* examples/kernels/mul_mat/q6_k.py:9-37; mul_mat_runtime.cpp:386 */
void production_mul_mat_q6_k(const uint8_t *W, const float *X, uint8_t *Xq, float *Y, size_t N,
                             size_t K, size_t M);
/* examples/kernels/mul_mat/q6_k_decode.py:10-20; mul_mat_runtime.cpp:383 */
void production_mul_mat_q6_k_decode(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/nvfp4.py:10-43; mul_mat_runtime.cpp:582 */
void production_mul_mat_nvfp4(const uint8_t *W, const float *X, uint8_t *Xq, const int8_t *codebook,
                              const float *scale, float *Y, size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/nvfp4_decode.py:10-23; mul_mat_runtime.cpp:579 */
void production_mul_mat_nvfp4_decode(const uint8_t *W, const float *X, uint8_t *Xq,
                                     const int8_t *codebook, const float *scale, float *Y,
                                     size_t N, size_t K, size_t M);
/* examples/kernels/mul_mat/q5_k.py:9-37; mul_mat_runtime.cpp:371 */
void production_mul_mat_q5_k(const uint8_t *W, const float *X, uint8_t *Xq, float *Y, size_t N,
                             size_t K, size_t M);
/* examples/kernels/mul_mat/q5_k_decode.py:10-20; mul_mat_runtime.cpp:368 */
void production_mul_mat_q5_k_decode(const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                                    size_t N, size_t K, size_t M);

/* ------------------------------- Q4_K GEMV over the Q4K_I[16] layout */
/* W is the persisted 16-row interleave of an M x K Q4_K matrix (M a multiple
 * of 16; examples/formats/ggml.py:286-290): superblock j of rows 16c..16c+15
 * is the 2304-byte block ((c * K/256) + j) * 2304 whose byte 16 b + r is byte
 * b of row 16 c + r's record (lib/Target/Emission/Memory.cpp:984-991).  X is
 * K/256 Q8_K records, Y gets M fp32.  _W_packed_size / _W_pack are the
 * artifact-phase functions Emitter::emitArtifact generates for the derived W
 * (lib/Target/Emission/Emitter.h:231-272): sizes in bytes, and a device-side
 * repack from a row-major Q4_K matrix (source and target are device pointers,
 * target 16-byte aligned).  The _groups4 and _contract variants are the same
 * function (the reference's RVV loop orders of one DSL computation). */

/* examples/kernels/gemv/q4_k.py:8-26; repro q4_k_gemv_runtime.cpp:28-32 */
size_t q4_k_q8_k_gemv_W_packed_size(size_t M, size_t K);
void q4_k_q8_k_gemv_W_pack(const uint8_t *source, uint8_t *target, size_t M, size_t K);
void q4_k_q8_k_gemv(const uint8_t *W, const uint8_t *X, float *Y, size_t M, size_t K);
/* examples/kernels/gemv/q4_k_groups4.py; repro q4_k_gemv_runtime.cpp:20-26 */
size_t q4_k_q8_k_gemv_groups4_W_packed_size(size_t M, size_t K);
void q4_k_q8_k_gemv_groups4_W_pack(const uint8_t *source, uint8_t *target, size_t M, size_t K);
void q4_k_q8_k_gemv_groups4(const uint8_t *W, const uint8_t *X, float *Y, size_t M, size_t K);
/* examples/kernels/gemv/q4_k_contract.py; repro q4_k_gemv_runtime.cpp:13-18 */
size_t q4_k_q8_k_gemv_contract_W_packed_size(size_t M, size_t K);
void q4_k_q8_k_gemv_contract_W_pack(const uint8_t *source, uint8_t *target, size_t M, size_t K);
void q4_k_q8_k_gemv_contract(const uint8_t *W, const uint8_t *X, float *Y, size_t M, size_t K);

/* ----------------------------------------------- GGML MUL_MAT boundary */
/* The quantized mul_mat behind GGML's MUL_MAT op, for a ggml-style graph
 * executor: ggml_compute_forward_mul_mat's contract
 * (source/c/ggml/llama.cpp/ggml/src/ggml-cpu/ggml-cpu.c:1245-1443) with
 * src0 of type Q4_0, Q4_K, Q5_K, Q6_K, IQ2_XXS, MXFP4 or NVFP4, src1 F32 (quantized into wdata
 * as GGML does) or already of src0's vec_dot type, dst F32; GGML's byte
 * strides and broadcast of src0 over src1's planes (ne12 / ne02, ne13 / ne03).
 * All data pointers are device pointers; the call is stream-ordered.
 * Returns 0, or the error it also records for weft_hip_get_last_error():
 * hipErrorInvalidValue where GGML asserts (nothing is launched),
 * hipErrorNotSupported for types outside this path. */

/* enum ggml_type values (ggml/include/ggml.h:389-431) of this path */
enum {
  WEFT_GGML_TYPE_F32 = 0,
  WEFT_GGML_TYPE_Q4_0 = 2,
  WEFT_GGML_TYPE_Q4_1 = 3,
  WEFT_GGML_TYPE_Q8_0 = 8,
  WEFT_GGML_TYPE_Q8_1 = 9,
  WEFT_GGML_TYPE_Q4_K = 12,
  WEFT_GGML_TYPE_Q5_K = 13,
  WEFT_GGML_TYPE_Q6_K = 14,
  WEFT_GGML_TYPE_Q8_K = 15,
  WEFT_GGML_TYPE_IQ2_XXS = 16,
  WEFT_GGML_TYPE_IQ2_XS = 17,
  WEFT_GGML_TYPE_MXFP4 = 39,
  WEFT_GGML_TYPE_NVFP4 = 40
};

/* the fields of struct ggml_tensor (ggml/include/ggml.h:667-692) MUL_MAT reads */
typedef struct weft_ggml_tensor {
  int32_t type;   /* enum ggml_type */
  int64_t ne[4];  /* elements per dimension */
  size_t nb[4];   /* bytes per step of each dimension */
  void *data;     /* device pointer */
} weft_ggml_tensor;

/* ggml_type_size / ggml_blck_size / ggml_row_size (ggml/src/ggml.c:1303-1320)
 * and type_traits_cpu[type].vec_dot_type (ggml-cpu.c:230-331) for this path's
 * types; 0 (-1 for the vec_dot type) for any other type */
size_t weft_ggml_type_size(int32_t type);
int64_t weft_ggml_blck_size(int32_t type);
size_t weft_ggml_row_size(int32_t type, int64_t ne);
int32_t weft_ggml_vec_dot_type(int32_t type);
/* MUL_MAT's work size in ggml_graph_plan (ggml-cpu.c:2819-2826):
 * ggml_row_size(vec_dot_type, nelements(src1)), 0 when src1 needs no quantization */
size_t weft_ggml_mul_mat_work_size(const weft_ggml_tensor *src0, const weft_ggml_tensor *src1);
/* GGML_OP_MUL_MAT (ggml-cpu.c:1245-1443); wdata: work buffer of wsize bytes,
 * 4-byte aligned, ends holding src1 quantized as GGML's wdata would */
int weft_ggml_mul_mat(const weft_ggml_tensor *src0, const weft_ggml_tensor *src1,
                      const weft_ggml_tensor *dst, void *wdata, size_t wsize);
/* MUL_MAT_ID's work size in ggml_graph_plan (ggml-cpu.c:2827-2845, cache line 64) */
size_t weft_ggml_mul_mat_id_work_size(const weft_ggml_tensor *src0, const weft_ggml_tensor *src1,
                                      const weft_ggml_tensor *ids);
/* GGML_OP_MUL_MAT_ID (ggml-cpu.c:1454-1698; shapes of ggml_mul_mat_id,
 * ggml/src/ggml.c:3293-3317): src0 = n_as expert matrices (ne02), ids = I32
 * expert choices (n_ids x n_tokens), dst (ne01, n_ids, n_tokens).  Every
 * (slot, token) pair runs in one launch, its expert read from ids on the
 * device; an id outside [0, n_as) (a GGML assert) leaves its dst row untouched. */
int weft_ggml_mul_mat_id(const weft_ggml_tensor *src0, const weft_ggml_tensor *src1,
                         const weft_ggml_tensor *ids, const weft_ggml_tensor *dst, void *wdata,
                         size_t wsize);
/* No counterpart in the reference.  weft_ggml_mul_mat_id for callers that
 * cannot allocate (HIP graph capture, serving loops that forbid hipMalloc):
 * the work buffer is a static device array the library holds per device
 * (WEFT_GGML_NOALLOC_SCRATCH_BYTES), so the call allocates nothing.  A call
 * whose work size (weft_ggml_mul_mat_id_work_size) exceeds it returns
 * hipErrorOutOfMemory and launches nothing.  Not safe from more than one
 * stream of a device: every call on a device uses the same array, so calls
 * that can overlap (issued by two threads, on two streams, or from two
 * captured graphs replayed concurrently) corrupt each other's quantized src1
 * and expert grouping without any error.  Calls on one stream are ordered
 * and safe. */
#define WEFT_GGML_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int weft_ggml_mul_mat_id_noalloc(const weft_ggml_tensor *src0, const weft_ggml_tensor *src1,
                                 const weft_ggml_tensor *ids, const weft_ggml_tensor *dst);

#ifdef __cplusplus
}
#endif

#endif /* WEFT_HIP_H */
