/*
 * MatMulNBits CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This is the checker the HIP path is compared against and the CPU baseline
 * that bench.py times beside it. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. The product library never links or
 * calls it.
 *
 * Operator contract (com.microsoft::MatMulNBits, bits = 4):
 *   A      fp32 [M, K] row-major
 *   B      uint8 [N, nb, bs/2] with nb = ceil(K / bs); element k = b*bs + j of
 *          row n is nibble j of B[n, b, :], low nibble first
 *   scales fp32 [N, nb]
 *   zp     uint8 [N, ceil(nb/2)] (nibble b of row n, low nibble first) or
 *          absent, meaning zp = 8
 *   Y      fp32 [M, N],  Y[m,n] = sum_k A[m,k] * (q[n,k] - zp[n,k/bs]) * scale[n,k/bs]
 *
 * Reference anchors (paths relative to the onnx-light-cpu tree):
 *   nibble order    onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.cc:60-65,
 *                   integer_gemm_vnni.h:42-51
 *   fp32 GEMV order onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258 (GemmSkinnyM:
 *                   one fp32 accumulator per output, k ascending, mul then add)
 *   partitioning    onnx_light_cpu/impl/execution.h:72-107 (ExecutionBlockCount,
 *                   grain 2^15, contiguous ranges)
 *   fp32 -> fp16    onnx_light_cpu/impl/math/half_conversion.h:42-78
 *   planned int4    docs/next_steps/2026/2026_08_qwen3_inference.rst:196-230
 *                   (fp32 accumulation, weights never fully expanded, output
 *                   columns partitioned so each weight byte streams once)
 */
#ifndef MNB_ORACLE_H
#define MNB_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* nibble i of a low-nibble-first packed buffer (integer_gemm_vnni.cc:60-65, unsigned) */
int mnbo_nibble(const uint8_t *packed, int64_t index);

/* W[n, k] = float(q - zp) * scale in fp32 (one rounding), W is [N, K] row-major */
void mnbo_dequantize(int64_t K, int64_t N, int64_t block_size, const uint8_t *B,
                     const float *scales, const uint8_t *zero_points, float *W);

/* Exact-product fp64 oracle: Y64[m, n] = sum_k (double)A * (double)(q - zp) * (double)scale */
void mnbo_matmul_nbits_f64(int64_t M, int64_t K, int64_t N, int64_t block_size,
                           const float *A, const uint8_t *B, const float *scales,
                           const uint8_t *zero_points, double *Y64, int threads);

/* Reference-order fp32: dequantize W in fp32, then for every output one fp32
 * accumulator, k ascending, acc = acc + a*w with separate rounding (GemmSkinnyM). */
void mnbo_matmul_nbits_ref_f32(int64_t M, int64_t K, int64_t N, int64_t block_size,
                               const float *A, const uint8_t *B, const float *scales,
                               const uint8_t *zero_points, float *Y, int threads);

/* Fused CPU GEMV (the roadmap's int4_gemv): unpack -> scale -> fp32 accumulate
 * without expanding W, output columns partitioned over threads. */
void mnbo_matmul_nbits_fused_f32(int64_t M, int64_t K, int64_t N, int64_t block_size,
                                 const float *A, const uint8_t *B, const float *scales,
                                 const uint8_t *zero_points, float *Y, int threads);

/* Sum over k of |A[m,k]| * |W[n,k]| in fp64: the error scale of one output. */
void mnbo_abs_dot_f64(int64_t M, int64_t K, int64_t N, int64_t block_size, const float *A,
                      const uint8_t *B, const float *scales, const uint8_t *zero_points,
                      double *out, int threads);

/* fp32 -> fp16 bits, round to nearest even (half_conversion.h:42-78) */
uint16_t mnbo_f32_to_f16_bits(float value);
/* fp16 bits -> fp32, exact */
float mnbo_f16_bits_to_f32(uint16_t bits);
/* array forms of the two conversions */
void mnbo_f32_to_f16_array(const float *in, uint16_t *out, int64_t count);
void mnbo_f16_to_f32_array(const uint16_t *in, float *out, int64_t count);

/* Number of contiguous blocks the reference's ExecutionBlockCount would make
 * for `total` items of cost `cost_per_item` with `threads` participants. */
int64_t mnbo_execution_block_count(int64_t total, double cost_per_item, int64_t threads);

#ifdef __cplusplus
}
#endif

#endif
