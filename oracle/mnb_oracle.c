/*
 * MatMulNBits CPU oracle -- TEST INFRASTRUCTURE ONLY (see mnb_oracle.h).
 *
 * Plain C restatement of the operator for the checker and the CPU baseline.
 * Compile with -ffp-contract=off: the reference-order mode must round the
 * product and the sum separately, as the reference's GemmSkinnyM does when it
 * is built without FMA (onnx_light_cpu/impl/math/gemm_kernel.cc:1238-1247).
 */
#include "mnb_oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* integer_gemm_vnni.cc:60-65: byte index >> 1, shift 4 * (index & 1), mask 0xF */
int mnbo_nibble(const uint8_t *packed, int64_t index) {
  return (packed[index >> 1] >> ((index & 1) * 4)) & 0x0F;
}

static int64_t num_blocks(int64_t K, int64_t bs) { return (K + bs - 1) / bs; }

static int zero_point_of(const uint8_t *zero_points, int64_t n, int64_t nb, int64_t b) {
  if (zero_points == NULL) return 8; /* 2^(bits-1) */
  const int64_t zp_row_bytes = (nb + 1) / 2;
  return mnbo_nibble(zero_points + n * zp_row_bytes, b);
}

void mnbo_dequantize(int64_t K, int64_t N, int64_t bs, const uint8_t *B, const float *scales,
                     const uint8_t *zero_points, float *W) {
  const int64_t nb = num_blocks(K, bs);
  const int64_t row_bytes = nb * bs / 2;
  for (int64_t n = 0; n < N; ++n) {
    const uint8_t *row = B + n * row_bytes;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t b = k / bs;
      const int q = mnbo_nibble(row, k); /* block b starts at nibble b*bs of the row */
      const int z = zero_point_of(zero_points, n, nb, b);
      W[n * K + k] = (float)(q - z) * scales[n * nb + b];
    }
  }
}

/* ---- threading: contiguous output-column ranges, as ExecuteRanges hands out ---- */

/* onnx_light_cpu/impl/execution.h:72-94 with kExecutionGrainSize = 2^15 */
int64_t mnbo_execution_block_count(int64_t total, double cost_per_item, int64_t threads) {
  if (total <= 0) return 0;
  if (threads <= 1) return 1;
  if (!(cost_per_item > 0.0)) cost_per_item = 1.0;
  const double work = (double)total * cost_per_item;
  const double grain = 32768.0;
  if (work < grain) return 1;
  int64_t useful = (int64_t)(work / grain);
  if (useful < 1) useful = 1;
  int64_t blocks = threads < useful ? threads : useful;
  return blocks < total ? blocks : total;
}

typedef struct {
  int64_t M, K, N, bs;
  const float *A;
  const uint8_t *B;
  const float *scales;
  const uint8_t *zp;
  void *out;
  int64_t n_begin, n_end;
  int mode;
} job_t;

enum { MODE_F64 = 0, MODE_REF_F32 = 1, MODE_FUSED_F32 = 2, MODE_ABS_F64 = 3 };

static void run_f64(const job_t *j, int absolute) {
  const int64_t nb = num_blocks(j->K, j->bs);
  const int64_t row_bytes = nb * j->bs / 2;
  double *Y = (double *)j->out;
  double *w = (double *)malloc(sizeof(double) * (size_t)j->K);
  for (int64_t n = j->n_begin; n < j->n_end; ++n) {
    const uint8_t *row = j->B + n * row_bytes;
    for (int64_t k = 0; k < j->K; ++k) {
      const int64_t b = k / j->bs;
      const int d = mnbo_nibble(row, k) - zero_point_of(j->zp, n, nb, b);
      w[k] = (double)d * (double)j->scales[n * nb + b]; /* exact in fp64 */
      if (absolute && w[k] < 0) w[k] = -w[k];
    }
    for (int64_t m = 0; m < j->M; ++m) {
      const float *a = j->A + m * j->K;
      double acc = 0.0;
      for (int64_t k = 0; k < j->K; ++k) {
        const double av = absolute ? (a[k] < 0 ? -(double)a[k] : (double)a[k]) : (double)a[k];
        acc += av * w[k];
      }
      Y[m * j->N + n] = acc;
    }
  }
  free(w);
}

static void run_ref_f32(const job_t *j) {
  const int64_t nb = num_blocks(j->K, j->bs);
  const int64_t row_bytes = nb * j->bs / 2;
  float *Y = (float *)j->out;
  float *w = (float *)malloc(sizeof(float) * (size_t)j->K);
  for (int64_t n = j->n_begin; n < j->n_end; ++n) {
    const uint8_t *row = j->B + n * row_bytes;
    for (int64_t k = 0; k < j->K; ++k) {
      const int64_t b = k / j->bs;
      w[k] = (float)(mnbo_nibble(row, k) - zero_point_of(j->zp, n, nb, b)) *
             j->scales[n * nb + b];
    }
    for (int64_t m = 0; m < j->M; ++m) {
      const float *a = j->A + m * j->K;
      float acc = 0.0f;
      for (int64_t k = 0; k < j->K; ++k) {
        const float p = a[k] * w[k];
        acc = acc + p;
      }
      Y[m * j->N + n] = acc;
    }
  }
  free(w);
}

/* int4_gemv of the qwen3 roadmap (:208-218): per block, sum a*(q - zp) in fp32,
 * then scale once and add to the fp32 row accumulator. The row's nibbles are
 * unpacked once into small integers and reused for every activation row. */
static void run_fused_f32(const job_t *j) {
  const int64_t nb = num_blocks(j->K, j->bs);
  const int64_t bs = j->bs;
  const int64_t row_bytes = nb * bs / 2;
  float *Y = (float *)j->out;
  float *d = (float *)malloc(sizeof(float) * (size_t)(nb * bs));
  for (int64_t n = j->n_begin; n < j->n_end; ++n) {
    const uint8_t *row = j->B + n * row_bytes;
    for (int64_t b = 0; b < nb; ++b) {
      const float z = (float)zero_point_of(j->zp, n, nb, b);
      const uint8_t *blk = row + b * (bs / 2);
      float *db = d + b * bs;
      for (int64_t i = 0; i < bs / 2; ++i) {
        db[2 * i] = (float)(blk[i] & 0x0F) - z;
        db[2 * i + 1] = (float)(blk[i] >> 4) - z;
      }
    }
    const float *s = j->scales + n * nb;
    for (int64_t m = 0; m < j->M; ++m) {
      const float *a = j->A + m * j->K;
      float acc = 0.0f;
      for (int64_t b = 0; b < nb; ++b) {
        const int64_t k0 = b * bs;
        const int64_t k1 = (k0 + bs < j->K) ? k0 + bs : j->K;
        float part = 0.0f;
        for (int64_t k = k0; k < k1; ++k) part += a[k] * d[k];
        acc += part * s[b];
      }
      Y[m * j->N + n] = acc;
    }
  }
  free(d);
}

static void *job_main(void *arg) {
  const job_t *j = (const job_t *)arg;
  switch (j->mode) {
  case MODE_F64: run_f64(j, 0); break;
  case MODE_ABS_F64: run_f64(j, 1); break;
  case MODE_REF_F32: run_ref_f32(j); break;
  default: run_fused_f32(j); break;
  }
  return NULL;
}

static void run_partitioned(int mode, int64_t M, int64_t K, int64_t N, int64_t bs,
                            const float *A, const uint8_t *B, const float *scales,
                            const uint8_t *zp, void *out, int threads) {
  /* cost per output column in work units of 64 FMAs (gemm_common.h:129) */
  const double cost = (double)M * (double)K / 64.0;
  int64_t blocks = mnbo_execution_block_count(N, cost, threads < 1 ? 1 : threads);
  if (blocks < 1) return;
  job_t *jobs = (job_t *)calloc((size_t)blocks, sizeof(job_t));
  pthread_t *tids = (pthread_t *)calloc((size_t)blocks, sizeof(pthread_t));
  /* execution.h:160-163: block = ceil(total / blocks), then blocks = ceil(total / block) */
  const int64_t block = (N + blocks - 1) / blocks;
  blocks = (N + block - 1) / block;
  for (int64_t t = 0; t < blocks; ++t) {
    job_t *j = &jobs[t];
    j->M = M; j->K = K; j->N = N; j->bs = bs;
    j->A = A; j->B = B; j->scales = scales; j->zp = zp; j->out = out; j->mode = mode;
    j->n_begin = t * block;
    j->n_end = (t + 1) * block < N ? (t + 1) * block : N;
  }
  for (int64_t t = 1; t < blocks; ++t) pthread_create(&tids[t], NULL, job_main, &jobs[t]);
  job_main(&jobs[0]);
  for (int64_t t = 1; t < blocks; ++t) pthread_join(tids[t], NULL);
  free(tids);
  free(jobs);
}

void mnbo_matmul_nbits_f64(int64_t M, int64_t K, int64_t N, int64_t bs, const float *A,
                           const uint8_t *B, const float *scales, const uint8_t *zp,
                           double *Y64, int threads) {
  run_partitioned(MODE_F64, M, K, N, bs, A, B, scales, zp, Y64, threads);
}

void mnbo_abs_dot_f64(int64_t M, int64_t K, int64_t N, int64_t bs, const float *A,
                      const uint8_t *B, const float *scales, const uint8_t *zp, double *out,
                      int threads) {
  run_partitioned(MODE_ABS_F64, M, K, N, bs, A, B, scales, zp, out, threads);
}

void mnbo_matmul_nbits_ref_f32(int64_t M, int64_t K, int64_t N, int64_t bs, const float *A,
                               const uint8_t *B, const float *scales, const uint8_t *zp,
                               float *Y, int threads) {
  run_partitioned(MODE_REF_F32, M, K, N, bs, A, B, scales, zp, Y, threads);
}

void mnbo_matmul_nbits_fused_f32(int64_t M, int64_t K, int64_t N, int64_t bs, const float *A,
                                 const uint8_t *B, const float *scales, const uint8_t *zp,
                                 float *Y, int threads) {
  run_partitioned(MODE_FUSED_F32, M, K, N, bs, A, B, scales, zp, Y, threads);
}

/* ---- fp16 conversion, half_conversion.h:42-78 restated ---- */

uint16_t mnbo_f32_to_f16_bits(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t biased = (bits >> 23) & 0xFFu;
  const uint32_t mant = bits & 0x7FFFFFu;
  if (biased == 0xFFu) return (uint16_t)(sign | (mant ? 0x7E00u : 0x7C00u));
  const int32_t e = (int32_t)biased - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t full = mant | 0x800000u;
    const int sh = 14 - e;
    uint32_t hm = full >> sh;
    const uint32_t rem = full & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return (uint16_t)(sign | hm);
  }
  const uint32_t hm = mant >> 13;
  const uint32_t rem = mant & 0x1FFFu;
  uint32_t h = sign | ((uint32_t)e << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++h; /* carry may roll into inf */
  return (uint16_t)h;
}

float mnbo_f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int32_t ee = 113; /* 127 - 15 + 1 */
      while (!(m & 0x400u)) { m <<= 1; --ee; }
      m &= 0x3FFu;
      bits = sign | ((uint32_t)ee << 23) | (m << 13);
    }
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

void mnbo_f32_to_f16_array(const float *in, uint16_t *out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = mnbo_f32_to_f16_bits(in[i]);
}

void mnbo_f16_to_f32_array(const uint16_t *in, float *out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = mnbo_f16_bits_to_f32(in[i]);
}
