// Decode GEMV for MatMulNBits, M <= 16, and the generic fallback kernel.
//
// Role in the reference: the roadmap's `int4_gemv` / `int4_small_m`
// (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-221): fp32
// accumulation, weights never expanded, each weight byte streamed once.
//
// Mapping. One wavefront owns R consecutive output columns n (weight rows).
// Lane l walks the 16-byte chunks c = l, l+64, ... of those rows: a wave issues
// 1 KiB coalesced 128-bit loads per row and instruction. A chunk holds 32
// nibbles k = 32c .. 32c+31; with block_size >= 32 it lies in one quantization
// block, so its scale and zero point are two scalars per row held in
// registers. Per chunk and activation row m the lane forms
//   dot  = sum_j a[m, 32c+j] * q[j]          (q in 0..15, exact in fp32)
//   asum = sum_j a[m, 32c+j]
//   acc += scale * (dot - zp * asum)
// which equals sum_j a * (q - zp) * scale up to fp32 rounding, with one
// conversion per nibble and no per-nibble zero-point subtraction. The A chunk
// and its sum are loaded once and reused for all R rows. A 64-lane butterfly
// reduces each accumulator at the end.
#include "mnb_decode_common.h"

namespace mnb {
namespace {

__device__ __forceinline__ float WaveSum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ int ZeroPoint(const uint8_t *zp_row, int blk) {
  return (zp_row[blk >> 1] >> ((blk & 1) * 4)) & 0xF;
}

// Unpacks the 32 nibbles of a 16-byte chunk into floats in k order.
__device__ __forceinline__ void UnpackChunk(const uint4 &w4, float *q) {
  const uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = words[t] & 0x0F0F0F0Fu;         // k = 8t + 0, 2, 4, 6
    const uint32_t hi = (words[t] >> 4) & 0x0F0F0F0Fu;  // k = 8t + 1, 3, 5, 7
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      q[8 * t + 2 * b] = static_cast<float>((lo >> (8 * b)) & 0xFFu);
      q[8 * t + 2 * b + 1] = static_cast<float>((hi >> (8 * b)) & 0xFFu);
    }
  }
}

template <int MT, int R, bool HAS_ZP>
__global__ __launch_bounds__(256) void GemvKernel(const float *__restrict__ A,
                                                  const uint8_t *__restrict__ B,
                                                  const float *__restrict__ S,
                                                  const uint8_t *__restrict__ Z,
                                                  float *__restrict__ Y, int M, int K, int N,
                                                  int nb, int chunk_shift, int row_bytes,
                                                  int zp_row_bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int n0 = wave * R;
  if (n0 >= N) return;  // uniform per wave
  const int nchunks = K >> 5;

  int rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = (n0 + r < N) ? n0 + r : N - 1;

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  for (int c = lane; c < nchunks; c += 64) {
    uint4 w4[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      w4[r] = *reinterpret_cast<const uint4 *>(B + static_cast<size_t>(rows[r]) * row_bytes +
                                               static_cast<size_t>(c) * 16);
    const int blk = c >> chunk_shift;
    float s[R], z[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      s[r] = S[static_cast<size_t>(rows[r]) * nb + blk];
      z[r] = HAS_ZP ? static_cast<float>(
                          ZeroPoint(Z + static_cast<size_t>(rows[r]) * zp_row_bytes, blk))
                    : 8.f;
    }
    float q[R][32];
#pragma unroll
    for (int r = 0; r < R; ++r) UnpackChunk(w4[r], q[r]);

#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) {
        const float4 *ap =
            reinterpret_cast<const float4 *>(A + static_cast<size_t>(m) * K + c * 32);
        float a[32];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float4 t = ap[v];
          a[4 * v] = t.x;
          a[4 * v + 1] = t.y;
          a[4 * v + 2] = t.z;
          a[4 * v + 3] = t.w;
        }
        float asum0 = 0.f, asum1 = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j += 2) {
          asum0 += a[j];
          asum1 += a[j + 1];
        }
        const float asum = asum0 + asum1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d0 = 0.f, d1 = 0.f;
#pragma unroll
          for (int j = 0; j < 32; j += 2) {
            d0 = fmaf(a[j], q[r][j], d0);
            d1 = fmaf(a[j + 1], q[r][j + 1], d1);
          }
          const float dot = d0 + d1;
          acc[r][m] = fmaf(s[r], fmaf(-z[r], asum, dot), acc[r][m]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = WaveSum(acc[r][m]);

  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r < N) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m < M) {
            float y = acc[r][m];
            // A non-finite activation: the reference's +-inf / NaN (the
            // zero point applied through asum gives inf - inf = NaN).
            if (!__builtin_isfinite(y)) {
              const size_t n = static_cast<size_t>(n0 + r);
              y = dec::ReferenceRowDotPlain(A + static_cast<size_t>(m) * K, K, chunk_shift + 5,
                                            B + n * row_bytes, S + n * nb,
                                            HAS_ZP ? Z + n * zp_row_bytes : nullptr);
            }
            Y[static_cast<size_t>(m) * N + n0 + r] = y;
          }
        }
      }
    }
  }
}

// One wavefront per weight row; lanes stride over k one nibble at a time. Any
// K (tails inside the last block are skipped), any even block_size, any M.
__global__ __launch_bounds__(256) void GenericKernel(const float *__restrict__ A,
                                                     const uint8_t *__restrict__ B,
                                                     const float *__restrict__ S,
                                                     const uint8_t *__restrict__ Z,
                                                     float *__restrict__ Y, int64_t M, int64_t K,
                                                     int64_t N, int64_t nb, int64_t bs,
                                                     int64_t row_bytes, int64_t zp_row_bytes) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint8_t *row = B + n * row_bytes;
  for (int64_t m = 0; m < M; ++m) {
    const float *a = A + m * K;
    float acc = 0.f;
    for (int64_t k = lane; k < K; k += 64) {
      const int64_t blk = k / bs;
      const int q = (row[k >> 1] >> ((k & 1) * 4)) & 0xF;
      const int z = Z ? ZeroPoint(Z + n * zp_row_bytes, static_cast<int>(blk)) : 8;
      acc = fmaf(a[k], static_cast<float>(q - z) * S[n * nb + blk], acc);
    }
    acc = WaveSum(acc);
    if (lane == 0) Y[m * N + n] = acc;
  }
}

// GenericKernel over a compact plan's fragment-ordered copy: row n = 64 g +
// 16 j + c is word j of lane (q, c) in the 1 KiB record of (g, 32-k step s),
// k = 32 s + 8 q + i its nibble i; its block scale and zero point sit at
// [g][b][c][j] of Sd and byte j of Zd[g][b][c]. Same arithmetic and order
// as GenericKernel.
__global__ __launch_bounds__(256) void GenericFragKernel(const float *__restrict__ A,
                                                         const uint32_t *__restrict__ Bp,
                                                         const float *__restrict__ Sd,
                                                         const uint32_t *__restrict__ Zd,
                                                         float *__restrict__ Y, int64_t M,
                                                         int64_t K, int64_t N, int64_t nb,
                                                         int log2_bs) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  const int64_t g = n >> 6, T = K >> 5;
  const int j = static_cast<int>((n >> 4) & 3), c = static_cast<int>(n & 15);
  for (int64_t m = 0; m < M; ++m) {
    const float *a = A + m * K;
    float acc = 0.f;
    for (int64_t k = lane; k < K; k += 64) {
      const int64_t s = k >> 5, q = (k >> 3) & 3, b = k >> log2_bs;
      const uint32_t word = Bp[((g * T + s) * 64 + q * 16 + c) * 4 + j];
      const int qv = static_cast<int>((word >> (4 * (k & 7))) & 0xFu);
      const int z = Zd ? static_cast<int>((Zd[(g * nb + b) * 16 + c] >> (8 * j)) & 0xFFu) : 8;
      acc = fmaf(a[k], static_cast<float>(qv - z) * Sd[((g * nb + b) * 16 + c) * 4 + j], acc);
    }
    acc = WaveSum(acc);
    if (lane == 0) Y[m * N + n] = acc;
  }
}

template <int MT, int R, bool HAS_ZP>
hipError_t LaunchGemvT(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s) {
  const int64_t waves = (w.N + R - 1) / R;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((GemvKernel<MT, R, HAS_ZP>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                     0, s, A, w.B, w.scales, w.zp, Y, static_cast<int>(M),
                     static_cast<int>(w.K), static_cast<int>(w.N), static_cast<int>(w.nb),
                     w.log2_bs - 5, static_cast<int>(w.row_bytes),
                     static_cast<int>(w.zp_row_bytes));
  return hipGetLastError();
}

template <bool HAS_ZP>
hipError_t LaunchGemvZ(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s) {
  if (M <= 1) return LaunchGemvT<1, 4, HAS_ZP>(w, M, A, Y, s);
  if (M <= 2) return LaunchGemvT<2, 4, HAS_ZP>(w, M, A, Y, s);
  if (M <= 4) return LaunchGemvT<4, 4, HAS_ZP>(w, M, A, Y, s);
  if (M <= 8) return LaunchGemvT<8, 2, HAS_ZP>(w, M, A, Y, s);
  return LaunchGemvT<16, 2, HAS_ZP>(w, M, A, Y, s);
}

} // namespace

bool GemvSupports(const WeightView &w, int64_t M) {
  return w.B != nullptr && M >= 1 && M <= 16 && (w.K % 32) == 0 && w.block_size >= 32 &&
         w.K <= (int64_t{1} << 30) && w.N <= (int64_t{1} << 30) &&
         w.row_bytes <= (int64_t{1} << 30) && (w.row_bytes % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(w.B) % 16) == 0;
}

hipError_t LaunchGemv(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s) {
  return w.zp ? LaunchGemvZ<true>(w, M, A, Y, s) : LaunchGemvZ<false>(w, M, A, Y, s);
}

hipError_t LaunchGeneric(const WeightView &w, int64_t M, const float *A, float *Y,
                         hipStream_t s) {
  const int64_t blocks = (w.N + 3) / 4;
  if (w.B == nullptr) {
    // a compact plan: the same over the fragment-ordered copy
    if (w.Bp == nullptr || w.Sd == nullptr || (w.has_zp && w.Zd == nullptr))
      return hipErrorInvalidValue;
    hipLaunchKernelGGL(GenericFragKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, A,
                       reinterpret_cast<const uint32_t *>(w.Bp), w.Sd, w.has_zp ? w.Zd : nullptr,
                       Y, M, w.K, w.N, w.nb, w.log2_bs);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(GenericKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, A, w.B,
                     w.scales, w.zp, Y, M, w.K, w.N, w.nb, static_cast<int64_t>(w.block_size),
                     w.row_bytes, w.zp_row_bytes);
  return hipGetLastError();
}

} // namespace mnb
