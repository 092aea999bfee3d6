// Prefill GEMM for MatMulNBits on CDNA4 fp16 MFMA (the roadmap's `int4_gemm`,
// docs/next_steps/2026/2026_08_qwen3_inference.rst:223-225).
//
// Y[M, N] = A[M, K] * W[N, K]^T with W dequantized from 4-bit blocks.
//
// Tiling. A workgroup of 256 threads (4 wavefronts, 2 x 2) owns a 128 x 128
// output tile and walks K in steps of 32. Per step:
//   - A (fp32 in HBM) is loaded with 128-bit loads, rounded to fp16 (round to
//     nearest even, as onnx_light_cpu/impl/math/half_conversion.h:42-78) and
//     stored to LDS as [128][32] fp16;
//   - B's packed nibbles for the tile's 128 rows are loaded (8 bytes per
//     thread), dequantized in fp32 as (q - zp) * scale, rounded once to fp16
//     and stored to LDS as [128][32];
//   - each wavefront runs 4 x 4 v_mfma_f32_16x16x32_f16 on its 64 x 64
//     sub-tile, accumulating in fp32.
// LDS rows are padded to 40 halves (80 bytes): the 16 lanes that read one
// 16-byte k-group of 16 consecutive rows then touch 16 disjoint 4-bank groups.
#include "mnb_kernels.h"

namespace mnb {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 32;
constexpr int kLdsStride = kBK + 8;  // halves

template <bool HAS_ZP>
__global__ __launch_bounds__(256) void GemmKernel(const float *__restrict__ A,
                                                  const uint8_t *__restrict__ B,
                                                  const float *__restrict__ S,
                                                  const uint8_t *__restrict__ Z,
                                                  float *__restrict__ Y, int M, int K, int N,
                                                  int nb, int log2_bs, int row_bytes,
                                                  int zp_row_bytes) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kBN * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // B loader assignment: row tid/2, 16 nibbles at k offset 16*(tid&1).
  const int b_row = tid >> 1;
  const int b_half = tid & 1;
  const int b_gn = n0 + b_row;
  const bool b_valid = b_gn < N;
  const uint8_t *b_ptr = B + static_cast<size_t>(b_valid ? b_gn : 0) * row_bytes;
  const float *s_ptr = S + static_cast<size_t>(b_valid ? b_gn : 0) * nb;
  const uint8_t *z_ptr = HAS_ZP ? Z + static_cast<size_t>(b_valid ? b_gn : 0) * zp_row_bytes
                                : nullptr;

  for (int k0 = 0; k0 < K; k0 += kBK) {
    // ---- A: 128 x 32 fp32 -> fp16, four float4 per thread ----
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx >> 3;
      const int c4 = idx & 7;
      const int gm = m0 + row;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (gm < M)
        v = *reinterpret_cast<const float4 *>(A + static_cast<size_t>(gm) * K + k0 + 4 * c4);
      half4 h = {static_cast<_Float16>(v.x), static_cast<_Float16>(v.y),
                 static_cast<_Float16>(v.z), static_cast<_Float16>(v.w)};
      *reinterpret_cast<half4 *>(&As[row * kLdsStride + 4 * c4]) = h;
    }
    // ---- B: 16 nibbles per thread -> fp16 ----
    {
      const int kk = k0 + 16 * b_half;
      half8 h0, h1;
      if (b_valid) {
        const uint2 raw = *reinterpret_cast<const uint2 *>(b_ptr + (kk >> 1));
        const int blk = kk >> log2_bs;
        const float sc = s_ptr[blk];
        const float zf =
            HAS_ZP ? static_cast<float>((z_ptr[blk >> 1] >> ((blk & 1) * 4)) & 0xF) : 8.f;
        const uint32_t words[2] = {raw.x, raw.y};
        _Float16 w[16];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t byte = (words[t] >> (8 * b)) & 0xFFu;
            w[8 * t + 2 * b] = static_cast<_Float16>((static_cast<float>(byte & 0xFu) - zf) * sc);
            w[8 * t + 2 * b + 1] = static_cast<_Float16>((static_cast<float>(byte >> 4) - zf) * sc);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h0[e] = w[e];
          h1[e] = w[8 + e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h0[e] = static_cast<_Float16>(0.f);
          h1[e] = static_cast<_Float16>(0.f);
        }
      }
      *reinterpret_cast<half8 *>(&Bs[b_row * kLdsStride + 16 * b_half]) = h0;
      *reinterpret_cast<half8 *>(&Bs[b_row * kLdsStride + 16 * b_half + 8]) = h1;
    }
    __syncthreads();

    half8 af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *reinterpret_cast<const half8 *>(
          &As[(wm * 64 + i * 16 + (lane & 15)) * kLdsStride + 8 * (lane >> 4)]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bf[j] = *reinterpret_cast<const half8 *>(
          &Bs[(wn * 64 + j * 16 + (lane & 15)) * kLdsStride + 8 * (lane >> 4)]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  // Output: lane holds column (lane & 15), rows 4*(lane >> 4) + v of each 16 x 16 tile.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int gm = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + v;
        if (gm < M && gn < N) Y[static_cast<size_t>(gm) * N + gn] = acc[i][j][v];
      }
    }
  }
}

} // namespace

bool GemmSupports(const WeightView &w, int64_t M) {
  return M >= 1 && M <= (int64_t{1} << 22) && (w.K % 32) == 0 && w.block_size >= 16 &&
         w.K <= (int64_t{1} << 30) && w.N <= (int64_t{1} << 30) &&
         w.row_bytes <= (int64_t{1} << 30) && (w.row_bytes % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(w.B) % 8) == 0;
}

hipError_t LaunchGemm(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((w.N + kBN - 1) / kBN),
                  static_cast<unsigned>((M + kBM - 1) / kBM));
  if (w.zp) {
    hipLaunchKernelGGL(GemmKernel<true>, grid, dim3(256), 0, s, A, w.B, w.scales, w.zp, Y,
                       static_cast<int>(M), static_cast<int>(w.K), static_cast<int>(w.N),
                       static_cast<int>(w.nb), w.log2_bs, static_cast<int>(w.row_bytes),
                       static_cast<int>(w.zp_row_bytes));
  } else {
    hipLaunchKernelGGL(GemmKernel<false>, grid, dim3(256), 0, s, A, w.B, w.scales, w.zp, Y,
                       static_cast<int>(M), static_cast<int>(w.K), static_cast<int>(w.N),
                       static_cast<int>(w.nb), w.log2_bs, static_cast<int>(w.row_bytes),
                       static_cast<int>(w.zp_row_bytes));
  }
  return hipGetLastError();
}

} // namespace mnb
