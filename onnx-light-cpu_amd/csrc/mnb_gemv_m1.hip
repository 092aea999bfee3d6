// Decode GEMV for a single activation row (M = 1): the HBM-bound hot path.
//
// Role in the reference: the roadmap's `int4_gemv`
// (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-218): fp32
// accumulation, weights never expanded, each weight byte streamed once.
//
// Mapping. The grid is persistent (a few workgroups per CU). Each wavefront
// takes batches of R consecutive weight rows, batch b = g, g + TW, ... (g its
// global index, TW the number of wavefronts), so at any moment the chip
// streams a contiguous band of rows. Lane l takes the 16-byte chunks
// c = l + 64 i (i < CPL) of each row: every load instruction of the wave reads
// 1 KiB of one row, coalesced. Loads are buffer loads whose row offset is a
// wave-uniform SGPR, so no per-row vector address arithmetic is spent. The
// next batch's chunks, scales and zero points are loaded while the current
// batch is computed. A chunk holds 32 nibbles k = 32c .. 32c+31, all in one
// quantization block (block_size >= 32).
//
// Activations. A is staged once per workgroup in LDS (8 float4 per chunk, the
// float4 index XOR-swizzled by (c & 7) so that the lanes of a half-wave spread
// over the banks), with the per-chunk sums asum = sum_j a_j. All staging loads
// are issued before the first LDS store (one memory round trip). The R rows
// of a batch share each chunk's LDS read.
//
// Arithmetic. v_fma_mix_f32 multiplies an fp32 activation by an fp16 operand
// taken straight from one half of a register. Masking a packed word with
// 0x000F000F leaves two nibbles q in the two halves, i.e. the fp16 subnormals
// q * 2^-24, exact. So per chunk the lane forms
//   dot  = sum_j a_j * q_j * 2^-24          (products exact, fp32 sums)
//   y   += scale * (dot * 2^24 - zp * asum)
// at seven bit operations per eight nibbles plus one FMA per nibble, with no
// per-nibble conversion or zero-point subtraction. This relies on fp16
// subnormal inputs being kept (the gfx950 HIP default FP16 denormal mode);
// the parity tests would see every product vanish otherwise.
//
// Reduction per row: 4 DPP steps give every lane its 16-lane row sum, 4
// readlanes add the rows in a fixed order; lane r stores row r of the batch.
#include "mnb_kernels.h"

namespace mnb {
namespace m1 {

// acc += a * f16(lo half of h), accumulator tied to the destination.
__device__ __forceinline__ void MixLo(float &acc, float a, uint32_t h) {
  __asm__("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(a), "v"(h));
}

// acc += a * f16(hi half of h)
__device__ __forceinline__ void MixHi(float &acc, float a, uint32_t h) {
  __asm__("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
          : "+v"(acc)
          : "v"(a), "v"(h));
}

// d0/d1 += sum_j a[j] * q_j * 2^-24 over the 32 nibbles of one chunk, k order.
__device__ __forceinline__ void DotChunk(const float *a, const uint4 &w4, float &d0, float &d1) {
  const uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t w = words[t];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t h = (w >> (4 * i)) & 0x000F000Fu;  // nibbles i (lo half) and i+4 (hi half)
      MixLo(d0, a[8 * t + i], h);
      MixHi(d1, a[8 * t + i + 4], h);
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float DppAdd(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false);
  return v + __int_as_float(moved);
}

// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float WaveTotal(float v) {
  v = DppAdd<0xB1>(v);   // quad_perm [1,0,3,2]
  v = DppAdd<0x4E>(v);   // quad_perm [2,3,0,1]
  v = DppAdd<0x141>(v);  // row_half_mirror
  v = DppAdd<0x140>(v);  // row_mirror: every lane holds its 16-lane row sum
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return (r0 + r1) + (r2 + r3);
}

// Copies A[0 .. 32*nchunks) into LDS as swizzled float4 chunks and writes the
// per-chunk sums. A 256-thread workgroup moves 256 float4 per pass; CPL * 2
// passes cover nchunks <= 64 * CPL chunks. Loads are all issued before the
// first store, so staging costs one memory round trip.
template <int CPL>
__device__ __forceinline__ void StageA(const float *__restrict__ A, float4 *lds4,
                                       float *asum_lds, int nchunks) {
  constexpr int kPasses = CPL * 2;  // 64*CPL chunks * 8 float4 / 256 threads
  const float4 *src = reinterpret_cast<const float4 *>(A);
  const int total = nchunks * 8;
  float4 t[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int f = threadIdx.x + 256 * p;
    t[p] = f < total ? src[f] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int f = threadIdx.x + 256 * p;
    const int c = f >> 3, v = f & 7;
    if (f < total) lds4[c * 8 + (v ^ (c & 7))] = t[p];
    float s = (t[p].x + t[p].y) + (t[p].z + t[p].w);
    s = DppAdd<0xB1>(s);   // quad_perm [1,0,3,2]
    s = DppAdd<0x4E>(s);   // quad_perm [2,3,0,1]
    s = DppAdd<0x141>(s);  // row_half_mirror: every lane holds its 8-lane sum
    if (v == 0 && f < total) asum_lds[c] = s;
  }
  __syncthreads();
}

// R rows x CPL chunks of weights with their scales and zero-point bytes.
template <int CPL, int R, bool FULL, bool HAS_ZP>
struct Batch {
  uint4 w[R][CPL];
  float s[R][CPL];
  uint32_t z[R][CPL];
};

struct Rsrc {
  __amdgpu_buffer_rsrc_t b, s, z;
};

// Buffer loads: the row offset is wave-uniform (SGPR), the lane offset is a
// per-lane constant, so no per-row vector address arithmetic is needed.
template <int CPL, int R, bool FULL, bool HAS_ZP>
__device__ __forceinline__ void LoadBatch(Batch<CPL, R, FULL, HAS_ZP> &bt, const Rsrc &rs,
                                          int row0, int N, int lane, int nchunks, int nb,
                                          int chunk_shift, int row_bytes, int zp_row_bytes) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = __builtin_amdgcn_readfirstlane(min(row0 + r, N - 1));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      if (FULL || c < nchunks) {
        const int blk = c >> chunk_shift;
        bt.w[r][i] =
            __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.b, c * 16, row * row_bytes, 0));
        bt.s[r][i] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rs.s, blk * 4, row * nb * 4, 0));
        if (HAS_ZP)
          bt.z[r][i] = __builtin_amdgcn_raw_buffer_load_b8(rs.z, blk >> 1, row * zp_row_bytes, 0);
      }
    }
  }
}

template <int CPL, int R, bool FULL, bool HAS_ZP>
__global__ __launch_bounds__(256) void GemvM1Kernel(const float *__restrict__ A,
                                                    const uint8_t *__restrict__ B,
                                                    const float *__restrict__ S,
                                                    const uint8_t *__restrict__ Z,
                                                    float *__restrict__ Y, int K, int N, int nb,
                                                    int chunk_shift, int row_bytes,
                                                    int zp_row_bytes) {
  extern __shared__ float4 lds4[];
  const int nchunks = K >> 5;
  const int lane = threadIdx.x & 63;
  const int TW = gridDim.x * (blockDim.x >> 6);
  const int nbatches = (N + R - 1) / R;
  int bi = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);

  Rsrc rs;
  rs.b = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(B), 0, 0x7FFFFFFF, 0x00020000);
  rs.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(S), 0, 0x7FFFFFFF, 0x00020000);
  rs.z = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(HAS_ZP ? Z : B), 0, 0x7FFFFFFF,
                                           0x00020000);

  // 1. the first batch goes in flight before anything else
  Batch<CPL, R, FULL, HAS_ZP> cur;
  if (bi < nbatches)
    LoadBatch(cur, rs, bi * R, N, lane, nchunks, nb, chunk_shift, row_bytes, zp_row_bytes);

  // 2. stage A once per workgroup: all global loads first (one round trip),
  //    then swizzled LDS stores; the 8 float4 of a chunk sit in 8 consecutive
  //    lanes, so the chunk sum is an 8-lane DPP reduction.
  float *asum_lds = reinterpret_cast<float *>(lds4 + nchunks * 8);
  StageA<CPL>(A, lds4, asum_lds, nchunks);
  float asum[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    asum[i] = (FULL || c < nchunks) ? asum_lds[c] : 0.f;
  }

  // 3. batches bi, bi + TW, ...: prefetch the next batch, compute this one
  for (; bi < nbatches; bi += TW) {
    Batch<CPL, R, FULL, HAS_ZP> nxt;
    const int bn = bi + TW;
    if (bn < nbatches)
      LoadBatch(nxt, rs, bn * R, N, lane, nchunks, nb, chunk_shift, row_bytes, zp_row_bytes);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      if (FULL || c < nchunks) {
        float a[32];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float4 t = lds4[c * 8 + (v ^ (c & 7))];
          a[4 * v] = t.x;
          a[4 * v + 1] = t.y;
          a[4 * v + 2] = t.z;
          a[4 * v + 3] = t.w;
        }
        const int blk = c >> chunk_shift;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d0 = 0.f, d1 = 0.f;
          DotChunk(a, cur.w[r][i], d0, d1);
          const float zf =
              HAS_ZP ? static_cast<float>((cur.z[r][i] >> ((blk & 1) * 4)) & 0xFu) : 8.f;
          acc[r] = fmaf(cur.s[r][i], fmaf(d0 + d1, 16777216.f, -zf * asum[i]), acc[r]);
        }
      }
    }
    float mine = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float t = WaveTotal(acc[r]);
      mine = lane == r ? t : mine;
    }
    const int n = bi * R + lane;
    if (lane < R && n < N) Y[n] = mine;
    cur = nxt;
  }
}

template <int CPL, int R, bool FULL, bool HAS_ZP>
hipError_t LaunchT(const WeightView &w, const float *A, float *Y, hipStream_t s, int wgs) {
  const int nchunks = static_cast<int>(w.K / 32);
  const size_t lds = static_cast<size_t>(nchunks) * (8 * sizeof(float4) + sizeof(float));
  // Equalise batches per wavefront over the persistent grid.
  const int64_t nbatches = (w.N + R - 1) / R;
  const int64_t max_waves = static_cast<int64_t>(wgs) * 4;
  const int64_t per_wave = (nbatches + max_waves - 1) / max_waves;
  const int64_t waves = (nbatches + per_wave - 1) / per_wave;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((GemvM1Kernel<CPL, R, FULL, HAS_ZP>), dim3(static_cast<unsigned>(blocks)),
                     dim3(256), lds, s, A, w.B, w.scales, w.zp, Y, static_cast<int>(w.K),
                     static_cast<int>(w.N), static_cast<int>(w.nb), w.log2_bs - 5,
                     static_cast<int>(w.row_bytes), static_cast<int>(w.zp_row_bytes));
  return hipGetLastError();
}

template <int CPL, bool HAS_ZP>
hipError_t LaunchF(const WeightView &w, const float *A, float *Y, hipStream_t s, int wgs, int R) {
  const bool full = (w.K / 32) == 64 * CPL;
  if (R >= 4)
    return full ? LaunchT<CPL, 4, true, HAS_ZP>(w, A, Y, s, wgs)
                : LaunchT<CPL, 4, false, HAS_ZP>(w, A, Y, s, wgs);
  if (R == 2)
    return full ? LaunchT<CPL, 2, true, HAS_ZP>(w, A, Y, s, wgs)
                : LaunchT<CPL, 2, false, HAS_ZP>(w, A, Y, s, wgs);
  return full ? LaunchT<CPL, 1, true, HAS_ZP>(w, A, Y, s, wgs)
              : LaunchT<CPL, 1, false, HAS_ZP>(w, A, Y, s, wgs);
}

template <bool HAS_ZP>
hipError_t LaunchZ(const WeightView &w, const float *A, float *Y, hipStream_t s, int wgs, int R) {
  switch ((w.K / 32 + 63) / 64) {
  case 1: return LaunchF<1, HAS_ZP>(w, A, Y, s, wgs, R);
  case 2: return LaunchF<2, HAS_ZP>(w, A, Y, s, wgs, R);
  case 3: return LaunchF<3, HAS_ZP>(w, A, Y, s, wgs, R);
  case 4: return LaunchF<4, HAS_ZP>(w, A, Y, s, wgs, R);
  case 5: return LaunchF<5, HAS_ZP>(w, A, Y, s, wgs, R);
  case 6: return LaunchF<6, HAS_ZP>(w, A, Y, s, wgs, R);
  case 7: return LaunchF<7, HAS_ZP>(w, A, Y, s, wgs, R);
  default: return LaunchF<8, HAS_ZP>(w, A, Y, s, wgs, R);
  }
}

} // namespace m1

bool GemvM1Supports(const WeightView &w) {
  // Buffer offsets are 32-bit: every byte of B, scales and zero points must
  // be addressable below 2^31.
  return (w.K % 32) == 0 && w.K <= 16384 && w.block_size >= 32 && (w.row_bytes % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(w.B) % 16) == 0 &&
         w.row_bytes * w.N < (int64_t{1} << 31) && w.nb * 4 * w.N < (int64_t{1} << 31);
}

hipError_t LaunchGemvM1(const WeightView &w, const float *A, float *Y, hipStream_t s,
                        int workgroups, int rows_per_batch) {
  if (workgroups < 1) workgroups = 1;
  return w.zp ? m1::LaunchZ<true>(w, A, Y, s, workgroups, rows_per_batch)
              : m1::LaunchZ<false>(w, A, Y, s, workgroups, rows_per_batch);
}

} // namespace mnb
