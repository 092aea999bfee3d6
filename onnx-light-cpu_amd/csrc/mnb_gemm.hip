// Prefill GEMM for MatMulNBits on CDNA4 fp16 MFMA (the roadmap's `int4_gemm`,
// docs/next_steps/2026/2026_08_qwen3_inference.rst:223-225).
//
// Y[M, N] = A[M, K] * W[N, K]^T with W dequantized from 4-bit blocks; fp16
// operands, fp32 accumulation. Two kernels per call:
//
// 1. ConvertAKernel rounds A to fp16 once (round to nearest even, as
//    onnx_light_cpu/impl/math/half_conversion.h:42-78) into the caller's
//    workspace, already laid out as the LDS image of each 128 x 64 A tile
//    (tile-major, rows swizzled as below, rows past M zero). Rounding A once
//    instead of once per N tile removes that work from the GEMM and halves the
//    A bytes it streams.
//
// 2. GemmKernel: one workgroup (256 threads, 4 wavefronts as 2 x 2) owns a
//    BM x 128 output tile (BM = 128, 64 or 32, by M); each wavefront a
//    BM/2 x 64 sub-tile of v_mfma_f32_16x16x32_f16 tiles. K advances in
//    k-tiles of 64, optionally split over several workgroups (split-K; the
//    partial sums are added in split order by SplitReduceKernel). 80 KiB of
//    LDS per workgroup (BM = 128) lets two workgroups share a CU, so one
//    hides the other's barrier and dequantization stalls.
//    - A tiles go global -> LDS directly (global_load_lds_dwordx4 through
//      inline asm, no registers) into a 3-stage ring, two k-tiles ahead.
//    - B tiles: each thread loads 32 nibbles of one weight row into
//      registers four k-tiles ahead, dequantizes them one k-tile ahead into a
//      double-buffered LDS tile (DequantWord: masks and fp16 exponent
//      constants give 1024 + q and 64 + q exactly, a packed add of the
//      matching -(1024 + zp) or -(64 + zp) makes q - zp exact, one packed
//      multiply by the block's fp16 scale rounds the weight once).
//    - One barrier per k-tile; the loop is written so that the compiler's
//      own waits never drain the prefetch (see the pipeline comment below).
//    Inside every group of 8 k the LDS order is [0,4,1,5,2,6,3,7] for both A
//    and B (the order the masked words produce); the contraction is unchanged.
//    LDS rows are 64 fp16 = 8 units of 16 B; unit u of row r is stored at
//    r * 8 + (u ^ ((r >> 1) & 7)), so the 16 lanes of an MFMA fragment read
//    (16 consecutive rows, one unit) hit 16 distinct 16-byte bank groups.
//    Tile order is XCD-aware: workgroup b runs on XCD b % 8; when the M tiles
//    split evenly over the 8 XCDs, XCD x gets a contiguous band of M tiles with
//    all their N tiles, so each XCD's L2 holds one slab of A.
#include "mnb_kernels.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace mnb {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBM = 128;  // largest tile height; the workspace pads M to it
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kUnits = kBK / 8;             // 16-byte units per LDS row
constexpr int kBUnits = kBN * kUnits;       // units per B tile (16 KiB)
constexpr int kAStages = 3;
// Output tiles are BM x 128 with BM in {32, 64, 128}; A tiles BM x 64 fp16.
template <int BM>
constexpr int AUnits() { return BM * kUnits; }  // units per A tile
template <int BM>
constexpr size_t LdsBytes() { return (kAStages * AUnits<BM>() + 2 * kBUnits) * 16; }  // <= 80 KiB

__device__ __forceinline__ int Swz(int row, int unit) {
  return row * kUnits + (unit ^ ((row >> 1) & 7));
}

__device__ __forceinline__ uint32_t PackHalf2(float lo, float hi) {
  const half2v h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
  return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint32_t PkAddF16(uint32_t a, uint32_t b) {
  const half2v r = __builtin_bit_cast(half2v, a) + __builtin_bit_cast(half2v, b);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t PkMulF16(uint32_t a, uint32_t b) {
  const half2v r = __builtin_bit_cast(half2v, a) * __builtin_bit_cast(half2v, b);
  return __builtin_bit_cast(uint32_t, r);
}

// Per-thread constants of the dequantization, held in VGPRs (an empty asm
// hides their values from the compiler): VOP3 instructions on gfx9 take no
// literal, so with the masks as literals (w & m) | c costs two instructions
// instead of one v_and_or_b32.
struct DequantConsts {
  uint32_t lo, hi, e1024, e64;  // 0x000F000F, 0x00F000F0, fp16 pairs 1024.0, 64.0
};
__device__ __forceinline__ DequantConsts MakeDequantConsts() {
  DequantConsts c{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  __asm__ volatile("" : "+v"(c.lo), "+v"(c.hi), "+v"(c.e1024), "+v"(c.e64));
  return c;
}

// Per (row, k-tile) operands of DequantWord: -(1024 + zp) and -(64 + zp)
// (exact in fp16) and the block scale in fp16.
struct DequantRow {
  uint32_t neg_lo, neg_hi, s;
};
__device__ __forceinline__ DequantRow MakeDequantRow(float s, uint32_t zp) {
  const float z = static_cast<float>(zp);
  return DequantRow{PackHalf2(-(1024.f + z), -(1024.f + z)), PackHalf2(-(64.f + z), -(64.f + z)),
                    PackHalf2(s, s)};
}

// One packed word of 8 nibbles (k order) -> 8 fp16 weights in [0,4,1,5,2,6,3,7]
// order, with no per-nibble shift: in fp16, 1024.0 (0x6400) has an ulp of 1
// and 64.0 (0x5400) an ulp of 1/16, so (w & 0x000F000F) | 0x6400.. is the
// pair 1024 + q of nibbles 0 | 4 and (w & 0x00F000F0) | 0x5400.. the pair
// 64 + q of nibbles 1 | 5, both exact; the same of w >> 8 gives nibbles
// 2 | 6 and 3 | 7. Adding -(1024 + zp) or -(64 + zp) leaves q - zp exactly,
// and one multiply by the fp16 scale rounds the weight once. Per word: one
// shift, four v_and_or_b32, four packed adds and four packed multiplies.
__device__ __forceinline__ uint4 DequantWord(uint32_t w, const DequantRow &r,
                                             const DequantConsts &c) {
  const uint32_t w8 = w >> 8;
  const uint32_t h0 = (w & c.lo) | c.e1024;   // nibbles 0 | 4: 1024 + q
  const uint32_t h1 = (w & c.hi) | c.e64;     // nibbles 1 | 5: 64 + q
  const uint32_t h2 = (w8 & c.lo) | c.e1024;  // nibbles 2 | 6
  const uint32_t h3 = (w8 & c.hi) | c.e64;    // nibbles 3 | 7
  return make_uint4(PkMulF16(PkAddF16(h0, r.neg_lo), r.s), PkMulF16(PkAddF16(h1, r.neg_hi), r.s),
                    PkMulF16(PkAddF16(h2, r.neg_lo), r.s), PkMulF16(PkAddF16(h3, r.neg_hi), r.s));
}

// Largest value over the 256 threads of a workgroup (4 wavefronts); every
// thread gets it. `red` holds 4 floats of LDS.
__device__ __forceinline__ float BlockMax256(float v, float *red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  __syncthreads();  // red may still be read by an earlier reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float BlockSum256(float v, float *red) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row of A (rows past M, up to the tile padding, are written
// as zeros). The row is scaled by 2^f, f = RangeExponent(max_k |A[m][k]|, 14),
// and rounded to fp16 (round to nearest even, as FloatToFloat16Bits,
// onnx_light_cpu/impl/math/half_conversion.h:42-78): no finite input becomes
// inf, and only values below 2^-24 of the row's largest magnitude flush to
// zero. f goes to row_exp[m]; the GEMM's epilogue multiplies by 2^-f. Each
// 16-byte unit holds 8 consecutive k in [0,4,1,5,2,6,3,7] order and lands
// where GemmKernel's direct copy expects it.
// With gamma (RMSNorm folded in), the row is x * gamma * inv_rms with
// inv_rms = 1 / sqrt(mean_k x^2 + eps) reduced here as well.
// NV > 0: each thread keeps its NV units of the row in registers between the
// reduction and the conversion (K <= 2048 NV); NV = 0 reads the row twice.
template <int BM, int NV, bool RMS>
__global__ __launch_bounds__(256) void ConvertAKernel(const float *__restrict__ A,
                                                      uint4 *__restrict__ Ah,
                                                      int *__restrict__ row_exp, int M, int K,
                                                      const float *__restrict__ gamma,
                                                      float eps) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int units = K / 8;
  const int ktiles = K / kBK;
  const int mt = row / BM;
  const int r = row - mt * BM;
  uint4 *base = Ah + static_cast<size_t>(mt) * ktiles * AUnits<BM>();
  auto dst = [&](int u) -> uint4 & { return base[(u / kUnits) * AUnits<BM>() + Swz(r, u % kUnits)]; };
  if (row >= M) {
    for (int u = tid; u < units; u += 256) dst(u) = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) row_exp[row] = 0;
    return;
  }
  const float *src = A + static_cast<size_t>(row) * K;
  auto load = [&](int u, float4 &x, float4 &y, float &amax, float &ss) {
    x = reinterpret_cast<const float4 *>(src + 8 * u)[0];
    y = reinterpret_cast<const float4 *>(src + 8 * u)[1];
    if constexpr (RMS) {
      ss += ((x.x * x.x + x.y * x.y) + (x.z * x.z + x.w * x.w)) +
            ((y.x * y.x + y.y * y.y) + (y.z * y.z + y.w * y.w));
      const float4 g0 = reinterpret_cast<const float4 *>(gamma + 8 * u)[0];
      const float4 g1 = reinterpret_cast<const float4 *>(gamma + 8 * u)[1];
      x = make_float4(x.x * g0.x, x.y * g0.y, x.z * g0.z, x.w * g0.w);
      y = make_float4(y.x * g1.x, y.y * g1.y, y.z * g1.z, y.w * g1.w);
    }
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  };
  // x * mul, then * 2^f (exact): the value FloatToFloat16Bits rounds
  auto store = [&](int u, float4 x, float4 y, float mul, int f) {
    if constexpr (RMS) {
      x = make_float4(x.x * mul, x.y * mul, x.z * mul, x.w * mul);
      y = make_float4(y.x * mul, y.y * mul, y.z * mul, y.w * mul);
    }
    auto sc = [f](float v) { return __builtin_amdgcn_ldexpf(v, f); };
    dst(u) = make_uint4(PackHalf2(sc(x.x), sc(y.x)), PackHalf2(sc(x.y), sc(y.y)),
                        PackHalf2(sc(x.z), sc(y.z)), PackHalf2(sc(x.w), sc(y.w)));
  };
  float amax = 0.0f, ss = 0.0f;
  float4 kx[NV > 0 ? NV : 1], ky[NV > 0 ? NV : 1];
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = tid + 256 * i;
      if (u < units) load(u, kx[i], ky[i], amax, ss);
    }
  } else {
    for (int u = tid; u < units; u += 256) load(u, kx[0], ky[0], amax, ss);
  }
  amax = BlockMax256(amax, red);
  float mul = 1.0f;
  if constexpr (RMS) {
    mul = 1.0f / sqrtf(BlockSum256(ss, red) / static_cast<float>(K) + eps);
    amax *= mul;
  }
  const int f = RangeExponent(amax, kRowExpTarget);
  if (tid == 0) row_exp[row] = f;
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = tid + 256 * i;
      if (u < units) store(u, kx[i], ky[i], mul, f);
    }
  } else {
    for (int u = tid; u < units; u += 256) {
      float dummy_a = 0.0f, dummy_s = 0.0f;
      float4 x, y;
      load(u, x, y, dummy_a, dummy_s);
      store(u, x, y, mul, f);
    }
  }
}

// s_waitcnt vmcnt(N) with the other counters left free (gfx9 encoding: vmcnt
// in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void WaitVm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// One k-tile of B for this thread: 32 nibbles of one weight row (one
// quantization block, block_size >= 32), its scale, and the byte holding its
// zero point with the nibble's shift. The nibble is extracted only when the
// tile is dequantized: extracting it at load time would make the compiler wait
// for the load right after issuing it.
struct BRegs {
  uint4 b;
  float s;
  uint32_t z;
  uint32_t zshift;
};

template <int BM, bool HAS_ZP>
__global__ __launch_bounds__(256, 2) void GemmKernel(const uint4 *__restrict__ Ah,
                                                     const uint8_t *__restrict__ B,
                                                     const float *__restrict__ S,
                                                     const uint8_t *__restrict__ Z,
                                                     float *__restrict__ Y, int M, int K, int N,
                                                     int nb, int log2_bs, int row_bytes,
                                                     int zp_row_bytes, int kt_per_split,
                                                     float *__restrict__ partials,
                                                     float *__restrict__ H,
                                                     const int *__restrict__ row_exp,
                                                     const int *__restrict__ col_exp) {
  extern __shared__ uint4 lds[];
  constexpr int kAUnits = AUnits<BM>();
  uint4 *Astage = lds;                        // [kAStages][kAUnits]
  uint4 *Bbuf = lds + kAStages * kAUnits;     // [2][kBUnits]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // Workgroup b computes output tile b % tiles over the k-tiles of split
  // b / tiles. XCD-aware tile order.
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int split = static_cast<int>(blockIdx.x) / (tiles_m * tiles_n);
  int tm, tn;
  {
    const int b = static_cast<int>(blockIdx.x) - split * tiles_m * tiles_n;
    if (tiles_m % 8 == 0) {
      const int xcd = b & 7, local = b >> 3;
      const int band = tiles_m / 8;
      tm = xcd * band + local / tiles_n;
      tn = local % tiles_n;
    } else {
      tm = b / tiles_n;
      tn = b % tiles_n;
    }
  }
  const int m0 = tm * BM;
  const int n0 = tn * kBN;
  // This split's k-tiles: kt0 .. kt0 + ktiles - 1 (the host leaves no split empty).
  const int kt0 = split * kt_per_split;
  const int ktiles = min(kt_per_split, K / kBK - kt0);

  // B resources based at this tile's first weight row; rows past N read as
  // zero and their outputs are never stored.
  const int rows_b = min(kBN, N - n0);
  const auto rb_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(B + static_cast<size_t>(n0) * row_bytes), 0, rows_b * row_bytes,
      0x00020000);
  const auto rs_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(S + static_cast<size_t>(n0) * nb), 0, rows_b * nb * 4, 0x00020000);
  const auto rz_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(HAS_ZP ? Z + static_cast<size_t>(n0) * zp_row_bytes : B), 0,
      HAS_ZP ? rows_b * zp_row_bytes : 0, 0x00020000);

  // A: converted tile (tm, kt) is kAUnits contiguous units; instruction i of
  // wavefront w copies units i*256 + w*64 + lane to the same LDS offsets.
  const uint4 *a_tiles = Ah + (static_cast<size_t>(tm) * (K / kBK) + kt0) * kAUnits;
  // The copies go through CopyToLds16: with the builtin, the compiler waits
  // for every outstanding load (s_waitcnt vmcnt(0)) before the next LDS read,
  // which would stall each k-tile's MFMAs on the loads of tile kt + 2. The
  // WaitVm + barrier at the top of each iteration covers the copies.
  const uint32_t lds_a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(Astage)) +
                         __builtin_amdgcn_readfirstlane(wave) * 64 * 16;  // uniform
  const uint4 *a_src = a_tiles + wave * 64 + lane;
  auto issue_a = [&](int kt, int stage) {
    const uint4 *src = a_src + static_cast<size_t>(kt) * kAUnits;
#pragma unroll
    for (int i = 0; i < kAUnits / 256; ++i)
      CopyToLds16(src + i * 256, lds_a + (stage * kAUnits + i * 256) * 16);
  };

  // B: thread t -> weight row t >> 1, 32 nibbles at k offset 32 * (t & 1).
  // Buffer offsets are a per-thread constant (voffset) plus the k-tile's
  // uniform part (soffset), so the loads cost no address arithmetic. The
  // block of the thread's 32 nibbles is blk_u + blk_l: blk_u = (k-tile start)
  // >> log2_bs, plus the thread's half when blocks are 32 wide (then blk_u is
  // even, so the zero-point byte is blk_u >> 1 and the nibble blk_l).
  const int b_row = tid >> 1;
  const int b_half = tid & 1;
  const int blk_l = log2_bs == 5 ? b_half : 0;
  const int vo_b = b_row * row_bytes + 16 * b_half;
  const int vo_s = (b_row * nb + blk_l) * 4;
  const int vo_z = b_row * zp_row_bytes;
  auto load_b = [&](BRegs &r, int kt) {
    const int kg = kt0 + kt;
    const int blk_u = (kg * kBK) >> log2_bs;
    r.b = __builtin_bit_cast(uint4,
                             __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, vo_b, kg * 32, 0));
    r.s = __builtin_bit_cast(float,
                             __builtin_amdgcn_raw_buffer_load_b32(rs_rsrc, vo_s, blk_u * 4, 0));
    if (HAS_ZP) {
      r.z = __builtin_amdgcn_raw_buffer_load_b8(rz_rsrc, vo_z, blk_u >> 1, 0);
      r.zshift = ((blk_u & 1) + blk_l) * 4;
    } else {
      r.z = 8u;
      r.zshift = 0;
    }
  };
  const DequantConsts dq = MakeDequantConsts();
  // The weight row's power-of-two exponent (plan time): its block scales times
  // 2^e_b are normal fp16 numbers and (q - zp) * scale stays below 65504.
  const int e_b = col_exp[min(n0 + b_row, N - 1)];
  auto store_b = [&](const BRegs &r, int buf) {
    const uint32_t words[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const DequantRow dr =
        MakeDequantRow(__builtin_amdgcn_ldexpf(r.s, e_b), (r.z >> r.zshift) & 0xFu);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      Bbuf[buf * kBUnits + Swz(b_row, 4 * b_half + u)] = DequantWord(words[u], dr, dq);
  };

  constexpr int kMI = BM / 32;  // 16-row MFMA tiles per wavefront along M
  floatx4 acc[kMI][4];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto mma_tile = [&](int stage, int buf) {
    const uint4 *as = Astage + stage * kAUnits;
    const uint4 *bs = Bbuf + buf * kBUnits;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int unit = 4 * ks + (lane >> 4);
      half8 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = __builtin_bit_cast(half8, bs[Swz(wn * 64 + j * 16 + (lane & 15), unit)]);
#pragma unroll
      for (int i = 0; i < kMI; ++i) {
        const half8 af =
            __builtin_bit_cast(half8, as[Swz(wm * (BM / 2) + i * 16 + (lane & 15), unit)]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // Pipeline: A tile t is copied to LDS stage t % 3 two k-tiles ahead; the B
  // registers of tile t are loaded kPD k-tiles ahead (HBM latency under load
  // is several k-tiles long) and dequantized into LDS buffer t % 2 one k-tile
  // ahead. Iteration t:
  //  1. wait until A tile t (and with it B tile t+1) has landed, then a
  //     barrier: A tile t and B buffer t % 2 are complete and visible, and
  //     every read of stage (t+2) % 3 and buffer (t+1) % 2 from iteration
  //     t-1 is retired;
  //  2. dequantize B tile t+1 into buffer (t+1) % 2;
  //  3. copy A tile t+2, load the B registers of tile t+kPD into the set that
  //     held tile t;
  //  4. multiply tile t.
  // Every copy, load and store is issued unconditionally, with the k-tile
  // index clamped to the last one (the tail re-reads the last tile into
  // buffers nobody reads again): a branch around a load makes the compiler
  // wait for all outstanding loads where the paths join. So per iteration the
  // vector memory operations are exactly [kAOps A copies, kBOps B loads], and
  // after A tile t come B tile t+2, A tile t+1 and B tile t+3.
  constexpr int kPD = 4;
  constexpr int kAOps = kAUnits / 256;
  constexpr int kBOps = HAS_ZP ? 3 : 2;
  const int klast = ktiles - 1;
  BRegs rb[kPD];
  issue_a(0, 0);
  load_b(rb[0], 0);
  load_b(rb[1], min(1, klast));
  issue_a(min(1, klast), 1);
#pragma unroll
  for (int p = 2; p < kPD; ++p) load_b(rb[p], min(p, klast));
  store_b(rb[0], 0);

  // One iteration; u = t % kPD is a compile-time constant so the register
  // sets are static.
  auto step = [&](int t, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    // Nothing crosses the wait and barrier at the top of an iteration:
    // hoisted above them, the tile's dequantization would make the compiler
    // wait for its B registers with a count that ignores the A copies (it
    // cannot see them), i.e. for the copies just issued.
    __builtin_amdgcn_sched_barrier(0);
    WaitVm<2 * kBOps + kAOps>();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    store_b(rb[(u + 1) % kPD], (t + 1) & 1);
    issue_a(min(t + 2, klast), (t + 2) % kAStages);
    load_b(rb[u], min(t + kPD, klast));
    mma_tile(t % kAStages, t & 1);
  };
  // Whole groups of kPD iterations, then the remainder: a loop body with an
  // exit in the middle would merge different sets of outstanding loads at the
  // back edge, and the compiler would wait for all of them there.
  int kt = 0;
  for (; kt + kPD <= ktiles; kt += kPD) {
    step(kt, std::integral_constant<int, 0>{});
    step(kt + 1, std::integral_constant<int, 1>{});
    step(kt + 2, std::integral_constant<int, 2>{});
    step(kt + 3, std::integral_constant<int, 3>{});
  }
  if (kt < ktiles) step(kt, std::integral_constant<int, 0>{});
  if (kt + 1 < ktiles) step(kt + 1, std::integral_constant<int, 1>{});
  if (kt + 2 < ktiles) step(kt + 2, std::integral_constant<int, 2>{});
  // The remainder steps' B loads feed no later tile, so the compiler would
  // drop them, and from the second remainder step on the wait at a step's
  // top (which counts kBOps loads per step) would no longer cover that step's
  // A copy: a wavefront could read an A stage before the copy landed (seen as
  // one 8-row x 64-column block of an output tile off by a k-tile's share,
  // intermittently, with split K). Using the registers here keeps every load.
#pragma unroll
  for (int p = 0; p < kPD; ++p)
    __asm__ volatile("" ::"v"(rb[p].b.x), "v"(rb[p].b.y), "v"(rb[p].b.z), "v"(rb[p].b.w),
                     "v"(rb[p].s), "v"(rb[p].z));
  // No copy into this workgroup's LDS may land after it exits.
  WaitVm<0>();

  // Output: split 0 writes Y, split s > 0 of a split-K launch its partial sum
  // at partials + (s - 1) * M * N. Lane holds column (lane & 15), rows
  // 4*(lane >> 4) + v of each 16 x 16 tile. The accumulators are in units of
  // 2^(f_m + e_n) (A row m scaled by 2^f_m, weight row n by 2^e_n): one ldexp
  // per element undoes both exactly (a single rounding, only if the result is
  // an fp32 subnormal).
  {
    int ec[4], er[kMI][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ec[j] = col_exp[min(n0 + wn * 64 + j * 16 + (lane & 15), N - 1)];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        er[i][v] = row_exp[m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + v];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[i][j][v] = __builtin_amdgcn_ldexpf(acc[i][j][v], -(er[i][v] + ec[j]));
  }
  if (H != nullptr) {
    // Gate/up epilogue of a one-split launch. Column gn + 1 (the up of gate
    // gn, N even) is held by lane ^ 1 for the same four rows v = 0..3; the
    // even lane finishes rows 0 and 1 of each fragment, the odd lane rows 2
    // and 3, each receiving the two values it lacks through one DPP swap.
    // Stores are buffer stores at byte offsets from this tile's first output
    // row: rows past M fall beyond the resource and columns past N are sent
    // there, so nothing branches (the host fuses only when M * N / 2 * 4 <
    // 2^31 and N < 2^22, so a tile's offsets stay below 2^30).
    const int half_n = N >> 1;
    const bool odd = (lane & 1) != 0;
    const auto hr = __builtin_amdgcn_make_buffer_rsrc(
        H + static_cast<size_t>(m0) * half_n, 0, min(M - m0, BM) * half_n * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const floatx4 a = acc[i][j];
        const float r0 = PairSwap(odd ? a[0] : a[2]);
        const float r1 = PairSwap(odd ? a[1] : a[3]);
        const float h0 = odd ? SiluMul(r0, a[2]) : SiluMul(a[0], r0);
        const float h1 = odd ? SiluMul(r1, a[3]) : SiluMul(a[1], r1);
        const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
        const int row = wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + (odd ? 2 : 0);
        const int off = gn < N ? (row * half_n + (gn >> 1)) * 4 : 0x7FFFFFF0;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, h0), hr, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, h1), hr,
                                              gn < N ? off + half_n * 4 : off, 0, 0);
      }
    }
    return;
  }
  if (split > 0) Y = partials + static_cast<size_t>(split - 1) * M * N;
  if (N < (1 << 22)) {
    // Buffer stores at byte offsets from this tile's first output row (below
    // 2^31 for N < 2^22): rows past M fall beyond the resource and columns
    // past N are sent there, so no store needs a branch.
    const auto yr = __builtin_amdgcn_make_buffer_rsrc(Y + static_cast<size_t>(m0) * N, 0,
                                                      min(M - m0, BM) * N * 4, 0x00020000);
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
        const int row = wm * (BM / 2) + i * 16 + 4 * (lane >> 4);
        const int off = gn < N ? (row * N + gn) * 4 : 0x7FFFFFF0;
        // (one element of the MFMA result vector at a time, through a scalar:
        // a bit cast of the vector element itself was compiled into a store of
        // element 0 for every v on ROCm 7.2)
        const floatx4 a = acc[i][j];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float val = a[v];
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), yr,
                                                gn < N ? off + v * N * 4 : off, 0, 0);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int gm = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + v;
        if (gm < M && gn < N) Y[static_cast<size_t>(gm) * N + gn] = acc[i][j][v];
      }
    }
  }
}

// Split-K epilogue: Y += partials[0] + ... + partials[PARTS - 1], summed in
// that order for every element, so results do not depend on scheduling; then
// + bias[n] when a bias is given (Y is [mn / N, N]), after the sum, as a
// separate bias pass would add it. PARTS is a template argument so that every
// load is in flight before the first add (one HBM round trip per thread, not
// PARTS of them).
template <bool VEC, int PARTS>
__global__ __launch_bounds__(256) void SplitReduceKernel(float *__restrict__ Y,
                                                         const float *__restrict__ P,
                                                         int64_t mn, float *__restrict__ H,
                                                         const float *__restrict__ bias,
                                                         int64_t N) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * (VEC ? 4 : 1);
  if (i >= mn) return;
  if constexpr (VEC) {
    f32x4 v[PARTS];
#pragma unroll
    for (int p = 0; p < PARTS; ++p)
      v[p] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(P + p * mn + i));
    f32x4 y = *reinterpret_cast<const f32x4 *>(Y + i);
#pragma unroll
    for (int p = 0; p < PARTS; ++p) y += v[p];
    if (bias != nullptr) {  // N % 4 == 0 on this path: the 4 elements share a row
      const int64_t n = i % N;
      y += f32x4{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]};
    }
    if (H != nullptr)  // gate/up pairs (N even: a pair never straddles rows)
      *reinterpret_cast<float2 *>(H + i / 2) = make_float2(SiluMul(y[0], y[1]), SiluMul(y[2], y[3]));
    else
      *reinterpret_cast<f32x4 *>(Y + i) = y;
  } else {
    float v[PARTS];
#pragma unroll
    for (int p = 0; p < PARTS; ++p) v[p] = __builtin_nontemporal_load(P + p * mn + i);
    float y = Y[i];
#pragma unroll
    for (int p = 0; p < PARTS; ++p) y += v[p];
    if (bias != nullptr) y += bias[i % N];
    if (H != nullptr) {
      // mn is even: lanes i and i ^ 1 are both in range, in the same wavefront
      const float other = PairSwap(y);
      if ((i & 1) == 0) H[i / 2] = SiluMul(y, other);
    } else {
      Y[i] = y;
    }
  }
}

template <int PARTS>
hipError_t LaunchReduce(float *Y, const float *P, int64_t mn, hipStream_t s, float *H,
                        const float *bias, int64_t N) {
  if (mn % 4 == 0 && reinterpret_cast<uintptr_t>(Y) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(H) % 8 == 0 && (bias == nullptr || N % 4 == 0)) {
    hipLaunchKernelGGL((SplitReduceKernel<true, PARTS>),
                       dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0, s, Y, P,
                       mn, H, bias, N);
  } else {
    hipLaunchKernelGGL((SplitReduceKernel<false, PARTS>),
                       dim3(static_cast<unsigned>((mn + 255) / 256)), dim3(256), 0, s, Y, P, mn,
                       H, bias, N);
  }
  return hipGetLastError();
}

template <int... Ps>
hipError_t DispatchReduce(int parts, float *Y, const float *P, int64_t mn, hipStream_t s,
                          float *H, std::integer_sequence<int, Ps...>, const float *bias = nullptr,
                          int64_t N = 1) {
  hipError_t e = hipErrorInvalidValue;
  (void)((parts == Ps + 1 ? (e = LaunchReduce<Ps + 1>(Y, P, mn, s, H, bias, N), true) : false) ||
         ...);
  return e;
}

constexpr int kMaxSplits = 16;

struct Shape {
  int bm;      // tile height: 32, 64 or 128
  int splits;  // K splits, each a contiguous run of kt_per_split k-tiles
  int kt_per_split;
};

// Normalises a requested split count: no split is left without k-tiles.
inline Shape MakeShape(const WeightView &w, int bm, int splits) {
  const int ktiles = static_cast<int>(w.K / kBK);
  splits = std::max(1, std::min({splits, ktiles, kMaxSplits}));
  const int per = (ktiles + splits - 1) / splits;
  return Shape{bm, (ktiles + per - 1) / per, per};
}

inline int64_t PaddedRows(int64_t M) { return (M + kMaxBM - 1) / kMaxBM * kMaxBM; }

// The workspace starts with the fp16 image of A (every tile height's padding
// is covered by kMaxBM), then the rows' power-of-two exponents (int32 per
// padded row, rounded up to 256 bytes), then the split-K partial sums.
inline size_t AImageBytes(const WeightView &w, int64_t M) {
  return static_cast<size_t>(PaddedRows(M)) * static_cast<size_t>(w.K) * 2;
}

inline size_t RowExpBytes(int64_t M) {
  return (static_cast<size_t>(PaddedRows(M)) * 4 + 255) / 256 * 256;
}

inline size_t PartialBytes(const WeightView &w, int64_t M, const Shape &sh) {
  return static_cast<size_t>(sh.splits - 1) * static_cast<size_t>(M) * w.N * 4;
}

template <int BM, bool HAS_ZP>
hipError_t LaunchT(const WeightView &w, int64_t M, const uint4 *Ah, float *Y, float *partials,
                   const Shape &sh, hipStream_t s, float *H, const int *row_exp) {
  const int tiles = static_cast<int>(((M + BM - 1) / BM) * ((w.N + kBN - 1) / kBN));
  hipLaunchKernelGGL((GemmKernel<BM, HAS_ZP>), dim3(tiles * sh.splits), dim3(256), LdsBytes<BM>(),
                     s, Ah, w.B, w.scales, w.zp, Y, static_cast<int>(M), static_cast<int>(w.K),
                     static_cast<int>(w.N), static_cast<int>(w.nb), w.log2_bs,
                     static_cast<int>(w.row_bytes), static_cast<int>(w.zp_row_bytes),
                     sh.kt_per_split, partials, H, row_exp, w.col_exp);
  return hipGetLastError();
}

// ConvertAKernel over the padded rows of a BM tiling, keeping each thread's
// share of the row in registers when K allows.
template <int BM, bool RMS>
hipError_t LaunchConvertA(const WeightView &w, int64_t M, const float *A, uint4 *Ah, int *row_exp,
                          hipStream_t s, const float *gamma, float eps) {
  const dim3 grid(static_cast<unsigned>((M + BM - 1) / BM * BM)), block(256);
  const int K = static_cast<int>(w.K), m = static_cast<int>(M);
  if (K <= 2048 * 2)
    hipLaunchKernelGGL((ConvertAKernel<BM, 2, RMS>), grid, block, 0, s, A, Ah, row_exp, m, K, gamma, eps);
  else if (K <= 2048 * 4)
    hipLaunchKernelGGL((ConvertAKernel<BM, 4, RMS>), grid, block, 0, s, A, Ah, row_exp, m, K, gamma, eps);
  else if (K <= 2048 * 8)
    hipLaunchKernelGGL((ConvertAKernel<BM, 8, RMS>), grid, block, 0, s, A, Ah, row_exp, m, K, gamma, eps);
  else
    hipLaunchKernelGGL((ConvertAKernel<BM, 0, RMS>), grid, block, 0, s, A, Ah, row_exp, m, K, gamma, eps);
  return hipGetLastError();
}

template <int BM>
hipError_t LaunchBM(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                    const Shape &sh, hipStream_t s, float *H, const float *gamma, float eps) {
  uint4 *Ah = static_cast<uint4 *>(work);
  int *row_exp = reinterpret_cast<int *>(static_cast<char *>(work) + AImageBytes(w, M));
  float *partials = reinterpret_cast<float *>(static_cast<char *>(work) + AImageBytes(w, M) +
                                              RowExpBytes(M));
  hipError_t e = gamma != nullptr
                     ? LaunchConvertA<BM, true>(w, M, A, Ah, row_exp, s, gamma, eps)
                     : LaunchConvertA<BM, false>(w, M, A, Ah, row_exp, s, nullptr, 0.0f);
  if (e != hipSuccess) return e;
  // Gate/up activation: fused into the GEMM's stores with one split, into the
  // reduction (split 0 then writes the scratch Y) with several.
  float *Hk = sh.splits == 1 ? H : nullptr;
  e = w.zp != nullptr ? LaunchT<BM, true>(w, M, Ah, Y, partials, sh, s, Hk, row_exp)
                      : LaunchT<BM, false>(w, M, Ah, Y, partials, sh, s, Hk, row_exp);
  if (e != hipSuccess || sh.splits == 1) return e;
  return DispatchReduce(sh.splits - 1, Y, partials, M * w.N, s, H,
                        std::make_integer_sequence<int, kMaxSplits - 1>{});
}

// Tile height and K splits, from sweeps on MI355X of every tile height
// against 1..16 splits (c2..c5 shapes, M = 2..2048):
// - tile height: 32 for M <= 32, 64 for M <= 64, else 128 (taller tiles
//   amortise the B dequantization over more rows and won at every M >= 128,
//   once split-K supplies the workgroups);
// - splits: as many as keep the whole launch within one wave of two
//   workgroups per CU (a partial second wave costs a full k-loop), and no
//   fewer than 8 k-tiles per split (the prologue and the reduction are not
//   free).
inline Shape PickShape(const WeightView &w, int64_t M) {
  const int bm = M <= 32 ? 32 : M <= 64 ? 64 : 128;
  const int64_t tiles = (M + bm - 1) / bm * ((w.N + kBN - 1) / kBN);
  const int64_t slots = 2 * static_cast<int64_t>(w.num_cus);
  const int ktiles = static_cast<int>(w.K / kBK);
  int64_t splits = std::max<int64_t>(1, slots / tiles);
  splits = std::min<int64_t>({splits, kMaxSplits, std::max(1, ktiles / 8)});
  return MakeShape(w, bm, static_cast<int>(splits));
}

// ---------------------------------------------------------------------------
// Prefill GEMM over the plan's fragment-ordered weights (PrefillKernel).
//
// At plan creation the weights are re-laid for this kernel (RelayoutBKernel,
// RelayoutSKernel): for each group g of 64 weight rows and each 32-k step s,
// the 1 KiB record Bp[g][s][lane][j] holds in lane l's 16 bytes the packed
// word (8 nibbles, original order) of weight row 64g + 16j + (l & 15) at k =
// 32s + 8(l >> 4): exactly lane l's MFMA operand for the 16 rows of slice j.
// The 256-byte record Sp[g][b][c][j] holds, per quantization block b, the
// fp16 scale (times the row's 2^e) in the low half and the zero point in the
// high half, for row 64g + 16j + c. Rows past N are zero (scale 0). One record
// per block, not per step: every step of a block reads the same record.
//
// A workgroup of 8 wavefronts (two per SIMD, one workgroup per CU) computes a
// 128 x 256 output tile. Wavefronts w and w + 4 own columns 64(w % 4) ..
// 64(w % 4) + 63 of all 128 rows and split K: w takes the first 32-k step of
// every 64-k tile, w + 4 the second, so each dequantized weight fragment
// feeds 8 MFMAs (13 VALU per 8 nibbles: 1.6 VALU per MFMA) and each SIMD
// holds two independent instruction streams to fill the other's waits. At
// the end the two halves meet in LDS (each wavefront adds the other's sum
// for 64 of the rows, in a fixed order). The MFMA takes the weights as its A
// operand and the activations as its B operand, so each lane's result is 4
// consecutive output columns of one row: 16-byte stores, and a gate/up pair
// (columns 2n, 2n + 1) lands in one lane.
// Every operand streams global -> LDS through direct copies (no registers)
// into a ring of kPNS stages of one 64-k tile each (A 16 KiB, weights 8 KiB,
// scales 4 KiB); the copies of tile t + kPSA are issued as tile t starts.
// The copy order per k-tile is fixed (2 A copies and 1 weight copy per
// thread, plus 1 scale copy in the first four wavefronts), so each wait is an
// exact vmcnt. One barrier per k-tile, at its top, makes tile t + 1 visible:
// tile t's MFMAs then run on fragments read during the previous tile, while
// tile t + 1's fragments are read (into a second register set) and
// dequantized.
constexpr int kPTM = 128;                             // output tile rows
constexpr int kPTN = 256;                             // output tile columns
constexpr int kPThreads = 512;                        // 8 wavefronts
constexpr int kPNS = 5;                               // LDS stages (k-tiles)
constexpr int kPSA = kPNS - 1;                        // copy distance (k-tiles)
constexpr int kPAU = kPTM * kUnits;                   // A units per stage (1024)
constexpr int kPBU = 128;                             // weight units per column group per stage
constexpr int kPSU = 64;                              // scale units per column group per stage
constexpr int kPStage = kPAU + 4 * (kPBU + kPSU);     // 1792 units, 28 KiB
constexpr size_t kPLds = size_t{kPNS} * kPStage * 16; // 140 KiB
constexpr int kPOps0 = kPAU / kPThreads + 2;          // copies per k-tile, wavefronts 0-3
constexpr int kPOps1 = kPAU / kPThreads + 1;          // wavefronts 4-7 (no scale copy)
// Cache policy of the output stores: non-temporal. Y is not read again by
// this kernel; streaming it out keeps the L2 for the operand tiles (measured:
// c5 gate+up M = 2048, 224 MiB of Y, 472 -> 445 us; c4 unchanged). With K
// split, the split reduction reads Y and the partial sums straight back, and
// plain stores serve it better (c4 and c5 o at M = 512, 4 splits: 37.1 ->
// 35.4 and 38.0 -> 36.3 us per call; qkv at M = 256 33.2 -> 32.2).
constexpr int kStoreNT = 2;

// (scale fp16 | zp << 16) -> the operands of DequantWord.
template <bool HAS_ZP>
__device__ __forceinline__ DequantRow RowFromSz(uint32_t w) {
  DequantRow r;
  r.s = __builtin_amdgcn_perm(w, w, 0x01000100u);  // the fp16 scale in both halves
  if constexpr (HAS_ZP) {
    const uint32_t z = w >> 16;
    r.neg_lo = 0xE400E400u + z * 0x00010001u;  // fp16 -(1024 + z): ulp 1 at 1024
    r.neg_hi = 0xD400D400u + z * 0x00100010u;  // fp16 -(64 + z): ulp 1/16 at 64
  } else {
    r.neg_lo = 0xE408E408u;  // -(1024 + 8)
    r.neg_hi = 0xD480D480u;  // -(64 + 8)
  }
  return r;
}

template <bool HAS_ZP, bool BS32>
__global__ __launch_bounds__(kPThreads, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void
PrefillKernel(const uint4 *__restrict__ Ah, const uint8_t *__restrict__ Bp,
              const uint8_t *__restrict__ Sp, float *__restrict__ Y, int M, int N, int K,
              int log2_bs, int kt_per_split, float *__restrict__ partials, float *__restrict__ H,
              const int *__restrict__ row_exp, const int *__restrict__ col_exp,
              const float *__restrict__ bias) {
  extern __shared__ uint4 lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = wave & 3;   // column group: columns 64 cg .. 64 cg + 63 of the tile

  // Workgroup b -> (split, output tile). XCD x (b % 8) takes a contiguous run
  // of the tile order, which walks groups of 4 M tiles N tile by N tile, so
  // an XCD's L2 holds about 4 A bands and a run of weight bands.
  const int tiles_m = (M + kPTM - 1) / kPTM;
  const int tiles_n = (N + kPTN - 1) / kPTN;
  const int tiles = tiles_m * tiles_n;
  const int split = static_cast<int>(blockIdx.x) / tiles;
  int tm, tn;
  {
    int L = static_cast<int>(blockIdx.x) - split * tiles;
    if (tiles % 8 == 0) L = (L & 7) * (tiles / 8) + (L >> 3);
    constexpr int kGM = 4;
    const int group = L / (kGM * tiles_n);
    const int gm = min(kGM, tiles_m - group * kGM);
    const int rem = L - group * kGM * tiles_n;
    tm = group * kGM + rem % gm;
    tn = rem / gm;
  }
  const int m0 = tm * kPTM;
  const int n0 = tn * kPTN;
  const int T = K / 32;
  const int kt0 = split * kt_per_split;
  const int ktiles = min(kt_per_split, K / kBK - kt0);
  const int klast = ktiles - 1;
  const int g = n0 / 64 + cg;

  // The body, for the 32-k step sg (0 for wavefronts 0-3, 1 for 4-7) as a
  // template argument: no branch inside the loop, every index a constant.
  auto body = [&](auto sg_c) __attribute__((always_inline)) {
  constexpr int sg = decltype(sg_c)::value;
  // Copies per k-tile: A instruction i of wavefront w takes units
  // i * 512 + 64 w + lane; wavefront w the weight record of (g, step sg);
  // wavefronts 0-3 the scale records of g for both steps (lanes 16-31 the
  // second step's, lanes 32-63 repeat lanes 0-31). 32-k blocks: one record per
  // step; larger blocks hold both steps of a 64-k tile, whose record repeats.
  // Sources as a wave-uniform base (SGPRs) plus the lane's byte offset.
  const int nb = (K + (1 << log2_bs) - 1) >> log2_bs;
  const uint4 *a_base = Ah + (static_cast<size_t>(tm) * (K / kBK) + kt0) * kPAU + wave * 64;
  const uint8_t *b_base = Bp + (static_cast<size_t>(g) * T + 2 * kt0 + sg) * 1024;
  const uint8_t *s_base = Sp + static_cast<size_t>(g) * nb * 256;
  const uint32_t a_off = static_cast<uint32_t>(lane) * 16;
  const uint32_t s_off = static_cast<uint32_t>(lane & (BS32 ? 31 : 15)) * 16;
  const int bt_shift = BS32 ? 0 : log2_bs - 6;  // 64-k tiles per block, log2
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  auto issue = [&](int kt, int st) {
    const uint32_t base = lds0 + static_cast<uint32_t>(st * kPStage * 16);
#pragma unroll
    for (int i = 0; i < kPAU / kPThreads; ++i)
      CopyToLds16S(a_base + static_cast<size_t>(kt) * kPAU + i * kPThreads, a_off,
                   base + static_cast<uint32_t>((i * kPThreads + wave * 64) * 16));
    CopyToLds16S(b_base + static_cast<size_t>(kt) * 2048, a_off,
                 base + static_cast<uint32_t>((kPAU + cg * kPBU + sg * 64) * 16));
    if constexpr (sg == 0)
      CopyToLds16S(s_base + (BS32 ? static_cast<size_t>(2 * (kt0 + kt)) * 256
                                  : static_cast<size_t>((kt0 + kt) >> bt_shift) * 256),
                   s_off, base + static_cast<uint32_t>((kPAU + 4 * kPBU + cg * kPSU) * 16));
  };
  // Tile t + 1 has landed once only the copies of tiles t + 2 .. t + kPSA - 1
  // (issued at the tops of the iterations since) are outstanding.
  constexpr int kOps = sg == 0 ? kPOps0 : kPOps1;
  auto readA = [&](const uint4 *sb, int i) {
    return __builtin_bit_cast(half8, sb[Swz(i * 16 + (lane & 15), 4 * sg + (lane >> 4))]);
  };
  auto readB = [&](const uint4 *sb) { return sb[kPAU + cg * kPBU + sg * 64 + lane]; };
  auto readS = [&](const uint4 *sb) {
    return sb[kPAU + 4 * kPBU + cg * kPSU + sg * 16 + (lane & 15)];
  };

  floatx4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const DequantConsts dq = MakeDequantConsts();
  // Dequantized weight fragments of one 32-k step (MFMA A operands, slices j).
  auto dequant = [&](uint4 bw, uint4 sw, half8 (&bf)[4]) __attribute__((always_inline)) {
    const uint32_t w[4] = {bw.x, bw.y, bw.z, bw.w};
    const uint32_t z[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bf[j] = __builtin_bit_cast(half8, DequantWord(w[j], RowFromSz<HAS_ZP>(z[j]), dq));
  };
  // One k-tile: tile t + 1's weight words are dequantized and its activation
  // fragments read into the second register set while tile t's 32 MFMAs run
  // on the first, so no MFMA waits for an LDS read issued in the same
  // iteration (reading the fragments after their last use, into one set,
  // left the first MFMAs of every tile waiting for the reads: c4 75.9 ->
  // 69.3 us with the second set, bit-identical). The scheduler interleaves
  // each MFMA with up to two VALU of the dequantization.
  auto iter = [&](int t, half8 (&ac)[8], half8 (&an)[8], half8 (&bc)[4], half8 (&bn)[4])
                  __attribute__((always_inline)) {
    const uint4 *sb1 = lds + ((t + 1) % kPNS) * kPStage;
    // Tile t + 1 complete and visible (only the copies of tiles t + 2 ..
    // t + kPSA - 1 are outstanding); every wavefront is past tile t - 1.
    WaitVm<kOps * (kPSA - 2)>();
    __syncthreads();
    // Tile t + kPSA into stage (t - 1) % kPNS, last read in iteration t - 2.
    issue(min(t + kPSA, klast), (t + kPSA) % kPNS);
    const uint4 bwn = readB(sb1);
    const uint4 swn = readS(sb1);
#pragma unroll
    for (int i = 0; i < 8; ++i) an[i] = readA(sb1, i);
    __builtin_amdgcn_sched_barrier(0);
    dequant(bwn, swn, bn);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bc[j], ac[i], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
  };

  // Prologue: tiles 0 .. kPSA-1 into stages 0 .. kPSA-1; wait for tile 0.
#pragma unroll
  for (int p = 0; p < kPSA; ++p) issue(min(p, klast), p);
  WaitVm<kOps * (kPSA - 1)>();
  __syncthreads();
  half8 a0[8], a1[8], b0[4], b1[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) a0[i] = readA(lds, i);
  dequant(readB(lds), readS(lds), b0);
  // Two iterations per trip, the register sets trading roles.
  int t = 0;
  for (; t + 1 < ktiles; t += 2) {
    iter(t, a0, a1, b0, b1);
    iter(t + 1, a1, a0, b1, b0);
  }
  if (t < ktiles) iter(t, a0, a1, b0, b1);
  // No copy into this workgroup's LDS may land after it exits, or after the
  // LDS is reused below.
  WaitVm<0>();
  __syncthreads();

  // The two K halves meet: wavefront w + 4s finishes rows 64s .. 64s + 63
  // (fragments i = 4s .. 4s + 3) of column group cg and hands the other rows
  // to its partner through LDS (16 KiB per wavefront, as 16 x 16 fragments of
  // 16 bytes per lane). Sum order: step 0's half, then step 1's. The half is
  // a template argument so every accumulator index is a constant.
  float *out = split > 0 ? partials + static_cast<size_t>(split - 1) * M * N : Y;
  const int nl = n0 + cg * 64 + 4 * (lane >> 4);
  const int rows = min(M - m0, kPTM);
  {
    constexpr int S = sg;
    uint4 *xb = lds + wave * 1024;  // this wavefront's outgoing fragments
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const floatx4 v = acc[4 * (1 - S) + q][j];
        xb[(q * 4 + j) * 64 + lane] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                 __float_as_uint(v[2]), __float_as_uint(v[3]));
      }
    __syncthreads();
    const uint4 *pb = lds + (wave ^ 4) * 1024;  // the partner's fragments for my rows
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 u = pb[(q * 4 + j) * 64 + lane];
        const floatx4 o = {__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                           __uint_as_float(u.w)};
        acc[4 * S + q][j] = S == 0 ? acc[4 * S + q][j] + o : o + acc[4 * S + q][j];
      }

    // Epilogue over this wavefront's 64 rows. Lane l holds, for fragment i
    // (rows 16i .. 16i + 15) and slice j, row m0 + 16i + (l & 15) and the 4
    // columns n0 + 64 cg + 16j + 4(l >> 4) + v. The accumulators are in units
    // of 2^(f_m + e_n): one ldexp per element undoes both. Split 0 writes Y
    // (and adds the bias), split s > 0 its partial sum.
    int er[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) er[q] = row_exp[m0 + (4 * S + q) * 16 + (lane & 15)];
    if (H != nullptr) {
      const int half_n = N >> 1;
      const auto hr = __builtin_amdgcn_make_buffer_rsrc(H + static_cast<size_t>(m0) * half_n, 0,
                                                        rows * half_n * 4, 0x00020000);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = nl + 16 * j;
        const int nc = min(n, N - 4);
        const int e0 = col_exp[nc], e1 = col_exp[nc + 1], e2 = col_exp[nc + 2],
                  e3 = col_exp[nc + 3];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 a = acc[4 * S + q][j];
          const float x0 = a[0], x1 = a[1], x2 = a[2], x3 = a[3];
          const float h0 = SiluMul(__builtin_amdgcn_ldexpf(x0, -(er[q] + e0)),
                                   __builtin_amdgcn_ldexpf(x1, -(er[q] + e1)));
          const float h1 = SiluMul(__builtin_amdgcn_ldexpf(x2, -(er[q] + e2)),
                                   __builtin_amdgcn_ldexpf(x3, -(er[q] + e3)));
          const int row = (4 * S + q) * 16 + (lane & 15);
          const int off = n < N ? (row * half_n + (n >> 1)) * 4 : 0x7FFFFFF0;
          // H columns n / 2 and n / 2 + 1 are adjacent: one 8-byte store. (A
          // non-temporal hint on these partial-line stores made the fused
          // plan 20-30% slower than the plain product; they stay cached.)
          typedef unsigned int u32x2 __attribute__((vector_size(8)));
          const u32x2 hv = {__float_as_uint(h0), __float_as_uint(h1)};
          __builtin_amdgcn_raw_buffer_store_b64(hv, hr, off, 0, 0);
        }
      }
      return;
    }
    const auto yr = __builtin_amdgcn_make_buffer_rsrc(out + static_cast<size_t>(m0) * N, 0,
                                                      rows * N * 4, 0x00020000);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = nl + 16 * j;
      const int nc = min(n, N - 4);
      const int e0 = col_exp[nc], e1 = col_exp[nc + 1], e2 = col_exp[nc + 2], e3 = col_exp[nc + 3];
      float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
      if (bias != nullptr && split == 0) {
        b0 = bias[nc];
        b1 = bias[nc + 1];
        b2 = bias[nc + 2];
        b3 = bias[nc + 3];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 a = acc[4 * S + q][j];
        const float x0 = a[0], x1 = a[1], x2 = a[2], x3 = a[3];
        typedef unsigned int u32x4 __attribute__((vector_size(16)));
        const u32x4 v = {__float_as_uint(__builtin_amdgcn_ldexpf(x0, -(er[q] + e0)) + b0),
                         __float_as_uint(__builtin_amdgcn_ldexpf(x1, -(er[q] + e1)) + b1),
                         __float_as_uint(__builtin_amdgcn_ldexpf(x2, -(er[q] + e2)) + b2),
                         __float_as_uint(__builtin_amdgcn_ldexpf(x3, -(er[q] + e3)) + b3)};
        const int row = (4 * S + q) * 16 + (lane & 15);
        const int off = n < N ? (row * N + n) * 4 : 0x7FFFFFF0;
        if (kt_per_split < K / kBK)  // split K: read back by the reduction
          __builtin_amdgcn_raw_buffer_store_b128(v, yr, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b128(v, yr, off, 0, kStoreNT);
      }
    }
  }
  };
  if ((wave >> 2) == 0)
    body(std::integral_constant<int, 0>{});
  else
    body(std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------------------
// Small-M prefill (17 <= M <= 64) streaming the fragment-ordered weights
// (StreamKernel). With so few rows a 128 x 256 tile holds mostly padding and
// the GEMM is bound by reading the weights once, so the grid is laid out
// like the decode kernels': one workgroup per (group g of 64 weight rows, K
// segment), WPG wavefronts each taking SPW consecutive 32-k steps of the
// segment. Per step a wavefront loads the group's 1 KiB weight record and
// 256-byte scale record (the PrefillKernel layouts), dequantizes the four
// words exactly as PrefillKernel does (DequantWord on the fp16 scale times
// 2^e_n), reads TG activation fragments of the fp16 image ConvertAKernel
// wrote (BM = 64 tiling, rows scaled by 2^f_m, rows past M zero) and issues
// 4 TG v_mfma_f32_16x16x32_f16 into TG x 4 fp32 tiles. The operands are
// those of the prefill GEMM, so the product is the same up to the order of
// the fp32 sums. Loads stream through a rolling window of WIN steps in
// registers (multiply the oldest, issue the one WIN further on), with no
// branch around any load. The wavefronts' tiles meet in LDS and are added
// in wavefront order; segment 0 writes Y (adding the bias or applying the
// gate/up activation when K is not split), segment s > 0 its partial sum,
// added in segment order by SplitReduceKernel.
constexpr int kSGroupRows = 64;

//
// CVT: the wavefront converts its own activations instead of reading the
// image (no ConvertAKernel launch; used for small fragment counts, see
// StreamConverts): it loads A's fp32 values for its SPW steps first (L2-
// resident, ahead of the weights), reduces each row's largest magnitude over
// its own k range across the four lanes that hold the row, scales by 2^f and
// rounds to fp16 as ConvertAKernel does, and scales its tiles by 2^-f before
// the wavefronts' tiles meet. A finer exponent than the row's, so the
// operands are ConvertAKernel's except where those fall into fp16
// subnormals.
template <bool HAS_ZP, int TG, int SPW, int WIN, bool CVT>
__global__ __launch_bounds__(512) void StreamKernel(
    const uint4 *__restrict__ Ah, const float *__restrict__ A, const uint8_t *__restrict__ Bp,
    const uint8_t *__restrict__ Sp, float *__restrict__ Y, float *__restrict__ partials,
    float *__restrict__ H, const int *__restrict__ row_exp, const int *__restrict__ col_exp,
    const float *__restrict__ bias, int M, int N, int K, int log2_bs, int segs, int wpg) {
  extern __shared__ floatx4 sred[];  // [wave][tg * 4 + j][lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int g = static_cast<int>(blockIdx.x) / segs;
  const int seg = static_cast<int>(blockIdx.x) - g * segs;
  const int T = K / 32;
  const int s0 = (seg * wpg + wave) * SPW;  // first step of this wavefront
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(Bp + static_cast<size_t>(g) * T * 1024), 0, T * 1024, 0x00020000);
  const int nb = (K + (1 << log2_bs) - 1) >> log2_bs;
  const int sb_shift = log2_bs - 5;  // 32-k steps per block, log2
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(Sp + static_cast<size_t>(g) * nb * 256), 0, nb * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4 *>(Ah), 0, (K / kBK) * AUnits<kSGroupRows>() * 16, 0x00020000);
  // Lane l's activation fragment tg of step s: row 16 tg + (l & 15), unit
  // 4 (s & 1) + (l >> 4) of k-tile s / 2 (the PrefillKernel operand order).
  int aoff[TG][2];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg)
#pragma unroll
    for (int h = 0; h < 2; ++h) aoff[tg][h] = Swz(16 * tg + (lane & 15), 4 * h + (lane >> 4)) * 16;

  typedef uint32_t u32x4e __attribute__((ext_vector_type(4)));
  typedef float f32x4e __attribute__((ext_vector_type(4)));
  // CVT: the wavefront's fp32 activations, [step][tg] pairs of 4 k (k order
  // 0..3, 4..7 of the lane's 8), loaded before anything else.
  f32x4e alo[CVT ? SPW : 1][CVT ? TG : 1], ahi[CVT ? SPW : 1][CVT ? TG : 1];
  if constexpr (CVT) {
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, M * K * 4, 0x00020000);
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      const int m = 16 * tg + (lane & 15);
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        // rows past M read past the end of the buffer: zeros
        const int off = m < M ? (m * K + 32 * (s0 + i) + 8 * (lane >> 4)) * 4 : M * K * 4;
        alo[i][tg] = __builtin_bit_cast(f32x4e, __builtin_amdgcn_raw_buffer_load_b128(rA, off, 0, 0));
        ahi[i][tg] = __builtin_bit_cast(f32x4e, __builtin_amdgcn_raw_buffer_load_b128(rA, off + 16, 0, 0));
      }
    }
  }
  struct Slot {
    u32x4e w, sz;
    half8 a[CVT ? 1 : TG];
  };
  Slot ring[WIN];
  auto issue = [&](int i) __attribute__((always_inline)) {
    Slot &sl = ring[i % WIN];
    const int s = s0 + i;
    sl.w = __builtin_bit_cast(u32x4e, __builtin_amdgcn_raw_buffer_load_b128(rb, s * 1024 + 16 * lane, 0, 2));
    sl.sz = __builtin_bit_cast(u32x4e, __builtin_amdgcn_raw_buffer_load_b128(
                                           rs, (s >> sb_shift) * 256 + 16 * (lane & 15), 0, 0));
    if constexpr (!CVT) {
      const int kt = s >> 1;
#pragma unroll
      for (int tg = 0; tg < TG; ++tg)
        sl.a[tg] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(
                                                 ra, kt * (AUnits<kSGroupRows>() * 16) + aoff[tg][s & 1], 0, 0));
    }
  };
#pragma unroll
  for (int i = 0; i < WIN && i < SPW; ++i) issue(i);
  // The epilogue's exponents and bias for the fragments x = wave, wave + wpg,
  // ... this wavefront finishes (at most 4: wpg >= 4), loaded behind the
  // first weights so their latency hides under the main loop.
  constexpr int kMaxItems = (TG * 4 + 3) / 4;
  int er[kMaxItems];
  int4 ec[kMaxItems];
  float4 bv[kMaxItems];
#pragma unroll
  for (int it = 0; it < kMaxItems; ++it) {
    const int x = min(wave + it * wpg, TG * 4 - 1);
    const int m = min(16 * (x >> 2) + (lane & 15), M - 1);
    const int nc = min(kSGroupRows * g + 16 * (x & 3) + 4 * (lane >> 4), N - 4);
    er[it] = CVT ? 0 : row_exp[m];
    ec[it] = *reinterpret_cast<const int4 *>(col_exp + nc);
    bv[it] = bias != nullptr ? make_float4(bias[nc], bias[nc + 1], bias[nc + 2], bias[nc + 3])
                             : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __builtin_amdgcn_sched_barrier(0);

  // CVT: each row's exponent over this wavefront's k range (the row's values
  // sit in lanes r, r + 16, r + 32, r + 48), then the fp16 fragments.
  half8 af[CVT ? SPW : 1][CVT ? TG : 1];
  int fw[CVT ? TG : 1];
  if constexpr (CVT) {
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < SPW; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          amax = fmaxf(amax, fmaxf(fabsf(alo[i][tg][c]), fabsf(ahi[i][tg][c])));
      amax = fmaxf(amax, Xor16(amax));
      amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
      const int f = RangeExponent(amax, kRowExpTarget);
      fw[tg] = f;
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        auto sc = [f](float v) { return __builtin_amdgcn_ldexpf(v, f); };
        const f32x4e x = alo[i][tg], y = ahi[i][tg];
        // k order [0,4,1,5,2,6,3,7], the order DequantWord produces
        af[i][tg] = __builtin_bit_cast(
            half8, make_uint4(PackHalf2(sc(x[0]), sc(y[0])), PackHalf2(sc(x[1]), sc(y[1])),
                              PackHalf2(sc(x[2]), sc(y[2])), PackHalf2(sc(x[3]), sc(y[3]))));
      }
    }
  }

  const DequantConsts dq = MakeDequantConsts();
  floatx4 acc[TG][4];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[tg][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    Slot &sl = ring[i % WIN];
    __asm__ volatile("" : "+v"(sl.w), "+v"(sl.sz));
    const uint32_t wv[4] = {sl.w[0], sl.w[1], sl.w[2], sl.w[3]};
    const uint32_t zv[4] = {sl.sz[0], sl.sz[1], sl.sz[2], sl.sz[3]};
    half8 bf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bf[j] = __builtin_bit_cast(half8, DequantWord(wv[j], RowFromSz<HAS_ZP>(zv[j]), dq));
#pragma unroll
    for (int tg = 0; tg < TG; ++tg) {
      half8 a;
      if constexpr (CVT)
        a = af[i][tg];
      else
        a = sl.a[tg];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[tg][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], a, acc[tg][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i + WIN < SPW) issue(i + WIN);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The wavefronts' tiles meet in LDS; wavefront w then finishes the
  // fragments x = (tg, j) = w, w + wpg, ..., adding the wavefronts' tiles in
  // wavefront order. Lane l holds row 16 tg + (l & 15) and the 4 columns
  // 64 g + 16 j + 4 (l >> 4) .. + 3. A wavefront past K (the end of a
  // shorter last segment) ran on loads beyond the weights' buffers (zeros)
  // and activations past its rows: it adds nothing.
  const bool past_k = s0 >= T;
#pragma unroll
  for (int tg = 0; tg < TG; ++tg)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      floatx4 t = acc[tg][j];
      if constexpr (CVT) {
#pragma unroll
        for (int q = 0; q < 4; ++q) t[q] = __builtin_amdgcn_ldexpf(t[q], -fw[tg]);
      }
      sred[(wave * TG * 4 + tg * 4 + j) * 64 + lane] = past_k ? floatx4{0.f, 0.f, 0.f, 0.f} : t;
    }
  __syncthreads();
  float *out = seg == 0 ? Y : partials + static_cast<size_t>(seg - 1) * M * N;
#pragma unroll
  for (int it = 0; it < kMaxItems; ++it) {
    const int x = wave + it * wpg;
    if (x >= TG * 4) break;
    floatx4 sum = sred[x * 64 + lane];
    for (int w = 1; w < wpg; ++w) sum += sred[(w * TG * 4 + x) * 64 + lane];
    const int tg = x >> 2, j = x & 3;
    const int m = 16 * tg + (lane & 15);
    const int n = kSGroupRows * g + 16 * j + 4 * (lane >> 4);
    const int ecv[4] = {ec[it].x, ec[it].y, ec[it].z, ec[it].w};
    floatx4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = __builtin_amdgcn_ldexpf(sum[q], -((CVT ? 0 : er[it]) + ecv[q]));
    const bool ok = m < M && n < N;
    if (H != nullptr) {
      // gate/up pairs (columns n, n + 1 and n + 2, n + 3): H columns n / 2, n / 2 + 1
      const int half_n = N >> 1;
      const auto hr = __builtin_amdgcn_make_buffer_rsrc(H, 0, M * half_n * 4, 0x00020000);
      typedef unsigned int u32x2 __attribute__((vector_size(8)));
      const u32x2 hv = {__float_as_uint(SiluMul(v[0], v[1])), __float_as_uint(SiluMul(v[2], v[3]))};
      __builtin_amdgcn_raw_buffer_store_b64(hv, hr, ok ? (m * half_n + (n >> 1)) * 4 : M * half_n * 4, 0, 0);
    } else {
      if (bias != nullptr) {
        v[0] += bv[it].x;
        v[1] += bv[it].y;
        v[2] += bv[it].z;
        v[3] += bv[it].w;
      }
      const auto yr = __builtin_amdgcn_make_buffer_rsrc(out, 0, M * N * 4, 0x00020000);
      typedef unsigned int u32x4 __attribute__((vector_size(16)));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yr,
                                             ok ? (m * N + n) * 4 : M * N * 4, 0, 0);
    }
  }
}

struct StreamShape {
  int segs, wpg, spw;
  bool ragged = false;  // a shorter last segment
};

// K segments, wavefronts per workgroup and steps per wavefront (segs * wpg *
// spw = K / 32): the fewest segments whose workgroups cover 85% of the CUs
// (else the most that leave a workgroup at least 16 steps), then 8
// wavefronts before 4 and the longest spw in {16, 8, 4}. Step counts with no
// such division (K = 11008: 344 steps = 8 x 43) take segments of one length
// and a shorter last one: for each segment count the least padded wpg x spw
// of whole wavefronts (K / 32 a multiple of spw) that gives that count, the
// fewest covering 85% of the CUs; the wavefronts past K add nothing. Such
// shapes serve up to 32 rows (measured against GemmKernel, which took these
// shapes before: K = 11008, N = 4096 at M = 17 / 24 / 32 22.4 / 22.8 / 23.3
// -> 20.4 / 20.6 / 20.9 us, K = 18944, N = 3584 at M = 32 32.7 -> 29.8; at
// M = 40-64 level or slower, up to +21%).
inline StreamShape PickStreamShape(const WeightView &w, int segs_req, int spw_req) {
  const int64_t groups = (w.N + kSGroupRows - 1) / kSGroupRows;
  const int T = static_cast<int>(w.K / 32);
  if (segs_req > 0 && spw_req > 0) {
    const int per = segs_req * spw_req;
    return StreamShape{segs_req, T % per == 0 ? T / per : 0, spw_req};
  }
  auto fit = [](int per) {
    for (int wpg : {8, 4})
      for (int spw : {16, 8, 4})
        if (wpg * spw == per) return StreamShape{0, wpg, spw};
    return StreamShape{0, 0, 0};
  };
  StreamShape best{0, 0, 0};
  for (int segs = 1; segs <= kMaxSplits; ++segs) {
    if (T % segs != 0) continue;
    StreamShape sh = fit(T / segs);
    if (sh.wpg == 0) continue;
    sh.segs = segs;
    best = sh;
    if (groups * segs * 100 >= static_cast<int64_t>(w.num_cus) * 85) break;
  }
  if (best.wpg != 0) return best;
  for (int segs = 1; segs <= kMaxSplits; ++segs) {
    StreamShape sh{0, 0, 0};
    for (int wpg : {8, 4})
      for (int spw : {16, 8, 4}) {
        const int per = wpg * spw;
        if (T % spw != 0 || (T + per - 1) / per != segs) continue;
        if (sh.wpg == 0 || per < sh.wpg * sh.spw) sh = StreamShape{segs, wpg, spw, true};
      }
    if (sh.wpg == 0) continue;
    best = sh;
    if (groups * segs * 100 >= static_cast<int64_t>(w.num_cus) * 85) break;
  }
  return best;
}

// Whether the wavefronts convert their own activations: no RMSNorm input, at
// most 8 fragments per wavefront, and no more workgroups than CUs. Measured
// per call against ConvertAKernel + the image: c4 M = 17 / 32 10.45 -> 8.79
// / 10.76 -> 10.11 us; slower where the fragments or the workgroups are more
// (c4 M = 48 / 64 +0.4 / +1.2 us, c3 M = 32 with 8 steps per wavefront
// +4.9 us, c5 qkv M = 32 with 1.5 workgroups per CU +1.4 us).
inline bool StreamConverts(const WeightView &w, int64_t M, const StreamShape &sh, bool rms) {
  const int64_t wgs = (w.N + kSGroupRows - 1) / kSGroupRows * sh.segs;
  return !rms && (M + 15) / 16 * sh.spw <= 8 && wgs <= w.num_cus;
}

template <bool HAS_ZP, int TG, int SPW>
hipError_t LaunchStreamT(const WeightView &w, int64_t M, const uint4 *Ah, const float *A, float *Y,
                         float *P, float *H, const int *row_exp, const float *bias,
                         const StreamShape &sh, hipStream_t s) {
  const int64_t groups = (w.N + kSGroupRows - 1) / kSGroupRows;
  const size_t lds = static_cast<size_t>(sh.wpg) * TG * 4 * 64 * 16;
  const dim3 grid(static_cast<unsigned>(groups * sh.segs)), block(64 * sh.wpg);
  const int m = static_cast<int>(M), n = static_cast<int>(w.N), k = static_cast<int>(w.K);
  if (A != nullptr) {
    if constexpr (TG * SPW <= 16)
      hipLaunchKernelGGL((StreamKernel<HAS_ZP, TG, SPW, 4, true>), grid, block, lds, s, Ah, A, w.Bp,
                         w.Sp, Y, P, H, row_exp, w.col_exp, bias, m, n, k, w.log2_bs, sh.segs, sh.wpg);
    else
      return hipErrorInvalidValue;
  } else {
    hipLaunchKernelGGL((StreamKernel<HAS_ZP, TG, SPW, 4, false>), grid, block, lds, s, Ah, A, w.Bp,
                       w.Sp, Y, P, H, row_exp, w.col_exp, bias, m, n, k, w.log2_bs, sh.segs, sh.wpg);
  }
  return hipGetLastError();
}

template <bool HAS_ZP, int TG>
hipError_t LaunchStreamTG(const WeightView &w, int64_t M, const uint4 *Ah, const float *A, float *Y,
                          float *P, float *H, const int *row_exp, const float *bias,
                          const StreamShape &sh, hipStream_t s) {
  switch (sh.spw) {
  case 4: return LaunchStreamT<HAS_ZP, TG, 4>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  case 8: return LaunchStreamT<HAS_ZP, TG, 8>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  case 16: return LaunchStreamT<HAS_ZP, TG, 16>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  default: return hipErrorInvalidValue;
  }
}

template <bool HAS_ZP>
hipError_t LaunchStreamZp(const WeightView &w, int64_t M, const uint4 *Ah, const float *A, float *Y,
                          float *P, float *H, const int *row_exp, const float *bias,
                          const StreamShape &sh, hipStream_t s) {
  switch ((M + 15) / 16) {
  case 2: return LaunchStreamTG<HAS_ZP, 2>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  case 3: return LaunchStreamTG<HAS_ZP, 3>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  case 4: return LaunchStreamTG<HAS_ZP, 4>(w, M, Ah, A, Y, P, H, row_exp, bias, sh, s);
  default: return hipErrorInvalidValue;
  }
}

// Splits of a prefill launch: as many as keep the workgroups within one per
// CU when the tiles alone do not fill the chip (a second, partial wave costs
// a whole k-loop), at most kPrefillMaxSplits, each split at least 8 k-tiles.
// Up to 16 splits serve long rows on few tiles (against 8: K = 14336,
// N = 4096 at M = 65 / 128 38.1 / 40.4 -> 33.1 / 38.4 us; K = 14336,
// N = 2048 at M = 128 38.2 -> 31.8; K = 11008, N = 4096 at M = 65 33.0 ->
// 30.2; c4, c5 qkv and o unchanged). Whether the prefill kernel takes such
// rows at all is judged at 8 splits (UsePrefill, kPrefillCheckSplits).
constexpr int kPrefillMaxSplits = 16;
constexpr int kPrefillCheckSplits = 8;
inline int PrefillSplits(const WeightView &w, int64_t M) {
  const int64_t tiles = (M + kPTM - 1) / kPTM * ((w.N + kPTN - 1) / kPTN);
  const int ktiles = static_cast<int>(w.K / kBK);
  int64_t splits = std::max<int64_t>(1, w.num_cus / tiles);
  splits = std::min<int64_t>({splits, kPrefillMaxSplits, std::max(1, ktiles / 8)});
  const int per = static_cast<int>((ktiles + splits - 1) / splits);
  return (ktiles + per - 1) / per;
}

template <bool HAS_ZP, bool BS32>
hipError_t LaunchPrefillT(const WeightView &w, int64_t M, const uint4 *Ah, float *Y,
                          float *partials, int splits, hipStream_t s, float *H,
                          const int *row_exp, const float *bias) {
  const int ktiles = static_cast<int>(w.K / kBK);
  const int per = (ktiles + splits - 1) / splits;
  const int tiles = static_cast<int>((M + kPTM - 1) / kPTM * ((w.N + kPTN - 1) / kPTN));
  hipLaunchKernelGGL((PrefillKernel<HAS_ZP, BS32>), dim3(tiles * splits), dim3(kPThreads), kPLds, s, Ah,
                     w.Bp, w.Sp, Y, static_cast<int>(M), static_cast<int>(w.N),
                     static_cast<int>(w.K), w.log2_bs, per, partials, H, row_exp, w.col_exp, bias);
  return hipGetLastError();
}

// The plan-time re-layout (once per plan, see PrefillKernel).
__global__ __launch_bounds__(256) void RelayoutBKernel(const uint8_t *__restrict__ B,
                                                       uint32_t *__restrict__ Bp, int64_t N,
                                                       int64_t row_bytes, int64_t T,
                                                       int64_t words) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= words) return;
  const int j = static_cast<int>(idx & 3);
  const int l = static_cast<int>((idx >> 2) & 63);
  const int64_t gs = idx >> 8;
  const int64_t s = gs % T, g = gs / T;
  const int64_t n = 64 * g + 16 * j + (l & 15);
  Bp[idx] = n < N ? *reinterpret_cast<const uint32_t *>(B + n * row_bytes + 16 * s + 4 * (l >> 4))
                  : 0u;
}

__global__ __launch_bounds__(256) void RelayoutSKernel(const float *__restrict__ S,
                                                       const uint8_t *__restrict__ Z,
                                                       const int32_t *__restrict__ col_exp,
                                                       uint32_t *__restrict__ Sp, int64_t N,
                                                       int64_t nb, int64_t zp_row_bytes,
                                                       int64_t words) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= words) return;
  const int j = static_cast<int>(idx & 3);
  const int c = static_cast<int>((idx >> 2) & 15);
  const int64_t gb = idx >> 6;
  const int64_t b = gb % nb, g = gb / nb;
  const int64_t n = 64 * g + 16 * j + c;
  uint32_t v = 8u << 16;  // rows past N: scale 0
  if (n < N) {
    const _Float16 h = static_cast<_Float16>(__builtin_amdgcn_ldexpf(S[n * nb + b], col_exp[n]));
    const uint32_t z = Z != nullptr ? (Z[n * zp_row_bytes + (b >> 1)] >> (4 * (b & 1))) & 0xFu : 8u;
    v = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h)) | (z << 16);
  }
  Sp[idx] = v;
}

bool PrefillSupportsShape(const WeightView &w) {
  return w.Bp != nullptr && w.Sp != nullptr && (w.K % kBK) == 0 && w.block_size >= 32 &&
         (w.N % 4) == 0 && w.N < (int64_t{1} << 22) && w.K <= (int64_t{1} << 24);
}

bool PrefillSupportsM(const WeightView &w, int64_t M) {
  return M >= 1 && M <= (int64_t{1} << 30) && PrefillSupportsShape(w) &&
         (M + kPTM - 1) / kPTM * ((w.N + kPTN - 1) / kPTN) * kMaxSplits < (int64_t{1} << 31);
}

// Whether the streaming kernel's launch for M rows (M > 32) holds more than
// three workgroups per CU: each workgroup stages its K segment of every
// activation row, so with three or four 16-row token groups such launches
// fall behind the prefill kernel's 128 x 256 tiles, from 33 rows when K is
// split (the partial sums add their own traffic), from 49 when it is not.
// Measured on MI355X, us per call at M = 33 / 48 / 64, streaming against
// prefill: K = 5120, N = 13824 (1080 workgroups)
// 35.5 / 37.3 / 45.7 against 29.4 / 31.0 / 32.2; K = 3584, N = 18944 (2072)
// 29.5 / 32.5 / 45.8 against 28.5 / 30.0 / 31.7; K = 28672, N = 8192 (896)
// 74.1 / 75.7 / 89.5 against 68.7 / 71.7 / 74.5; K = 8192, N = 28672 (896)
// 68.3 / 70.4 / 83.2 against 66.9 / 65.4 / 73.8; K = 8192, N = 128256
// (4008) 257 / 264 / 317 against 242 / 248 / 253; K = 4096, N = 128256
// (2004, one segment) 127.8 / 129.6 / 155.3 against 130.9 / 134.3 / 137.7.
// Launches of
// up to 1.75 workgroups per CU stay faster streamed (K = 4096, N = 28672:
// 34.5 / 34.8 / 41.2 against 39.3 / 40.9 / 41.5; c2, c4, K = N = 8192,
// K = 14336, N = 4096 and K = 24576, N = 3072 by 15-40%).
bool StreamCrowded(const WeightView &w, int64_t M) {
  const StreamShape sh = PickStreamShape(w, 0, 0);
  const int64_t groups = (w.N + kSGroupRows - 1) / kSGroupRows;
  return M > 32 && sh.segs > 0 && (sh.segs > 1 || M > 48) &&
         groups * sh.segs > 3 * static_cast<int64_t>(w.num_cus);
}

// The prefill kernel serves the automatic GEMM path
// - when its 128 x 256 tiles alone fill at least one wave of CUs and the
//   last wave is at least half full: no split-K, one workgroup per CU (c5
//   qkv at M = 2048, 1.5 waves: 121.4 against GemmKernel's 130.6 us in one
//   process; a last wave below half stays with GemmKernel's smaller tiles);
// - when they do not fill one wave, with K split (PrefillSplits) as long as
//   each split keeps at least 12 k-tiles (shorter splits spend most of their
//   time in the prologue and the epilogue).
// Measured on MI355X (us per call, GemmKernel's best shape against the
// prefill kernel with PrefillSplits): M = 2048 c4, c5 o, gate+up, down
// 10-17% faster; M = 1024 c5 qkv 81.5 -> 61.8, o 61.8 -> 52.8, down
// 162.7 -> 125.9, c4 60.2 -> 52.6; M = 512 qkv 55.1 -> 46.3, down 96.4 ->
// 77.2, o and c4 within 3%; M = 256 gate+up 84.8 -> 63.8, qkv 34.6 -> about
// 32, down 56.8 -> 50.0; with fewer than 12 k-tiles per split (o and c4 at
// M <= 256, qkv at M = 128) GemmKernel's smaller tiles were 1-2 us faster;
// - from 33 rows where the streaming kernel's launch is crowded (above).
bool StreamSupportsM(const WeightView &w, int64_t M);

bool UsePrefill(const WeightView &w, int64_t M) {
  if (!PrefillSupportsM(w, M)) return false;
  // 17-64 rows the streaming kernel does not serve, on weights of 192 Mi
  // elements and more: the prefill kernel's tiles over GemmKernel's (K =
  // 29568, N = 8192 at M = 17 / 32 / 64: 66.5 / 67.2 / 74.1 against 80.2 /
  // 81.6 / 92.3 us; smaller weights stay: K = 20608, N = 2048 45 against 27).
  const bool large_unstreamed = M >= 17 && !StreamSupportsM(w, M) &&
                                w.K * w.N >= (int64_t{192} << 20);
  if (M < 65 && !StreamCrowded(w, M) && !large_unstreamed) return false;
  const int64_t tiles = (M + kPTM - 1) / kPTM * ((w.N + kPTN - 1) / kPTN);
  const int64_t cus = w.num_cus;
  if (tiles < cus) {
    const int64_t splits = std::min<int64_t>(cus / tiles, kPrefillCheckSplits);
    return w.K / kBK >= 12 * splits;
  }
  const int64_t last = tiles - (tiles - 1) / cus * cus;  // workgroups in the last wave
  return last * 2 >= cus;
}

size_t PrefillPartialBytes(const WeightView &w, int64_t M) {
  return static_cast<size_t>(PrefillSplits(w, M) - 1) * static_cast<size_t>(M) * w.N * 4;
}

bool StreamSupportsM(const WeightView &w, int64_t M) {
  if (M < 17 || M > 64 || !PrefillSupportsShape(w) || w.K > (int64_t{1} << 22)) return false;
  if (StreamCrowded(w, M)) return false;
  const StreamShape sh = PickStreamShape(w, 0, 0);
  return sh.segs > 0 && (!sh.ragged || M <= 32);  // shorter last segment: up to 32 rows
}

size_t StreamPartialBytes(const WeightView &w, int64_t M, int segs) {
  return static_cast<size_t>(std::max(segs, 1) - 1) * static_cast<size_t>(M) * w.N * 4;
}

} // namespace

size_t GemmWorkspaceBytes(const WeightView &w, int64_t M) {
  size_t partial = w.B != nullptr ? PartialBytes(w, M, PickShape(w, M)) : 0;
  if (PrefillSupportsM(w, M)) partial = std::max(partial, PrefillPartialBytes(w, M));
  if (StreamSupportsM(w, M))
    partial = std::max(partial, StreamPartialBytes(w, M, PickStreamShape(w, 0, 0).segs));
  return AImageBytes(w, M) + RowExpBytes(M) + partial;
}

bool StreamSupports(const WeightView &w, int64_t M) { return StreamSupportsM(w, M); }

size_t StreamWorkspaceBytes(const WeightView &w, int64_t M, int segs, int spw) {
  const StreamShape sh = PickStreamShape(w, segs, spw);
  return AImageBytes(w, M) + RowExpBytes(M) + StreamPartialBytes(w, M, sh.segs);
}

// The epilogue finishes fragments wave, wave + wpg, ... up to TG of them per
// wavefront, so it needs wpg >= 4 to reach all 4 TG; at most 8 wavefronts.
bool StreamShapeOk(const WeightView &w, int64_t M, int segs, int spw) {
  const StreamShape sh = PickStreamShape(w, segs, spw);
  // every step in a segment, no segment empty (the last may be shorter)
  const int64_t per = static_cast<int64_t>(sh.wpg) * sh.spw, T = w.K / 32;
  return StreamSupportsM(w, M) && sh.segs >= 1 && sh.segs <= kMaxSplits && sh.wpg >= 4 &&
         sh.wpg <= 8 && T % sh.spw == 0 && sh.segs * per >= T && (sh.segs - 1) * per < T;
}

// ConvertA (64-row tiling), the streaming kernel, and the ordered reduction
// of the segments' partial sums when K is split.
hipError_t LaunchStream(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                        hipStream_t s, float *H, const float *gamma, float eps, const float *bias,
                        int segs, int spw) {
  const StreamShape sh = PickStreamShape(w, segs, spw);
  if (!StreamShapeOk(w, M, segs, spw)) return hipErrorInvalidValue;
  uint4 *Ah = static_cast<uint4 *>(work);
  int *row_exp = reinterpret_cast<int *>(static_cast<char *>(work) + AImageBytes(w, M));
  float *P = reinterpret_cast<float *>(static_cast<char *>(work) + AImageBytes(w, M) +
                                       RowExpBytes(M));
  const bool cvt = StreamConverts(w, M, sh, gamma != nullptr);
  hipError_t e = hipSuccess;
  if (!cvt)
    e = gamma != nullptr
            ? LaunchConvertA<kSGroupRows, true>(w, M, A, Ah, row_exp, s, gamma, eps)
            : LaunchConvertA<kSGroupRows, false>(w, M, A, Ah, row_exp, s, nullptr, 0.0f);
  if (e != hipSuccess) return e;
  float *Hk = sh.segs == 1 ? H : nullptr;
  const float *bk = sh.segs == 1 ? bias : nullptr;
  const float *Ak = cvt ? A : nullptr;
  e = w.has_zp ? LaunchStreamZp<true>(w, M, Ah, Ak, Y, P, Hk, row_exp, bk, sh, s)
                      : LaunchStreamZp<false>(w, M, Ah, Ak, Y, P, Hk, row_exp, bk, sh, s);
  if (e != hipSuccess || sh.segs == 1) return e;
  return DispatchReduce(sh.segs - 1, Y, P, M * w.N, s, H,
                        std::make_integer_sequence<int, kMaxSplits - 1>{}, bias, w.N);
}

bool PrefillSupports(const WeightView &w, int64_t M) { return PrefillSupportsM(w, M); }


size_t PrefillLayoutBytes(const WeightView &w, size_t *sp_bytes) {
  const int64_t groups = (w.N + kPTN - 1) / kPTN * (kPTN / 64);
  const int64_t steps = w.K / 32;
  if (sp_bytes != nullptr) *sp_bytes = static_cast<size_t>(groups * w.nb * 256);
  return static_cast<size_t>(groups * steps * 1024);
}

bool PrefillLayoutWanted(const WeightView &w) {
  WeightView v = w;
  v.Bp = v.Sp = reinterpret_cast<const uint8_t *>(16);  // the shape checks only
  return PrefillSupportsShape(v) && (w.row_bytes % 16) == 0;
}

hipError_t LaunchPrefillRelayout(const WeightView &w, uint8_t *Bp, uint8_t *Sp, hipStream_t s) {
  size_t sp_bytes = 0;
  const size_t bp_bytes = PrefillLayoutBytes(w, &sp_bytes);
  const int64_t T = w.K / 32;
  const int64_t bw = static_cast<int64_t>(bp_bytes / 4), sw = static_cast<int64_t>(sp_bytes / 4);
  hipLaunchKernelGGL(RelayoutBKernel, dim3(static_cast<unsigned>((bw + 255) / 256)), dim3(256), 0,
                     s, w.B, reinterpret_cast<uint32_t *>(Bp), w.N, w.row_bytes, T, bw);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(RelayoutSKernel, dim3(static_cast<unsigned>((sw + 255) / 256)), dim3(256), 0,
                     s, w.scales, w.zp, w.col_exp, reinterpret_cast<uint32_t *>(Sp), w.N, w.nb,
                     w.zp_row_bytes, sw);
  return hipGetLastError();
}

// ConvertA, the prefill kernel, and the split reduction when K is split.
static hipError_t LaunchPrefillGemm(const WeightView &w, int64_t M, const float *A, float *Y,
                                    void *work, hipStream_t s, float *H, const float *gamma,
                                    float eps, const float *bias, int splits) {
  uint4 *Ah = static_cast<uint4 *>(work);
  int *row_exp = reinterpret_cast<int *>(static_cast<char *>(work) + AImageBytes(w, M));
  float *partials = reinterpret_cast<float *>(static_cast<char *>(work) + AImageBytes(w, M) +
                                              RowExpBytes(M));
  hipError_t e = gamma != nullptr
                     ? LaunchConvertA<kPTM, true>(w, M, A, Ah, row_exp, s, gamma, eps)
                     : LaunchConvertA<kPTM, false>(w, M, A, Ah, row_exp, s, nullptr, 0.0f);
  if (e != hipSuccess) return e;
  // One split: the kernel's stores apply the gate/up activation or add the
  // bias. Several: the ordered reduction does, after the partial sums.
  float *Hk = splits == 1 ? H : nullptr;
  const float *bk = splits == 1 ? bias : nullptr;
  const bool zp = w.has_zp != 0, bs32 = w.block_size == 32;
  if (zp)
    e = bs32 ? LaunchPrefillT<true, true>(w, M, Ah, Y, partials, splits, s, Hk, row_exp, bk)
             : LaunchPrefillT<true, false>(w, M, Ah, Y, partials, splits, s, Hk, row_exp, bk);
  else
    e = bs32 ? LaunchPrefillT<false, true>(w, M, Ah, Y, partials, splits, s, Hk, row_exp, bk)
             : LaunchPrefillT<false, false>(w, M, Ah, Y, partials, splits, s, Hk, row_exp, bk);
  if (e != hipSuccess || splits == 1) return e;
  return DispatchReduce(splits - 1, Y, partials, M * w.N, s, H,
                        std::make_integer_sequence<int, kMaxSplits - 1>{}, bias, w.N);
}

size_t GemmShapeWorkspaceBytes(const WeightView &w, int64_t M, int splits) {
  return AImageBytes(w, M) + RowExpBytes(M) + PartialBytes(w, M, MakeShape(w, 32, splits));
}

bool GemmSupports(const WeightView &w, int64_t M) {
  return GemmKernelSupports(w, M) || PrefillSupportsM(w, M);
}

bool GemmKernelSupports(const WeightView &w, int64_t M) {
  // Buffer offsets are 32-bit within one tile of 128 weight rows; up to 16
  // splits of the BM = 32 tiling must fit one grid.
  const int64_t tiles = ((M + 31) / 32) * ((w.N + kBN - 1) / kBN) * 16;
  return w.B != nullptr && M >= 1 && (w.K % kBK) == 0 && w.block_size >= 32 &&
         tiles < (int64_t{1} << 31) &&
         int64_t{kBN} * w.row_bytes < (int64_t{1} << 31) &&
         int64_t{kBN} * w.nb * 4 < (int64_t{1} << 31) && (w.row_bytes % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(w.B) % 16) == 0 && M <= (int64_t{1} << 30) &&
         w.N <= (int64_t{1} << 30) && w.K <= (int64_t{1} << 24);
}

hipError_t LaunchPrefill(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                         hipStream_t s, float *H, const float *gamma, float eps, const float *bias,
                         bool *bias_done) {
  if (bias_done != nullptr) *bias_done = bias != nullptr;
  return LaunchPrefillGemm(w, M, A, Y, work, s, H, gamma, eps, bias, PrefillSplits(w, M));
}

hipError_t LaunchGemmShape(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                           hipStream_t s, int bm, int splits, float *H, const float *gamma,
                           float eps) {
  if (bm == kPrefillTileCode) {
    if (!PrefillSupportsShape(w)) return hipErrorInvalidValue;
    const int ktiles = static_cast<int>(w.K / kBK);
    splits = std::max(1, std::min({splits, ktiles, kMaxSplits}));
    const int per = (ktiles + splits - 1) / splits;
    return LaunchPrefillGemm(w, M, A, Y, work, s, H, gamma, eps, nullptr, (ktiles + per - 1) / per);
  }
  if (w.B == nullptr) return hipErrorInvalidValue;  // GemmKernel reads the original layout
  Shape sh = PickShape(w, M);
  if (bm > 0) sh = MakeShape(w, bm, splits > 0 ? splits : 1);
  switch (sh.bm) {
  case 32: return LaunchBM<32>(w, M, A, Y, work, sh, s, H, gamma, eps);
  case 64: return LaunchBM<64>(w, M, A, Y, work, sh, s, H, gamma, eps);
  case 128: return LaunchBM<128>(w, M, A, Y, work, sh, s, H, gamma, eps);
  default: return hipErrorInvalidValue;
  }
}

hipError_t LaunchGemm(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                      hipStream_t s, float *H, const float *gamma, float eps, const float *bias,
                      bool *bias_done) {
  if (bias_done != nullptr) *bias_done = false;
  if (StreamSupportsM(w, M)) {
    if (bias_done != nullptr) *bias_done = bias != nullptr;
    return LaunchStream(w, M, A, Y, work, s, H, gamma, eps, bias, 0, 0);
  }
  // A compact plan (no original layout) always takes the prefill kernel.
  if (UsePrefill(w, M) || w.B == nullptr) {
    if (bias_done != nullptr) *bias_done = bias != nullptr;
    return LaunchPrefillGemm(w, M, A, Y, work, s, H, gamma, eps, bias, PrefillSplits(w, M));
  }
  return LaunchGemmShape(w, M, A, Y, work, s, 0, 0, H, gamma, eps);
}

bool GemmUsesPrefill(const WeightView &w, int64_t M) { return UsePrefill(w, M) || w.B == nullptr; }

bool GemmUsesStream(const WeightView &w, int64_t M) { return StreamSupportsM(w, M); }

} // namespace mnb
