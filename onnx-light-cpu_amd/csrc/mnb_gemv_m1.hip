// Decode GEMV for a single activation row (M = 1): the HBM-bound hot path.
//
// Role in the reference: the roadmap's `int4_gemv`
// (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-218): fp32
// accumulation, weights never expanded, each weight byte streamed once.
//
// Mapping. A workgroup owns a band of G consecutive weight rows; wavefront w
// owns band rows [w R, w R + R). Short rows (K <= 4096) use several 4-wave
// workgroups per CU, long rows one workgroup of up to 16 wavefronts per CU
// (see PickShape). Lane l takes the 16-byte chunks c = l + 64 i (i < CPL) of
// each row, so every load instruction of a wavefront reads 1 KiB of one row,
// coalesced. A chunk holds 32 nibbles k = 32c .. 32c+31, all in one
// quantization block (block_size >= 32).
//
// Order of work, chosen so that neither HBM nor the arithmetic waits on the
// other:
//  1. the workgroup issues its staging loads: A, and each wavefront the scale
//     and zero point of every (row, block) of its rows;
//  2. every wavefront issues the first few non-temporal buffer loads of its
//     rows' weights (row offsets are wave-uniform SGPRs); the rest are issued
//     one by one behind the dot products of step 4, a fixed number ahead, so
//     that a wavefront stalled at issue (the memory pipeline full) still has
//     arrived data to compute on: with every load issued up front, waves
//     spent up to 5 us of a 7.6 us launch issuing, and the last ones did all
//     their arithmetic after HBM had gone idle (per-wave timestamps);
//  3. the staged values go to LDS as they return (loads complete in issue
//     order, so this never waits behind the weights): A as swizzled float4
//     chunks with the per-chunk sums asum = sum_j a_j, and the pairs
//     (scale * 2^24, zp * 2^-24), so the inner loop does no small global
//     loads;
//  4. one barrier, then each wavefront computes its rows as their weights
//     arrive and reduces them across lanes.
// When the grid is one workgroup per CU, more than half of the LDS is
// requested so that the dispatcher places exactly one on each CU.
//
// Arithmetic. v_fma_mix_f32 multiplies an fp32 activation by an fp16 operand
// taken straight from one half of a register. A packed word w holds nibbles
// 0..7 (k order); masking w and w >> 8 with 0x000F000F and 0x00F000F0 leaves
// two nibbles per mask in the two halves as the exact fp16 subnormals
// q * 2^-24 (bits 0-3 of a half) or q * 2^-20 (bits 4-7). The LDS copy of A
// holds a_j / 16 at odd j (exact), so every product is a_j q_j 2^-24 and per
// chunk
//   d  = sum_j a_j q_j 2^-24
//   y += (scale 2^24) * (d - (zp 2^-24) * asum)
// costs five bit operations per eight nibbles plus one FMA per nibble, with
// no per-nibble conversion or zero-point subtraction; products are exact.
// This relies on fp16 subnormal inputs being kept (the gfx950 HIP default
// FP16 denormal mode); the parity tests would see every product vanish
// otherwise.
//
// Reduction per row: 4 DPP steps give every lane its 16-lane row sum, 4
// readlanes add the rows in a fixed order; lane r stores row r of the wave.
#include "mnb_decode_common.h"

#include <algorithm>

namespace mnb {
namespace m1 {

using namespace dec;

constexpr int kMaxWaves = 16;             // 1024 threads per workgroup
constexpr size_t kLdsLimit = 150 * 1024;  // of the 160 KiB per CU
constexpr size_t kOnePerCu = 81 * 1024;   // more than half: one workgroup per CU
constexpr int kAPasses = 4;               // A float4 per thread staged ahead of the weights
constexpr int kPPasses = 2;               // (scale, zp) work items per thread ahead of the weights
// Weight loads kept in flight per wavefront behind the dot products: 4, or 2
// when a wavefront owns one long row (interleaved medians on MI355X, window
// 2/4/6/all: c2 8.09/7.99/8.33/8.40 us, c3 9.82/10.22/11.40/11.85 us).
template <int R>
constexpr int M1Window() { return R == 1 ? 2 : 4; }

// sum_j a'[j] * f16-subnormal masks of one chunk = sum_j a_j q_j 2^-24, where
// a' holds a_j / 16 at odd j (k order inside the chunk).
__device__ __forceinline__ float DotChunk(const float *a, const uint4 &w4) {
  const uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t w = words[t];
    const uint32_t w8 = w >> 8;
    const uint32_t h0 = w & 0x000F000Fu;   // nibbles 0 | 4, as q * 2^-24
    const uint32_t h1 = w & 0x00F000F0u;   // nibbles 1 | 5, as q * 2^-20
    const uint32_t h2 = w8 & 0x000F000Fu;  // nibbles 2 | 6, as q * 2^-24
    const uint32_t h3 = w8 & 0x00F000F0u;  // nibbles 3 | 7, as q * 2^-20
    if (t == 0) {
      lo = MixLo0(a[0], h0);
      hi = MixHi0(a[4], h0);
    } else {
      MixLo(lo, a[8 * t + 0], h0);
      MixHi(hi, a[8 * t + 4], h0);
    }
    MixLo(lo, a[8 * t + 1], h1);
    MixHi(hi, a[8 * t + 5], h1);
    MixLo(lo, a[8 * t + 2], h2);
    MixHi(hi, a[8 * t + 6], h2);
    MixLo(lo, a[8 * t + 3], h3);
    MixHi(hi, a[8 * t + 7], h3);
  }
  return lo + hi;
}

// LDS layout of one workgroup: A as nchunks * 8 swizzled float4 plus one
// spare float4, the chunk sums plus one spare float, then per wavefront its
// R * nb pairs (scale, zp), row-major, plus 4 spare pairs. Float4 v of chunk
// c sits at c * 8 + (v ^ ((c ^ c >> 3) & 7)): in the dot products lanes l
// and l + 8 read chunks 8 * 128 bytes apart, which an XOR by c & 7 alone
// left in the same banks (at c3 921,088 bank-conflict cycles per dispatch
// against 3,584, and 9.45 against 9.04 us per call). Staging lanes with
// nothing to store write to the spares, so the staging code has no branches
// (a branch between a load and its use lets the compiler sink the load below
// the weight loads). A wavefront writes and reads only its own pairs: LDS
// operations of one wavefront execute in order, so the pairs need no
// workgroup barrier and the barrier waits only for A.
__host__ __device__ inline size_t AsumOffsetF4(int nchunks) { return static_cast<size_t>(nchunks) * 8 + 1; }
__host__ __device__ inline size_t PairsOffsetF2(int nchunks) {
  return (AsumOffsetF4(nchunks) * 16 + (static_cast<size_t>(nchunks) + 1) * 4 + 7) / 8;
}
// Byte offset of the 16 per-wavefront partial sums of squares (RMSNorm).
__host__ __device__ inline size_t SqOffsetBytes(int nchunks, int wave_rows, int64_t nb) {
  return (PairsOffsetF2(nchunks) + static_cast<size_t>(wave_rows) * nb + 4) * 8;
}
inline size_t LdsBytes(int nchunks, int wave_rows, int64_t nb) {
  return SqOffsetBytes(nchunks, wave_rows, nb) + 16 * sizeof(float);
}

// A float4 f of the chunk layout: stored swizzled, odd k divided by 16, the
// 8-lane DPP sum of the original values gives the chunk sum. total is a
// multiple of 8, so the 8 lanes of a chunk are all valid or all clamped;
// clamped lanes write to the spare slots.
// With RMS (RMSNorm fused into the input): the stored value is x * gamma and
// sq accumulates x * x of the valid lanes.
template <bool RMS>
__device__ __forceinline__ void StoreA(float4 *lds4, float *asum_lds, int nchunks, int f, int total,
                                       float4 t, float4 g, float &sq) {
  const int c = f >> 3, v = f & 7;
  const bool valid = f < total;
  if constexpr (RMS) {
    const float q = (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
    sq += valid ? q : 0.0f;
    t = make_float4(t.x * g.x, t.y * g.y, t.z * g.z, t.w * g.w);
  }
  float sum = (t.x + t.y) + (t.z + t.w);
  sum = DppAdd<0xB1>(sum);   // quad_perm [1,0,3,2]
  sum = DppAdd<0x4E>(sum);   // quad_perm [2,3,0,1]
  sum = DppAdd<0x141>(sum);  // row_half_mirror: every lane holds its 8-lane sum
  t.y *= 0.0625f;
  t.w *= 0.0625f;
  lds4[valid ? c * 8 + (v ^ ((c ^ (c >> 3)) & 7)) : nchunks * 8] = t;
  asum_lds[valid && v == 0 ? c : nchunks] = sum;
}

template <int CPL, int R, bool FULL, bool HAS_ZP, int PW, bool RMS>
__global__ __launch_bounds__(1024) void GemvM1Kernel(const float *__restrict__ A,
                                                     const uint8_t *__restrict__ B,
                                                     const float *__restrict__ S,
                                                     const uint8_t *__restrict__ Z,
                                                     float *__restrict__ Y, int K, int N, int nb,
                                                     int chunk_shift, int row_bytes,
                                                     int zp_row_bytes, int G,
                                                     float *__restrict__ H,
                                                     const float *__restrict__ gamma, float eps,
                                                     const float *__restrict__ bias) {
  extern __shared__ float4 lds4[];
  const int nchunks = K >> 5;
  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int row0 = blockIdx.x * G;    // first row of the band
  const int rows = min(G, N - row0);  // rows in the band
  const int wr0 = wave * R;           // first band row of this wavefront

  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(B), 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(S), 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(HAS_ZP ? Z : B), 0, 0x7FFFFFFF, 0x00020000);

  float *asum_lds = reinterpret_cast<float *>(lds4 + AsumOffsetF4(nchunks));
  float2 *pair_lds = reinterpret_cast<float2 *>(lds4) + PairsOffsetF2(nchunks);
  float2 *wpairs = pair_lds + wr0 * nb;  // this wavefront's pairs
  const int spare = blockDim.x / 64 * R * nb;
  const float4 *src = reinterpret_cast<const float4 *>(A);
  const int total = nchunks * 8;      // float4 of A
  const int nitems = R * nb / PW;     // (scale, zp) work items of this wavefront
  const int last_row = row0 + rows - 1;
  const float rnb = 1.0f / static_cast<float>(nb);

  // 1. the first staging loads (A, scales, zero points) go out first: loads
  //    complete in issue order, so staging never waits behind the weights.
  // All loads below are unconditional with clamped addresses: a branch
  // around a load makes the compiler wait for it at the join.
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, 0x7FFFFFFF, 0x00020000);
  float4 ta[kAPasses], tg[kAPasses];
  const __amdgpu_buffer_rsrc_t rgm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(RMS ? gamma : A), 0, 0x7FFFFFFF, 0x00020000);
#pragma unroll
  for (int p = 0; p < kAPasses; ++p) {
    ta[p] = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(ra, min(nthreads * p + tid, total - 1) * 16, 0, 0));
    if constexpr (RMS)
      tg[p] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rgm, min(nthreads * p + tid, total - 1) * 16, 0, 0));
  }
  // (scale, zp): with one row per wavefront (long rows), each lane loads the
  // scale and zero-point byte of its own chunks straight into registers;
  // otherwise the wavefront stages its rows' pairs in LDS (fewer load
  // instructions when a wavefront owns several short rows). Interleaved
  // medians, direct vs staged: c3 8.9 vs 9.8 us, c5 down 8.4 vs 8.7 us, c2
  // 7.92 vs 7.86 us, c5 gate+up 13.1 vs 12.8 us.
  constexpr bool kDirect = R == 1;
  PairItem<PW, HAS_ZP> pi[kDirect ? 1 : kPPasses];
  float dsc[CPL];
  uint32_t dzb[CPL];
  if constexpr (kDirect) {
    const int row = __builtin_amdgcn_readfirstlane(row0 + min(wr0, rows - 1));
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int blk = (FULL ? lane + 64 * i : min(lane + 64 * i, nchunks - 1)) >> chunk_shift;
      dsc[i] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rsc, blk * 4, row * nb * 4, 0));
      dzb[i] = HAS_ZP ? __builtin_amdgcn_raw_buffer_load_b8(rz, blk >> 1, row * zp_row_bytes, 0)
                      : 0x88u;
    }
  } else {
#pragma unroll
    for (int q = 0; q < kPPasses; ++q)
      pi[q].Load(64 * q + lane, nitems, nb, rnb, row0 + wr0, last_row, zp_row_bytes, rsc, rz);
  }

  // Keep the issue order: the scheduler must not sink the staging loads below
  // the weight loads (completion is in issue order).
  __builtin_amdgcn_sched_barrier(0);

  // 2. then the first kWin weight loads of this wavefront (rows past the band
  //    re-read the band's last row; their results are not stored). Load j is
  //    chunk i = j / R of row r = j % R, the order the dot products consume
  //    them; the rest are issued one by one behind the dot products (step 4).
  constexpr int kLoads = R * CPL;
  constexpr int kWin = M1Window<R>() < kLoads ? M1Window<R>() : kLoads;
  uint4 w[R][CPL];
  int row_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    row_off[r] = __builtin_amdgcn_readfirstlane(row0 + min(wr0 + r, rows - 1)) * row_bytes;
  auto issue = [&](int j) __attribute__((always_inline)) {
    const int i = j / R, r = j % R;
    const int c = FULL ? lane + 64 * i : min(lane + 64 * i, nchunks - 1);
    w[r][i] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, c * 16, row_off[r], kNonTemporal));
  };
#pragma unroll
  for (int j = 0; j < kWin; ++j) issue(j);

  __builtin_amdgcn_sched_barrier(0);

  // 3. LDS stores of A; further passes (long K) load and store behind the
  //    weights.
  float sq = 0.0f;
#pragma unroll
  for (int p = 0; p < kAPasses; ++p)
    StoreA<RMS>(lds4, asum_lds, nchunks, nthreads * p + tid, total, ta[p], tg[p], sq);
  for (int f0 = nthreads * kAPasses; f0 < total; f0 += nthreads) {
    const int f = f0 + tid;
    const float4 g = RMS ? reinterpret_cast<const float4 *>(gamma)[min(f, total - 1)] : float4{};
    StoreA<RMS>(lds4, asum_lds, nchunks, f, total, src[min(f, total - 1)], g, sq);
  }
  float *sq_lds = reinterpret_cast<float *>(reinterpret_cast<char *>(lds4) +
                                            SqOffsetBytes(nchunks, nthreads / 64 * R, nb));
  if constexpr (RMS) {
    const float wsq = WaveTotal(sq);
    if (lane == 0) sq_lds[wave] = wsq;
  }
  __syncthreads();
  // RMSNorm: 1 / sqrt(mean(x^2) + eps), applied to the row totals (the staged
  // A already carries gamma).
  float inv_rms = 1.0f;
  if constexpr (RMS) {
    float tot = 0.0f;
    for (int w = 0; w < nthreads / 64; ++w) tot += sq_lds[w];
    inv_rms = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
  }

  // The wavefront's own pairs: stored after the barrier, which therefore
  // never waits for the (cold) scales.
  if constexpr (!kDirect) {
#pragma unroll
    for (int q = 0; q < kPPasses; ++q) pi[q].Store(wpairs, spare - wr0 * nb);
    for (int i0 = 64 * kPPasses; i0 < nitems; i0 += 64) {
      PairItem<PW, HAS_ZP> it;
      it.Load(i0 + lane, nitems, nb, rnb, row0 + wr0, last_row, zp_row_bytes, rsc, rz);
      it.Store(wpairs, spare - wr0 * nb);
    }
  }

  // 4. dot products of this wavefront's rows. LDS addresses are a per-lane
  //    base plus compile-time offsets: chunk c = lane + 64 i sits 8192 i bytes
  //    after chunk lane, and its swizzle ((c ^ c >> 3) & 7) is lane's (64 i
  //    leaves bits 0-5 alone).
  const float4 *ab = lds4 + lane * 8;
  const int sw = (lane ^ (lane >> 3)) & 7;
  const float2 *pr = wpairs;
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
        const float4 t = ab[512 * i + (v ^ sw)];
        a[4 * v] = t.x;
        a[4 * v + 1] = t.y;
        a[4 * v + 2] = t.z;
        a[4 * v + 3] = t.w;
      }
      const float asum = asum_lds[c];
      const int blk = c >> chunk_shift;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (wr0 + r < rows) {  // wave-uniform
          const float d = DotChunk(a, w[r][i]);
          float2 sz;
          if constexpr (kDirect) {
            sz.x = dsc[i] * 16777216.f;  // scale * 2^24 (exact)
            sz.y = static_cast<float>((dzb[i] >> ((blk & 1) * 4)) & 0xFu) * 5.9604644775390625e-8f;
          } else {
            sz = pr[r * nb + blk];
          }
          acc[r] = fmaf(sz.x, fmaf(-sz.y, asum, d), acc[r]);
        }
        // The load kWin places later in the order, issued here, behind this
        // dot product: a wavefront whose loads cannot issue (the memory
        // pipeline is full) is then still doing arithmetic on data that has
        // arrived, instead of stalling in front of all of it.
        if (i * R + r + kWin < kLoads) issue(i * R + r + kWin);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (i * R + r + kWin < kLoads) issue(i * R + r + kWin);
    }
  }

  // 5. one total per row; lane r stores row r
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float t = WaveTotal(acc[r]);
    mine = lane == r ? t : mine;
  }
  if constexpr (RMS) mine *= inv_rms;
  if constexpr (!RMS) {
    // A non-finite activation: the reference's +-inf / NaN (see ReferenceRowDot).
    if (lane < R && wr0 + lane < rows && !__builtin_isfinite(mine)) {
      const size_t n = static_cast<size_t>(row0 + wr0 + lane);
      mine = ReferenceRowDotPlain(A, K, chunk_shift + 5, B + n * row_bytes, S + n * nb,
                                  HAS_ZP ? Z + n * zp_row_bytes : nullptr);
    }
  }
  if (H != nullptr) {
    // Gate/up pairs: band row 2n is a gate, 2n + 1 its up (R and G even, so a
    // pair never straddles wavefronts or bands).
    const float other = PairSwap(mine);
    if (lane < R && (lane & 1) == 0 && wr0 + lane < rows)
      H[(row0 + wr0 + lane) >> 1] = SiluMul(mine, other);
  } else if (lane < R && wr0 + lane < rows) {
    if (bias != nullptr) mine += bias[row0 + wr0 + lane];  // MatMulNBits input 5
    Y[row0 + wr0 + lane] = mine;
  }
}

struct Shape {
  int G, R, waves, grid;
  size_t lds;
};

// Band rows per workgroup G and rows per wavefront R (a power of two), from
// measured sweeps on MI355X (c1, c2, c3 and the c5 projections):
//  - short rows (CPL <= 2): workgroups of at most 4 wavefronts x 4 rows, k
//    workgroups per CU with k = ceil(rows per CU / 16), so that every CU gets
//    the same number of rows and several independent workgroups (one
//    workgroup's staging and barrier overlap another's arithmetic); when
//    that gives 3 wavefronts per workgroup, k + 1 (qkv: 12 x 4 6.4 us,
//    8 x 2 5.2 us). Interleaved medians put c2's 14 x 4 within 2 % of the
//    best of 8 x 2 and 16 x 4, whose order changes from box to box;
//  - long rows: one workgroup of up to 16 wavefronts per CU owning the CU's
//    whole band (A, up to 64 KiB, is staged once per CU).
// Both keep the LDS within kLdsLimit, shrinking G (more rounds) if needed.
inline int RMax(int cpl) { return cpl <= 2 ? 8 : (cpl <= 4 ? 4 : 2); }

inline int RowsPerWave(int G) {
  const int need = (G + kMaxWaves - 1) / kMaxWaves;
  int R = 1;
  while (R < need) R *= 2;
  return R;
}

inline Shape PickShape(const WeightView &w, int cpl, int G, int R) {
  const int nchunks = static_cast<int>(w.K / 32);
  const int64_t cus = w.num_cus;
  const int rows_per_cu = static_cast<int>((w.N + cus - 1) / cus);
  Shape sh{};
  if (G <= 0) {
    if (cpl <= 2) {
      auto rows_per_wave = [](int g) { return g > 8 ? 4 : (g > 4 ? 2 : 1); };
      int k = (rows_per_cu + 15) / 16;
      G = (rows_per_cu + k - 1) / k;
      const int r0 = R > 0 ? R : rows_per_wave(G);
      if ((G + r0 - 1) / r0 == 3) {
        ++k;
        G = (rows_per_cu + k - 1) / k;
      }
      if (R <= 0) R = rows_per_wave(G);
    } else {
      G = std::min(rows_per_cu, kMaxWaves * RMax(cpl));
    }
    // Pair space is allocated for waves * R rows.
    auto lds_for = [&](int g) {
      const int r = R > 0 ? R : RowsPerWave(g);
      return LdsBytes(nchunks, (g + r - 1) / r * r, w.nb);
    };
    while (G > 1 && lds_for(G) > kLdsLimit) G = (G + 1) / 2;
  }
  if (R <= 0) R = RowsPerWave(G);
  sh.G = G;
  sh.R = R;
  sh.waves = (G + R - 1) / R;
  sh.grid = static_cast<int>((w.N + G - 1) / G);
  sh.lds = LdsBytes(nchunks, sh.waves * R, w.nb);
  if (sh.grid <= w.num_cus) sh.lds = std::max(sh.lds, kOnePerCu);
  return sh;
}

template <int CPL, int R, bool HAS_ZP>
hipError_t LaunchT(const WeightView &w, const float *A, float *Y, hipStream_t s, const Shape &sh,
                   float *H, const float *gamma, float eps, const float *bias) {
  const bool full = (w.K / 32) == 64 * CPL;
  const bool quads = (w.nb % 4) == 0;
  const dim3 grid(static_cast<unsigned>(sh.grid)), block(static_cast<unsigned>(sh.waves * 64));
  const int K = static_cast<int>(w.K), N = static_cast<int>(w.N), nb = static_cast<int>(w.nb);
  const int cs = w.log2_bs - 5, rb = static_cast<int>(w.row_bytes);
  const int zb = static_cast<int>(w.zp_row_bytes);
#define MNB_M1_LAUNCH(FULLV, PWV)                                                                  \
  if (gamma != nullptr)                                                                            \
    hipLaunchKernelGGL((GemvM1Kernel<CPL, R, FULLV, HAS_ZP, PWV, true>), grid, block, sh.lds, s,  \
                       A, w.B, w.scales, w.zp, Y, K, N, nb, cs, rb, zb, sh.G, H, gamma, eps, bias);\
  else                                                                                             \
    hipLaunchKernelGGL((GemvM1Kernel<CPL, R, FULLV, HAS_ZP, PWV, false>), grid, block, sh.lds, s, \
                       A, w.B, w.scales, w.zp, Y, K, N, nb, cs, rb, zb, sh.G, H, gamma, eps, bias)
  if (full) {
    if (quads) MNB_M1_LAUNCH(true, 4);
    else MNB_M1_LAUNCH(true, 1);
  } else {
    if (quads) MNB_M1_LAUNCH(false, 4);
    else MNB_M1_LAUNCH(false, 1);
  }
#undef MNB_M1_LAUNCH
  return hipGetLastError();
}

template <int CPL, bool HAS_ZP>
hipError_t LaunchC(const WeightView &w, const float *A, float *Y, hipStream_t s, int G, int R,
                   float *H, const float *gamma, float eps, const float *bias) {
  Shape sh = PickShape(w, CPL, G, R);
  if (H != nullptr && (sh.R < 2 || (sh.G & 1) != 0)) {
    // Gate/up epilogue: an even number of rows per wavefront and per band.
    const int r2 = std::max(sh.R, 2);
    sh = PickShape(w, CPL, sh.G + (sh.G & 1), r2);
  }
  // Rows per wavefront are capped so that R * CPL weight chunks stay within
  // 16 VGPR quads (no spills under the 1024-thread launch bound).
  constexpr int kRMax = CPL <= 2 ? 8 : (CPL <= 4 ? 4 : 2);
  if (sh.waves < 1 || sh.waves > kMaxWaves || sh.lds > 160 * 1024 || sh.R > kRMax)
    return hipErrorInvalidValue;
  switch (sh.R) {
  case 1: return LaunchT<CPL, 1, HAS_ZP>(w, A, Y, s, sh, H, gamma, eps, bias);
  case 2: return LaunchT<CPL, 2, HAS_ZP>(w, A, Y, s, sh, H, gamma, eps, bias);
  case 4:
    if constexpr (kRMax >= 4) return LaunchT<CPL, 4, HAS_ZP>(w, A, Y, s, sh, H, gamma, eps, bias);
    return hipErrorInvalidValue;
  case 8:
    if constexpr (kRMax >= 8) return LaunchT<CPL, 8, HAS_ZP>(w, A, Y, s, sh, H, gamma, eps, bias);
    return hipErrorInvalidValue;
  default: return hipErrorInvalidValue;
  }
}

template <bool HAS_ZP>
hipError_t LaunchZ(const WeightView &w, const float *A, float *Y, hipStream_t s, int G, int R,
                   float *H, const float *gamma, float eps, const float *bias) {
  switch ((w.K / 32 + 63) / 64) {
  case 1: return LaunchC<1, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 2: return LaunchC<2, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 3: return LaunchC<3, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 4: return LaunchC<4, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 5: return LaunchC<5, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 6: return LaunchC<6, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  case 7: return LaunchC<7, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  default: return LaunchC<8, HAS_ZP>(w, A, Y, s, G, R, H, gamma, eps, bias);
  }
}

} // namespace m1

bool GemvM1Supports(const WeightView &w) {
  // Buffer offsets are 32-bit: every byte of B, scales and zero points must
  // be addressable below 2^31. K <= 16384 keeps a row within 8 chunks per
  // lane (the largest CPL instantiated) and A within 64 KiB of LDS; the
  // 16-byte scale loads need 16-byte aligned scales, the 2-byte zero-point
  // loads 2-byte aligned zero points.
  return w.B != nullptr && (w.K % 32) == 0 && w.K <= 16384 && w.block_size >= 32 &&
         (w.row_bytes % 16) == 0 && (reinterpret_cast<uintptr_t>(w.B) % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(w.scales) % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(w.zp) % 2) == 0 &&
         w.row_bytes * w.N < (int64_t{1} << 31) && w.nb * 4 * w.N < (int64_t{1} << 31);
}

hipError_t LaunchGemvM1(const WeightView &w, const float *A, float *Y, hipStream_t s,
                        int band_rows, int rows_per_wave, float *H, const float *gamma,
                        float eps, const float *bias) {
  return w.zp ? m1::LaunchZ<true>(w, A, Y, s, band_rows, rows_per_wave, H, gamma, eps, bias)
              : m1::LaunchZ<false>(w, A, Y, s, band_rows, rows_per_wave, H, gamma, eps, bias);
}

} // namespace mnb
