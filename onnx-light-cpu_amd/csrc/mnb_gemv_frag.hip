// Decode GEMV for 1 <= M <= 4 activation rows on fp16 MFMA, streaming the
// plan's fragment-ordered weights.
//
// Role in the reference: the roadmap's `int4_gemv` / `int4_small_m` decode
// side (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-221): fp32
// accumulation, weights never expanded, each weight byte streamed once; the
// fp32 semantics are those of the reference engine's skinny-M product
// (onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258).
//
// Why the matrix cores at M = 1. GemvM1Kernel spends one v_fma_mix_f32 per
// nibble plus the bit operations that expose it, 1.6 VALU per nibble and 667
// per wavefront at the c2 shape: on every CU the vector ALUs are busy for
// about 60% of the time the weights take to stream. Here the products go to
// the matrix cores, idle otherwise. Masking a packed word w with 0x000F000F
// and 0x00F000F0, and w >> 8 with the same, leaves its eight nibbles as the
// fp16 subnormals q 2^-24 (even k) and 16 q 2^-24 (odd k): exactly one lane's
// B operand of v_mfma_f32_16x16x32_f16 (8 k values, in the order
// [0,4,1,5,2,6,3,7]). That is 5 VALU per 8 nibbles. On MI355X every single
// product is exact (every normal fp16 a against every q 2^-24 and 16 q 2^-24),
// but the matrix core adds a step's products after aligning them to the
// largest one's nominal exponent, and a subnormal's nominal exponent is -14
// whatever its leading bit: products of the nibbles in the low four mantissa
// bits (even k) keep up to 10 fewer bits of that window. Measured on random
// operands spanning five binades: 0.12% of the sums inexact, by up to 2.3e-6
// of sum |a b|; with the nibbles in bits 4-7 (odd k) or with normal operands,
// none. Per output the error is at most about 2^-22 of sum_k |a_k w_k|
// (2.5e-7 measured at c2); moving the even nibbles to bits 4-7 as well
// (1.5e-8) takes two more VALU per word and 3% more time at c2.
//
// Activations. Each wavefront first turns its own part of the fp32 rows (the
// 256-k units of its steps) into LDS MFMA A operands. Per unit u and row m a
// power of two 2^e brings the largest magnitude into [2^14, 2^15) (exact), and
// each scaled value x is split into three fp16 terms, t0 = fp16(x), t1 =
// fp16(x - t0), t2 = fp16(x - t0 - t1): the differences are exact in fp32 and
// three 11-bit significands hold x's 24 bits, so x = t0 + t1 + t2 exactly for
// every x not far below the unit's largest magnitude (absolute error at most
// 2^-25, i.e. 2^-39 of it, for the rest). A-operand row 4 m + t holds term t
// of activation row m (rows 4 m + 3 repeat term 0, rows of m >= M repeat row
// 0; both are ignored), so one MFMA multiplies all terms of all rows and
// lanes 16 m .. 16 m + 15 of its result hold row m's three partial sums of the
// same 16 weight rows. Values at odd k are stored divided by 16 (exact),
// undoing the odd nibbles' factor. Per quantization block b and row m the
// wavefront also keeps S = 2^-24 sum_k x_k over the block, and per unit e
// (scalars at M = 1, LDS tables otherwise). Per block, weight row and
// activation row:
//   y += 2^(24 - e) scale (C_0 + C_1 + C_2 - zp S)
// with the 2^(24 - e) applied once per unit (exact). No workgroup barrier
// precedes the stream: a wavefront only reads the operands it wrote itself.
//
// Mapping. One workgroup per group g of 64 weight rows and the whole of K (or,
// for rows too long for one workgroup, one per group and K segment: see K
// segments below); its wavefront w takes SPW consecutive 32-k steps (whole
// units and blocks), i.e.
// SPW records of the plan's fragment-ordered copy Bp (1 KiB each: lane l holds
// the words of rows 64 g + 16 j + (l & 15), j = 0..3, at k = 32 s + 8 (l >> 4),
// the B operands of four 16-row slices), with 16-byte non-temporal loads kept
// WIN steps ahead; the activation loads go first, then the first WIN weight
// records, then the staging arithmetic. Block scales and zero points come
// from the plan's decode re-layout (Sd, Zd: per group and block, lane c's
// float4 holds the scales of rows 64 g + 16 j + c, byte j of its word the zero
// points). The wavefronts' row sums meet in LDS and are added in wavefront
// order by one thread per output. No workspace; results do not depend on
// scheduling.
//
// K segments. Rows longer than 16 wavefronts of 32 steps (K > 16384) do not
// fit one workgroup, and GemvM1Kernel (whose activation row must fit its LDS)
// does not take them either. For up to 2 rows (and for 2 to 4 rows of
// K >= 5120 on narrow weights, below) the launch splits K into
// `segs` segments of whole units, all of one length but the last (shorter
// when the units do not divide evenly: its wavefronts past the row's end read
// only zeros beyond the weights' buffers and add nothing): workgroup
// (g, seg) stages and streams only its segment (its LDS image indexed from
// the segment's first step), segment 0 writes Y and segment s > 0 the
// partial sums P[s - 1], and
// SumPartialsKernel adds them in segment order (with the bias). A row with a
// non-finite activation gets, per segment, the reference's sum over that
// segment, so the ordered total is the reference's +-inf or NaN. Measured on
// MI355X at K = 28672, N = 8192 (2 segments): M = 1 25.8 us against 43.9 for
// the fp32-FMA GemvKernel the shape took before, M = 2 28.5 against 40.6 for
// GemvSmallMKernel; K = 24576, N = 4096 (4 segments) at M = 1 13.5 against
// 26.8; K = 18944, N = 3584 (74 units: 4 segments of 20, the last of 14) at
// M = 1 11.0 against 22.5. Shorter rows stay with their kernels (the
// segmented launch is slower there: c3 M = 1 11.5 against GemvM1Kernel's
// 10.0 us, c1 7.2 against 4.4).
//
// At 3 or 4 rows (the 4-row launch) the segments serve narrow weights better
// than DecodeFragKernel, the small-M MFMA decode: at M = 4, K = 24576,
// N = 3072 13.6 us against 18.7; K = 18944, N = 3584 13.2 against 18.3;
// K = 11008, N = 4096 9.9 against 12.5; K = 5120, N = 5120 8.2 against 10.8;
// K = 8192, N = 8192 11.7 against 13.5. Not for K <= 4096 (K = N = 4096:
// 8.0 against 7.1, the second launch) nor for the largest weights (K = 8192,
// N = 28672: 33.3 against 31.0; K = 28672, N = 8192: 33.1 against 32.3).
// At 2 rows they beat GemvSmallMKernel, the fp32-FMA GEMV, on such weights
// of 48 Mi elements and more: K = 5120, N = 13824 11.9 us against 17.0;
// K = N = 8192 11.1 against 14.1 (K = 8192, N = 3072: 7.8 against 7.3;
// K = N = 6144: 10.0 against 9.6).
#include "mnb_decode_common.h"

#include <algorithm>

namespace mnb {
namespace gf {

using namespace dec;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnitK = 256;                 // k per activation exponent
constexpr int kUnitSteps = kUnitK / 32;     // 32-k steps per unit
constexpr int kTerms = 3;                   // fp16 terms per activation
constexpr int kOpBytes = kTerms * 16;       // one row's three 16-byte operands
constexpr int kMaxWaves = 16;
constexpr size_t kLdsLimit = 150 * 1024;

// LDS byte offsets for MT activation rows: the operand image (K / 32 steps,
// each [quarter][row][term] 16-byte operands), the block sums (nb x MT
// floats) and unit exponents (K / 256 x MT ints) when MT > 1, the wavefront
// sums (waves x MT x 64 floats).
// Image bytes per 32-k step ([quarter][row][term] operands). With several
// rows each step is padded by 16 bytes: 768-byte steps (4 rows) start in the
// same banks, and the staging writes of a pass, 8 steps apart, conflicted
// (measured at c2 M = 4: 645,120 conflict cycles per dispatch, 301,056
// padded; 9.72 -> 9.50 us per call at M = 4, 9.45 -> 9.30 at M = 3).
__host__ __device__ constexpr int StepBytes(int mt) { return 4 * mt * kOpBytes + (mt > 1 ? 16 : 0); }
struct LdsLayout {
  int sums, exps, red, sq, bytes;
};
__host__ __device__ inline LdsLayout Layout(int K, int nb, int waves, int mt) {
  LdsLayout l;
  l.sums = (K / 32) * StepBytes(mt);
  l.exps = l.sums + (mt > 1 ? nb * mt * 4 : 0);
  l.red = l.exps + (mt > 1 ? (K / kUnitK) * mt * 4 : 0);
  l.sq = l.red + waves * mt * 256;  // per wavefront and row: its units' sum of squares (RMSNorm)
  l.bytes = l.sq + kMaxWaves * 4 * 4;
  return l;
}

// SPB = 32-k steps per quantization block (bs / 32, 1..8); SPW = steps per
// wavefront (whole units); WIN = weight records in flight per wavefront; MT =
// activation rows the launch is built for (1, 2 or 4; M <= MT). RMS: the
// input is RMSNorm(A) = A / sqrt(mean(A^2) + eps) * gamma, row by row; the
// staging multiplies by gamma and sums A^2 per row over the wavefront's
// units, and each row's 1 / rms scales its final sums (it is common to
// every product of the row).
template <bool HAS_ZP, int SPB, int SPW, int WIN, int MT, bool RMS, bool SEG = false>
__global__ __launch_bounds__(64 * kMaxWaves) void GemvFragKernel(
    const float *__restrict__ A, const uint8_t *__restrict__ Bp, const float *__restrict__ Sd,
    const uint32_t *__restrict__ Zd, float *__restrict__ Y, float *__restrict__ H,
    const float *__restrict__ bias, const float *__restrict__ gamma, float eps, int M, int N,
    int K, int nb, int segs, int seg_steps, float *__restrict__ P) {
  constexpr int kUnits = SPW / kUnitSteps;      // units of this wavefront
  constexpr int kItems = kUnits * MT;           // (unit, row) staging items, 32 lanes each
  constexpr int kPasses = (kItems + 1) / 2;     // two items per pass
  constexpr int kBlocks = SPW / SPB;            // quantization blocks of this wavefront
  constexpr int kBlocksPerUnit = kUnitSteps / SPB;
  constexpr int kStepBytes = StepBytes(MT);     // image bytes per step
  extern __shared__ uint4 lds16[];
  char *lds = reinterpret_cast<char *>(lds16);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int waves = static_cast<int>(blockDim.x) >> 6;
  // SEG: workgroup (g, seg) of `segs` K segments of `seg_steps` steps (the
  // last may be shorter); otherwise one per group (every segment term below
  // folds away).
  const int nseg = SEG ? segs : 1;
  const int g = SEG ? static_cast<int>(blockIdx.x) / nseg : static_cast<int>(blockIdx.x);
  const int seg = SEG ? static_cast<int>(blockIdx.x) - g * nseg : 0;
  const int T = K >> 5;
  const int sbase = SEG ? seg * seg_steps : 0;  // first step of this workgroup's K segment
  const int send = SEG ? min(sbase + seg_steps, T) : T;
  const int ubase = sbase / kUnitSteps;
  const int c = lane & 15;
  const int s0 = sbase + wave * SPW;   // first step of this wavefront
  const int u0 = s0 / kUnitSteps;      // its first unit
  // The LDS image and tables cover a segment (steps from sbase).
  const LdsLayout L = SEG ? Layout(32 * seg_steps, seg_steps / SPB, waves, MT)
                          : Layout(K, nb, waves, MT);
  float *sums = reinterpret_cast<float *>(lds + L.sums);
  int *exps = reinterpret_cast<int *>(lds + L.exps);
  float *red = reinterpret_cast<float *>(lds + L.red);
  float *sq_lds = reinterpret_cast<float *>(lds + L.sq);

  // 1. This wavefront's activations, before every weight load: in pass p,
  //    the 32 lanes of half h take the 8 values of quarter l & 31 of item
  //    2 p + h = (unit, row) (clamped items re-read a valid one and store
  //    nothing).
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, M * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(RMS ? gamma : A), 0, K * 4, 0x00020000);
  floatx4 va[kPasses][2], vg[RMS ? kPasses : 1][2];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int it = min(2 * p + (lane >> 5), kItems - 1);
    const int ul = it / MT, m = min(it % MT, M - 1);
    const int kk = (u0 + ul) * kUnitK + 8 * (lane & 31);
    // SEG: k past a K that does not fill its last unit reads past the end
    // of the buffer (zeros), not the next row
    const int off = !SEG || kk < K ? (m * K + kk) * 4 : M * K * 4;
    va[p][0] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
    va[p][1] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, off + 16, 0, 0));
    if constexpr (RMS) {
      const int goff = ((u0 + ul) * kUnitK + 8 * (lane & 31)) * 4;
      vg[p][0] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rg, goff, 0, 0));
      vg[p][1] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rg, goff + 16, 0, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. The first WIN weight records of this wavefront and their blocks'
  //    scales and zero points.
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(Bp + static_cast<size_t>(g) * T * 1024), 0, T * 1024, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(Sd + static_cast<size_t>(g) * nb * 64), 0, nb * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(HAS_ZP ? Zd + static_cast<size_t>(g) * nb * 16 : Zd), 0,
      HAS_ZP ? nb * 64 : 0, 0x00020000);
  struct Slot {
    u32x4 w;
    floatx4 s;
    uint32_t z;
  };
  Slot ring[WIN];
  auto issue = [&](int i) __attribute__((always_inline)) {
    Slot &sl = ring[i % WIN];
    const int s = s0 + i;
    sl.w = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, s * 1024 + 16 * lane, 0, kNonTemporal));
    if (i % SPB == 0) {
      const int blk = s / SPB;
      sl.s = __builtin_bit_cast(floatx4,
                                __builtin_amdgcn_raw_buffer_load_b128(rs, blk * 256 + 16 * c, 0, 0));
      if constexpr (HAS_ZP) sl.z = __builtin_amdgcn_raw_buffer_load_b32(rz, blk * 64 + 4 * c, 0, 0);
    }
  };
#pragma unroll
  for (int i = 0; i < WIN && i < SPW; ++i) issue(i);
  __builtin_amdgcn_sched_barrier(0);

  // 3. Staging of this wavefront's own steps (no workgroup barrier: a
  //    wavefront's LDS accesses execute in order): scale each (unit, row),
  //    split into three fp16 terms, write the operands; the block sums (a
  //    fixed butterfly over the block's lanes) and unit exponents go to
  //    scalars (M = 1) or to the LDS tables.
  float sb[MT == 1 ? kBlocks : 1];
  int eu[MT == 1 ? kUnits : 1];
  float sq[MT];  // RMS: per row, the sum of A^2 over this lane's valid values
#pragma unroll
  for (int r = 0; r < MT; ++r) sq[r] = 0.f;
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    if constexpr (RMS) {
      float q2 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q2 += va[p][0][i] * va[p][0][i] + va[p][1][i] * va[p][1][i];
        va[p][0][i] *= vg[p][0][i];
        va[p][1][i] *= vg[p][1][i];
      }
      const int itv = 2 * p + (lane >> 5);
#pragma unroll
      for (int r = 0; r < MT; ++r) sq[r] += itv < kItems && itv % MT == r ? q2 : 0.f;
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fmaxf(fabsf(va[p][0][i]), fabsf(va[p][1][i])));
    amax = HalfMax(amax);
    const int e = RangeExponent(amax, 14);
    half8 h[kTerms];
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = ldexpf(i < 4 ? va[p][0][i] : va[p][1][i - 4], e);
      ssum += x;
      const float xs = (i & 1) ? x * 0.0625f : x;
      const _Float16 t0 = static_cast<_Float16>(xs);
      const float r1 = __builtin_isfinite(xs) ? xs - static_cast<float>(t0) : 0.f;
      const _Float16 t1 = static_cast<_Float16>(r1);
      const _Float16 t2 = static_cast<_Float16>(r1 - static_cast<float>(t1));
      const int o = (i & 3) * 2 + (i >> 2);  // [0,4,1,5,2,6,3,7]
      h[0][o] = t0;
      h[1][o] = t1;
      h[2][o] = t2;
    }
    ssum = GroupSum<4 * SPB>(ssum);
    ssum *= 5.9604644775390625e-8f;  // 2^-24 (exact), before the block sums leave the lanes
    const int it = 2 * p + (lane >> 5);
    const int ul = it / MT, m = it % MT;
    const int q = lane & 31;  // quarter of the unit
    if (it < kItems && m < M) {
      uint4 *dst = reinterpret_cast<uint4 *>(lds + ((u0 + ul - ubase) * kUnitSteps + (q >> 2)) * kStepBytes +
                                             (q & 3) * (MT * kOpBytes) + m * kOpBytes);
#pragma unroll
      for (int t = 0; t < kTerms; ++t) dst[t] = __builtin_bit_cast(uint4, h[t]);
      if constexpr (MT > 1) {
        if (q == 0) exps[(u0 + ul - ubase) * MT + m] = e;
        if ((q & (4 * SPB - 1)) == 0)
          sums[((u0 + ul - ubase) * kBlocksPerUnit + q / (4 * SPB)) * MT + m] = ssum;
      }
    }
    if constexpr (MT == 1) {
#pragma unroll
      for (int uh = 0; uh < 2; ++uh) {
        if (2 * p + uh >= kUnits) continue;
        eu[2 * p + uh] = __builtin_amdgcn_readlane(e, 32 * uh);
#pragma unroll
        for (int bb = 0; bb < kBlocksPerUnit; ++bb)
          sb[(2 * p + uh) * kBlocksPerUnit + bb] =
              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssum), 32 * uh + 4 * SPB * bb));
      }
    }
  }
  if constexpr (RMS) {
    // the wavefront's sums of squares per row (fixed butterfly), to LDS
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      float t = sq[r];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o, 64);
      if (lane == 0) sq_lds[wave * MT + r] = t;
    }
  }

  // The image writes above precede the operand reads below.
  __asm__ volatile("" ::: "memory");

  // 4. The wavefront's steps. Lane l's A operand is term (l & 3) of row
  //    (l & 15) >> 2 of quarter l >> 4 (term 3 -> 0, rows past M -> row 0);
  //    lane l's results are row mc = l >> 4's (clamped: rows past M are
  //    computed and not stored).
  const int ma = min((lane & 15) >> 2, M - 1), ta = (lane & 3) == 3 ? 0 : (lane & 3);
  const int mc = min(lane >> 4, M - 1);
  const int a16 =
      ((s0 - sbase) * kStepBytes + (lane >> 4) * (MT * kOpBytes) + ma * kOpBytes + ta * 16) >> 4;
  const floatx4 zero4 = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 tmp[4];
  float racc[4], acc[4];  // per slice: the unit's sum, the wavefront's sum
  floatx4 bsc = zero4;
  uint32_t zw = 0x08080808u;  // zero points 8 without the input
  float sbv = 0.f;
  int ev = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    tmp[j] = zero4;
    racc[j] = 0.f;
    acc[j] = 0.f;
  }
  auto step = [&](int i) __attribute__((always_inline)) {
    Slot &sl = ring[i % WIN];
    // Pins the step's arithmetic here (left free, the compiler hoists work
    // on later steps' registers into this one and waits for their loads).
    // The operand's LDS index passes through the pin too, so its read is
    // issued here and not hoisted to the top (a register quad per step).
    int ai = a16;
    __asm__ volatile("" : "+v"(sl.w), "+v"(ai));
    const half8 a = __builtin_bit_cast(half8, lds16[ai + i * (kStepBytes / 16)]);
    if (i % SPB == 0) {
      bsc = sl.s;
      if constexpr (HAS_ZP) zw = sl.z;
      if constexpr (MT > 1) sbv = sums[((s0 - sbase + i) / SPB) * MT + mc];
    }
    if constexpr (MT > 1) {
      if (i % kUnitSteps == 0) ev = exps[((s0 - sbase + i) / kUnitSteps) * MT + mc];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = sl.w[j], w8 = w >> 8;
      const u32x4 qv = u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u};
      tmp[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, qv),
                                                      i % SPB == 0 ? zero4 : tmp[j], 0, 0, 0);
    }
    if ((i + 1) % SPB == 0) {
      const float sbi = MT == 1 ? sb[MT == 1 ? i / SPB : 0] : sbv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // rows 4 mc .. 4 mc + 2 of the tile: the three terms' sums
        float t = (tmp[j][0] + tmp[j][1]) + tmp[j][2];
        const float zp = static_cast<float>((zw >> (8 * j)) & 0xFFu);
        t = fmaf(-zp, sbi, t);
        racc[j] = fmaf(bsc[j], t, racc[j]);
      }
      // Only some lanes store these sums: unpinned, the compiler sinks the
      // block and unit arithmetic into that branch after the last step and
      // keeps every block's tiles live until then.
      __asm__ volatile("" : "+v"(racc[0]), "+v"(racc[1]), "+v"(racc[2]), "+v"(racc[3]));
    }
    if ((i + 1) % kUnitSteps == 0) {
      const int e = MT == 1 ? eu[MT == 1 ? i / kUnitSteps : 0] : ev;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] += __builtin_amdgcn_ldexpf(racc[j], 24 - e);
        racc[j] = 0.f;
      }
      __asm__ volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
    }
  };
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    step(i);
    __builtin_amdgcn_sched_barrier(0);
    if (i + WIN < SPW) issue(i + WIN);
    __builtin_amdgcn_sched_barrier(0);
  }

  // A wavefront past the end of a shorter last segment ran on loads beyond the
  // weights' buffers (zeros) and activations past its row: it adds nothing.
  if constexpr (SEG) {
    if (s0 >= send) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = 0.f;
    }
  }

  // 5. Wavefront sums in LDS (lanes 16 m + c hold rows 16 j + c of
  //    activation row m), added in wavefront order; one thread per output.
  if ((lane >> 4) < M) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[(wave * MT + (lane >> 4)) * 64 + 16 * j + c] = acc[j];
  }
  __syncthreads();
  // whole wavefronts per iteration (M * 64 and the block are multiples of 64)
  for (int idx = static_cast<int>(threadIdx.x); idx < M * 64; idx += static_cast<int>(blockDim.x)) {
    const int m = idx >> 6, r = idx & 63;
    float y = red[m * 64 + r];
    for (int w = 1; w < waves; ++w) y += red[(w * MT + m) * 64 + r];
    if constexpr (RMS) {
      // row m's 1 / rms: its sum of squares over the wavefronts, in order
      float tot = 0.0f;
      for (int w = 0; w < waves; ++w) tot += sq_lds[w * MT + m];
      y *= 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
    }
    const int n = 64 * g + r;
    if constexpr (!RMS) {
      // A non-finite activation: the reference's +-inf / NaN (see
      // ReferenceRowDot) over this workgroup's K segment. Row r of the group
      // is slice j = r >> 4, lane column r & 15 of the fragment-ordered
      // records.
      if (!__builtin_isfinite(y) && n < N) {
        constexpr int kLog2Bs = 5 + (SPB == 1 ? 0 : (SPB == 2 ? 1 : (SPB == 4 ? 2 : 3)));
        const int j = r >> 4, cc = r & 15;
        // the segment's first step, 8-k word and block
        const uint8_t *grp = Bp + (static_cast<size_t>(g) * T + sbase) * 1024;
        const float *sg = Sd + (static_cast<size_t>(g) * nb + sbase / SPB) * 64;
        const uint32_t *zg = HAS_ZP ? Zd + (static_cast<size_t>(g) * nb + sbase / SPB) * 16 : Zd;
        y = ReferenceRowDot(
            A + static_cast<size_t>(m) * K + 32 * sbase, 32 * (send - sbase), kLog2Bs,
            [&](int k8) {
              return *reinterpret_cast<const uint32_t *>(grp + (k8 >> 2) * 1024 +
                                                         16 * ((k8 & 3) * 16 + cc) + 4 * j);
            },
            [&](int b) {
              const float zp = HAS_ZP ? static_cast<float>((zg[b * 16 + cc] >> (8 * j)) & 0xFFu)
                                      : 8.0f;
              return make_float2(sg[b * 64 + cc * 4 + j], zp);
            });
      }
    }
    if (H != nullptr) {
      // gate/up pairs: rows 2 n', 2 n' + 1 in lanes r, r ^ 1 (N even)
      const float other = PairSwap(y);
      if ((r & 1) == 0 && n < N) H[m * (N >> 1) + (n >> 1)] = SiluMul(y, other);
    } else if (n < N) {
      // MatMulNBits input 5 (segments: added after their sum)
      if (bias != nullptr && !SEG) y += bias[n];
      (seg == 0 ? Y : P + static_cast<size_t>(seg - 1) * M * N)[m * N + n] = y;
    }
  }
}

inline int RowsBuilt(int64_t M) { return M == 1 ? 1 : (M == 2 ? 2 : 4); }

// segs > 1: K segments with their partial sums at P (no H, no RMSNorm input:
// checked by the caller); the sum pass follows in LaunchGemvFragSeg.
template <bool HAS_ZP, int SPB>
hipError_t LaunchSpw(const WeightView &w, int M, const float *A, float *Y, hipStream_t s, int spw,
                     int win, float *H, const float *bias, const float *gamma, float eps,
                     int segs = 1, int seg_steps = 0, float *P = nullptr) {
  const int K = static_cast<int>(w.K), N = static_cast<int>(w.N), nb = static_cast<int>(w.nb);
  if (segs <= 1) seg_steps = K / 32;
  const int waves = seg_steps / spw;
  const int mt = RowsBuilt(M);
  const int lds = segs > 1 ? Layout(32 * seg_steps, seg_steps / SPB, waves, mt).bytes
                           : Layout(K, nb, waves, mt).bytes;
  const dim3 grid(static_cast<unsigned>((w.N + 63) / 64 * segs)),
      block(static_cast<unsigned>(64 * waves));
#define MNB_GF_LAUNCH(SPWV, WINV, MTV, RMSV)                                                    \
  hipLaunchKernelGGL((GemvFragKernel<HAS_ZP, SPB, SPWV, WINV, MTV, RMSV>), grid, block, lds, s, \
                     A, w.Bp, w.Sd, w.Zd, Y, H, bias, gamma, eps, M, N, K, nb, segs, seg_steps, P)
  if (segs > 1) {
    // K segments: window 8, no RMSNorm input, 8 steps per wavefront at 4 rows
    // with 32-k blocks (checked by the caller)
#define MNB_GF_LAUNCH_SEG(SPWV, MTV)                                                         \
  hipLaunchKernelGGL((GemvFragKernel<HAS_ZP, SPB, SPWV, 8, MTV, false, true>), grid, block, lds, \
                     s, A, w.Bp, w.Sd, w.Zd, Y, nullptr, nullptr, nullptr, 0.0f, M, N, K, nb, segs,     \
                     seg_steps, P)
    if (mt == 1) {
      switch (spw) {
      case 8: MNB_GF_LAUNCH_SEG(8, 1); break;
      case 16: MNB_GF_LAUNCH_SEG(16, 1); break;
      default: MNB_GF_LAUNCH_SEG(32, 1); break;
      }
    } else if (mt == 2) {
      if (spw == 8) MNB_GF_LAUNCH_SEG(8, 2);
      else MNB_GF_LAUNCH_SEG(16, 2);
    } else {
      if (spw == 8) MNB_GF_LAUNCH_SEG(8, 4);
      else if constexpr (SPB > 1) MNB_GF_LAUNCH_SEG(16, 4);
    }
#undef MNB_GF_LAUNCH_SEG
    return hipGetLastError();
  }
  if (gamma != nullptr) {
    // RMSNorm input (window 8; no 32-step launch with 32-k blocks; 8 steps
    // for M > 1, not with 32-k blocks at 4 rows: checked by the caller, see
    // RmsSpw)
    if (mt == 1) {
      switch (spw) {
      case 8: MNB_GF_LAUNCH(8, 8, 1, true); break;
      case 16: MNB_GF_LAUNCH(16, 8, 1, true); break;
      default:
        if constexpr (SPB > 1) MNB_GF_LAUNCH(32, 8, 1, true);
        break;
      }
    } else if (mt == 2) {
      MNB_GF_LAUNCH(8, 8, 2, true);
    } else {
      if constexpr (SPB > 1) MNB_GF_LAUNCH(8, 8, 4, true);
    }
  } else if (mt > 1) {
    // more rows: window 8, 8 or 16 steps per wavefront (checked by the caller)
    if (mt == 2) {
      if (spw == 8) MNB_GF_LAUNCH(8, 8, 2, false);
      else MNB_GF_LAUNCH(16, 8, 2, false);
    } else {
      // 16 steps at 4 rows only above 32-k blocks (ShapeFits; that launch
      // with 32-k blocks spills registers and is not built)
      if (spw == 8) MNB_GF_LAUNCH(8, 8, 4, false);
      else if constexpr (SPB > 1) MNB_GF_LAUNCH(16, 8, 4, false);
    }
  } else if (win == 8) {
    switch (spw) {
    case 8: MNB_GF_LAUNCH(8, 8, 1, false); break;
    case 16: MNB_GF_LAUNCH(16, 8, 1, false); break;
    default: MNB_GF_LAUNCH(32, 8, 1, false); break;
    }
  } else {
    switch (spw) {
    case 8: MNB_GF_LAUNCH(8, 4, 1, false); break;
    case 16: MNB_GF_LAUNCH(16, 4, 1, false); break;
    default: MNB_GF_LAUNCH(32, 4, 1, false); break;
    }
  }
#undef MNB_GF_LAUNCH
  return hipGetLastError();
}

template <bool HAS_ZP>
hipError_t LaunchZp(const WeightView &w, int M, const float *A, float *Y, hipStream_t s, int spw,
                    int win, float *H, const float *bias, const float *gamma, float eps,
                    int segs = 1, int seg_steps = 0, float *P = nullptr) {
  switch (w.block_size / 32) {
  case 1:
    return LaunchSpw<HAS_ZP, 1>(w, M, A, Y, s, spw, win, H, bias, gamma, eps, segs, seg_steps, P);
  case 2:
    return LaunchSpw<HAS_ZP, 2>(w, M, A, Y, s, spw, win, H, bias, gamma, eps, segs, seg_steps, P);
  case 4:
    return LaunchSpw<HAS_ZP, 4>(w, M, A, Y, s, spw, win, H, bias, gamma, eps, segs, seg_steps, P);
  default:
    return LaunchSpw<HAS_ZP, 8>(w, M, A, Y, s, spw, win, H, bias, gamma, eps, segs, seg_steps, P);
  }
}

inline bool ShapeFits(const WeightView &w, int64_t M, int spw, int win) {
  const int T = static_cast<int>(w.K / 32);
  if (spw != 8 && spw != 16 && spw != 32) return false;
  if (win != 4 && win != 8) return false;
  if (M > 1 && (spw == 32 || win != 8)) return false;  // the launches built for M > 1
  if (M > 2 && w.block_size == 32 && spw != 8) return false;  // 16 steps spill registers
  if (T % spw != 0 || T / spw > kMaxWaves) return false;
  return static_cast<size_t>(
             Layout(static_cast<int>(w.K), static_cast<int>(w.nb), T / spw, RowsBuilt(M)).bytes) <=
         kLdsLimit;
}

// Steps per wavefront: 16 where that gives at most 16 wavefronts, else 32
// (M = 1), else 8 (K below 512); window 8. Measured on MI355X at M = 1
// (interleaved medians; steps / window): c2 16 / 8 7.31 us, 16 / 4 7.42,
// 8 / 4 7.70, 8 / 8 7.94, 32 / 4 8.47; c5 gate+up 12.69, 12.65, 13.04,
// 14.38, 12.76.
inline int PickSpw(const WeightView &w, int64_t M) {
  for (int spw : {16, 32, 8})
    if (ShapeFits(w, M, spw, 8)) return spw;
  return 0;
}

// K segments: for 2, 3, ... 16 segments asked for, steps per wavefront in
// PickSpw's order, the segment length rounded up to whole units and whole
// wavefronts (the last segment takes the rest), every wavefront wholly inside
// the row or past its end; among the shapes with at most 16 wavefronts and
// the LDS image of one segment within the limit, the least work on the
// busiest CU: ceil(groups x segs / CUs) workgroups of `steps` steps, each
// costing 16 steps more for its staging, sums and launch share, fewer
// segments on a tie. Against the first shape covering 85% of the CUs:
// K = 27648, N = 5120 at M = 2 6 segments of 144 steps instead of 4 of 224
// (64 CUs with two workgroups), 22.7 -> 19.9 us; K = 8192, N = 10240 at
// M = 2 3 segments of 88 steps instead of 2 of 128, 14.9 -> 13.0 us;
// K = 20480, N = 512 at M = 1 (8 groups) 16 segments of 40 steps instead of
// 14 of 48, 6.46 -> 6.65 us. segs = 0: none.
struct SegShape {
  int segs = 0, steps = 0, spw = 0;
};
inline int64_t SegCost(int64_t groups, int segs, int steps, int64_t cus) {
  return (groups * segs + cus - 1) / cus * (steps + 16);
}
inline SegShape SegmentShape(const WeightView &w, int64_t M) {
  // steps of whole units: a K that does not fill its last unit ends in steps
  // that read zeros (weights beyond the group's records, masked activations)
  const int T = static_cast<int>((w.K + kUnitK - 1) / kUnitK * kUnitSteps);
  const int64_t groups = (w.N + 63) / 64;
  const int64_t cus = std::max<int64_t>(1, w.num_cus);
  SegShape best;
  int64_t best_cost = 0;
  for (int sg = 2; sg <= 16; ++sg) {
    for (int spw : {16, 32, 8}) {
      if ((M > 1 && spw == 32) || T % spw != 0) continue;  // the launches built for M > 1
      if (RowsBuilt(M) == 4 && w.block_size == 32 && spw != 8) continue;
      const int gran = std::max(spw, kUnitSteps);
      const int steps = ((T + sg - 1) / sg + gran - 1) / gran * gran;
      const int segs = (T + steps - 1) / steps;
      if (segs < 2 || steps / spw > kMaxWaves) continue;
      const int seg_nb = steps * 32 / static_cast<int>(w.block_size);
      if (static_cast<size_t>(Layout(32 * steps, seg_nb, steps / spw, RowsBuilt(M)).bytes) >
          kLdsLimit)
        continue;
      const int64_t cost = SegCost(groups, segs, steps, cus);
      if (best.segs == 0 || cost < best_cost || (cost == best_cost && segs < best.segs)) {
        best = SegShape{segs, steps, spw};
        best_cost = cost;
      }
    }
  }
  return best;
}

// Steps per wavefront with an RMSNorm input (0: none): M = 1 as PickSpw
// except 32 steps with 32-k blocks; M > 1 only 8 steps, and not 4 rows with
// 32-k blocks (the other launches of the per-row sums of squares spill
// registers under the 1024-thread bound).
inline int RmsSpw(const WeightView &w, int64_t M) {
  if (M == 1) {
    const int spw = PickSpw(w, 1);
    return spw == 32 && w.block_size == 32 ? 0 : spw;
  }
  if (RowsBuilt(M) == 4 && w.block_size == 32) return 0;
  return ShapeFits(w, M, 8, 8) ? 8 : 0;
}

} // namespace gf

bool GemvFragSupports(const WeightView &w, int64_t M) {
  // The plan's fragment-ordered weights and decode scales; blocks of 32 to
  // 256 k (each block inside one 256-k unit, each step inside one block);
  // whole units per wavefront for some SPW with the image in LDS; 32-bit
  // buffer offsets.
  return M >= 1 && M <= 4 && w.Bp != nullptr && w.Sd != nullptr &&
         (!w.has_zp || w.Zd != nullptr) && w.block_size >= 32 && w.block_size <= 256 &&
         (w.block_size & (w.block_size - 1)) == 0 && (w.K % gf::kUnitK) == 0 &&
         gf::PickSpw(w, M) > 0 && (w.K / 32) * 1024 < (int64_t{1} << 31) &&
         w.nb * 256 < (int64_t{1} << 31) && M * w.K * 4 < (int64_t{1} << 31) &&
         M * w.N < (int64_t{1} << 30);
}

bool GemvFragShapeOk(const WeightView &w, int64_t M, int spw, int win) {
  return GemvFragSupports(w, M) && gf::ShapeFits(w, M, spw == 0 ? gf::PickSpw(w, M) : spw,
                                                  win == 0 ? 8 : win);
}

bool GemvFragWide(const WeightView &w) {
  return ((w.N + 63) / 64) * 100 >= static_cast<int64_t>(w.num_cus) * 85;
}

bool GemvFragPreferred(const WeightView &w, int64_t M, bool rms) {
  // One workgroup per 64-row group: worth it where the groups cover most of
  // the CUs. The RMSNorm input: not 32 steps per wavefront with 32-k blocks
  // (the launch that would spill registers).
  if (rms && gf::RmsSpw(w, M) == 0) return false;
  return GemvFragSupports(w, M) && GemvFragWide(w);
}

hipError_t LaunchGemvFrag(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s,
                          int spw, int win, float *H, const float *bias, const float *gamma,
                          float eps) {
  if (spw == 0) spw = gamma != nullptr ? gf::RmsSpw(w, M) : gf::PickSpw(w, M);
  if (win == 0) win = 8;
  if (!GemvFragSupports(w, M) || !gf::ShapeFits(w, M, spw, win)) return hipErrorInvalidValue;
  if (gamma != nullptr &&
      (win != 8 || (spw == 32 && w.block_size == 32) ||
       (M > 1 && (spw != 8 || (gf::RowsBuilt(M) == 4 && w.block_size == 32))) ||
       (reinterpret_cast<uintptr_t>(gamma) % 16) != 0))
    return hipErrorInvalidValue;
  const int m = static_cast<int>(M);
  return w.has_zp ? gf::LaunchZp<true>(w, m, A, Y, s, spw, win, H, bias, gamma, eps)
                         : gf::LaunchZp<false>(w, m, A, Y, s, spw, win, H, bias, gamma, eps);
}

// Wide weights whose single-workgroup launch (one per 64-row group, one per
// CU at a time) leaves a second round on a few CUs: K segments when the
// busiest CU's work (SegmentShape's measure, the sum pass counted as 60
// steps) drops by more than 10%. Measured at M = 1: K = 7168, N = 18432
// (288 groups) 18.2 -> 16.3 us with 4 segments; the shapes it takes have
// 272 to 384 groups and rows of 7168 and more.
static bool SegmentsBalance(const WeightView &w, int64_t M) {
  const gf::SegShape sh = gf::SegmentShape(w, M);
  if (sh.segs < 2) return false;
  const int64_t groups = (w.N + 63) / 64, cus = std::max<int64_t>(1, w.num_cus);
  const int64_t single = gf::SegCost(groups, 1, static_cast<int>(w.K / 32), cus);
  return (gf::SegCost(groups, sh.segs, sh.steps, cus) + 60) * 10 < single * 9;
}

bool GemvFragSegSupports(const WeightView &w, int64_t M) {
  // As GemvFragSupports, K split into segments of whole units (a K that is
  // not a multiple of 256 ends in a partly filled unit). Where the single-
  // workgroup launch is the automatic choice (GemvFragPreferred): only where
  // the segments balance the CUs (SegmentsBalance). Elsewhere: 1 or 2 rows
  // too long for one workgroup (no single-workgroup launch fits); 3 or 4
  // rows of at least 5120 on weights of at most 192 Mi elements, where the
  // segments beat the small-M MFMA decode (shorter rows pay more for the
  // partial sums' second launch than they gain; the largest weights fill the
  // CUs with the decode's own split); 2 such rows on weights of at least
  // 48 Mi elements, where they beat the fp32-FMA GEMV.
  if (M < 1 || M > 4 || w.Bp == nullptr || w.Sd == nullptr || (w.has_zp && w.Zd == nullptr) ||
      w.block_size < 32 || w.block_size > 256 || (w.block_size & (w.block_size - 1)) != 0 ||
      (w.K % 32) != 0)
    return false;
  const int64_t kn = w.K * w.N;
  const bool long_narrow = w.K >= 5120 && kn <= (int64_t{192} << 20);
  // Rows too long for one workgroup; with a K that is not a whole number of
  // units (no single-workgroup launch at all) those past the M = 1 GEMV's
  // limit at M = 1 and past 8192 at M = 2, as for whole units.
  const bool too_long =
      M <= 2 && ((w.K % gf::kUnitK) != 0 ? w.K > (M == 1 ? 16384 : 8192) : gf::PickSpw(w, M) == 0);
  if (GemvFragPreferred(w, M, false) ? !SegmentsBalance(w, M)
                                     : !too_long && !(M >= 3 && long_narrow) &&
                                           !(M == 2 && long_narrow && kn >= (int64_t{48} << 20)))
    return false;
  // K <= 2^20: the offsets of wavefronts past the end of a shorter last
  // segment (up to one segment beyond the row and the weights' buffers) stay
  // far below 2^31.
  const int segs = gf::SegmentShape(w, M).segs;
  return segs > 1 && w.K <= (int64_t{1} << 20) && segs * M * w.N < (int64_t{1} << 29);
}

size_t GemvFragSegWorkspaceBytes(const WeightView &w, int64_t M) {
  const int segs = GemvFragSegSupports(w, M) ? gf::SegmentShape(w, M).segs : 1;
  return static_cast<size_t>(segs - 1) * static_cast<size_t>(M) * w.N * 4;
}

hipError_t LaunchGemvFragSeg(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                             hipStream_t s, const float *bias) {
  if (!GemvFragSegSupports(w, M) || work == nullptr) return hipErrorInvalidValue;
  const gf::SegShape sh = gf::SegmentShape(w, M);
  float *P = static_cast<float *>(work);
  const int m = static_cast<int>(M);
  const hipError_t e =
      w.has_zp ? gf::LaunchZp<true>(w, m, A, Y, s, sh.spw, 8, nullptr, nullptr, nullptr, 0.0f,
                                    sh.segs, sh.steps, P)
               : gf::LaunchZp<false>(w, m, A, Y, s, sh.spw, 8, nullptr, nullptr, nullptr, 0.0f,
                                     sh.segs, sh.steps, P);
  if (e != hipSuccess) return e;
  // Y += the segments' partial sums in segment order, then the bias.
  return LaunchSumPartials(Y, P, M * w.N, sh.segs - 1, nullptr, s, bias, w.N);
}

} // namespace mnb
