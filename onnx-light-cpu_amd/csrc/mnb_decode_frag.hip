// Decode GEMV for 2 <= M <= 16 activation rows on fp16 MFMA with 22-bit
// activations and fp32 sums, streaming the plan's fragment-ordered weights.
//
// Role in the reference: the roadmap's `int4_gemv` / `int4_small_m` decode
// side (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-221: each
// weight byte streamed once, unpacked blocks reused across the batch rows);
// the fp32 semantics are those of the reference engine's skinny-M product
// (onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258): q - zp is exact, each
// activation keeps 22 significant bits (relative error at most 2^-22, against
// fp32's 2^-24 rounding of each product) and the products are summed in fp32.
//
// Two kernels per call:
//
// 1. SplitActKernel (one wavefront per unit of 256 k and pair of tokens)
//    scales each token's values in the unit by a power of two 2^e (largest
//    magnitude in [2^14, 2^15); exact) and splits every scaled value into two
//    fp16 terms,
//    a 2^e ~ a0 + a1 with a0 = fp16(a 2^e) and a1 = fp16(a 2^e - a0) (the
//    difference is exact in fp32; 2 x 11 significand bits, so |a 2^e - a0 -
//    a1| <= 2^-22 |a 2^e|, and below 2^-39 of the unit's largest magnitude
//    for values under fp16's normal range), written to the workspace as the
//    MFMA operand image [unit][step][term][lane] (16 bytes per lane: token
//    lane & 15, 8 k of quarter lane >> 4, in the weight decode's
//    [0,4,1,5,2,6,3,7] order) plus e per (unit, token). Tokens past M are
//    zero.
//
// 2. DecodeFragKernel. The plan's prefill weight copy Bp holds, for each
//    group g of 64 weight rows and 32-k step s, a 1 KiB record whose lane l
//    holds the packed words of rows 64 g + 16 j + (l & 15), j = 0..3, at
//    k = 32 s + 8 (l >> 4): the MFMA B operands of four 16-row slices. A
//    unit (8 steps) of one group is therefore 8 KiB of contiguous weights,
//    read with 16-byte loads that cover 1 KiB per wavefront instruction
//    (measured on MI355X: such records stream the c2 and c3 weights in
//    6.1 us against 7.9-8.6 us for 64-byte pieces of 16 rows). A third
//    activation term (exact products) cost 15-25% more time on c1-c3 at
//    M = 16 for no gain under the decode bound.
//    - A workgroup of WPG wavefronts owns one group and a run of
//      WPG * U consecutive units; wavefront w multiplies U of them. Per step
//      it decodes the record's four words (q - zp exact in fp16, exponent
//      constants), reads the two activation terms of the step (from L2:
//      the image is shared by every group) and issues 2 x 4
//      v_mfma_f32_16x16x32_f16 into one fp32 tile per slice; at each block's
//      end the tile is multiplied by the rows' fp32 block scales into the
//      unit's sum, at each unit's end the unit's sum is scaled by 2^-e
//      (exact) into the wavefront's sum.
//    - Up to 8 tokens (TOKS = 8) the two terms of token t are rows 2 t and
//      2 t + 1 of one A operand: a step reads 1 KiB of operands instead of
//      2 (the operand loads bound the kernel at 16 tokens) and issues 4
//      MFMAs; the two terms' rows are added at each block's end. c2 M = 5 /
//      8 14.0 / 14.1 -> 11.5 / 11.6 us, c3 17.6 / 17.9 -> 14.4 / 15.0.
//    - The wavefronts' sums meet in LDS and are added in wavefront order;
//      a run that does not cover K writes a partial sum, added in run order
//      by the ordered partial-sum pass. Results do not depend on scheduling.
//    - Weights, activation terms, block scales and zero points stream
//      through a rolling window of WIN steps in registers: multiply the
//      oldest, issue the one WIN further on. Every load is unconditional and
//      in bounds (rows past N are zero in the re-laid copies).
//    The MFMA takes the activations as its A operand (rows = tokens) and the
//    weights as its B operand (columns = weight rows): lane l's value v is
//    token 4 (l >> 4) + v of weight row 16 j + (l & 15), so a lane's block
//    scale is its own row's.
#include "mnb_decode_common.h"

#include <algorithm>

namespace mnb {
namespace df {

using namespace dec;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnitK = 256;            // k per unit: one activation exponent per token
constexpr int kUnitSteps = kUnitK / 32;
constexpr int kTok = 16;               // tokens per MFMA tile (M padded)
constexpr int kMaxWaves = 8;
constexpr int kTerms = 2;              // fp16 terms per activation
constexpr int kStepBytes = kTerms * 1024;  // image bytes per 32-k step (16 tokens)
// Up to 8 tokens: the two terms of each token are rows 2 t and 2 t + 1 of
// one MFMA A operand, so a step's image is 1 KiB and one MFMA per slice
// multiplies both terms.
template <int TOKS>
constexpr int StepBytesT() { return TOKS == 16 ? kStepBytes : 1024; }
constexpr int kMaxSqUnits = 64;            // RMSNorm input: K <= 64 units (16384)

__device__ __forceinline__ uint32_t PkAddF16(uint32_t a, uint32_t b) {
  const half2v r = __builtin_bit_cast(half2v, a) + __builtin_bit_cast(half2v, b);
  return __builtin_bit_cast(uint32_t, r);
}

// 8 nibbles (k order) of one word -> q - zp as fp16 in [0,4,1,5,2,6,3,7]
// order, exact: (w & 0x000F000F) | 0x6400.. is the fp16 pair 1024 + q of
// nibbles 0 | 4 (ulp 1 at 1024), (w & 0x00F000F0) | 0x5400.. the pair 64 + q
// of nibbles 1 | 5 (ulp 1/16 at 64); the same of w >> 8 gives nibbles 2 | 6
// and 3 | 7. neg_lo / neg_hi are the fp16 pairs -(1024 + zp) / -(64 + zp).
// The masks sit in VGPRs (v_and_or_b32 takes no literal on gfx9).
struct Masks {
  uint32_t lo, hi, e1024, e64;
};
__device__ __forceinline__ Masks MakeMasks() {
  Masks c{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  __asm__ volatile("" : "+v"(c.lo), "+v"(c.hi), "+v"(c.e1024), "+v"(c.e64));
  return c;
}
__device__ __forceinline__ half8 DecodeQ(uint32_t w, uint32_t neg_lo, uint32_t neg_hi,
                                         const Masks &c) {
  const uint32_t w8 = w >> 8;
  const uint4 r = make_uint4(PkAddF16((w & c.lo) | c.e1024, neg_lo),
                             PkAddF16((w & c.hi) | c.e64, neg_hi),
                             PkAddF16((w8 & c.lo) | c.e1024, neg_lo),
                             PkAddF16((w8 & c.hi) | c.e64, neg_hi));
  return __builtin_bit_cast(half8, r);
}

// One wavefront (a workgroup of 64 threads) per unit u and pair of tokens:
// lane (t, ch) of workgroup (u, pair) takes the 8 values k = 256 u + 8 ch ..
// + 7 of token t = 2 pair + (lane >> 5), so each token's unit spans 32 lanes
// and its largest magnitude is a 5-step butterfly within them. Writes
// img[((u * 8 + ch / 4) * kTerms + term) * 64 + 16 (ch % 4) + t] and
// exps[u * 16 + t]; with TOKS = 8 (M <= 8) TOKS / 2 workgroups per unit and
// img[(u * 8 + ch / 4) * 64 + 16 (ch % 4) + 2 t + term]. (One 128-thread
// workgroup per unit, each thread taking 32 values, kept 16 workgroups busy
// for about 4 us at M = 16.)
// RMS (RMSNorm fused into the input): the values split are a * gamma, and
// sq[u * 16 + t] receives the token's sum of a^2 over the unit (a fixed
// butterfly), from which the main kernel forms 1 / rms.
template <bool RMS, int TOKS>
__global__ __launch_bounds__(64) void SplitActKernel(const float *__restrict__ A,
                                                     uint4 *__restrict__ img,
                                                     int *__restrict__ exps,
                                                     float *__restrict__ sq,
                                                     const float *__restrict__ gamma, int M,
                                                     int K) {
  constexpr int kPairs = TOKS / 2;  // workgroups per unit
  const int u = static_cast<int>(blockIdx.x) / kPairs;
  const int t = (static_cast<int>(blockIdx.x) % kPairs) * 2 + static_cast<int>(threadIdx.x >> 5);
  const int ch = threadIdx.x & 31;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, M * K * 4, 0x00020000);
  // tokens past M, and k past K in a last unit that K does not fill, read
  // past the end of the buffer: zeros
  const int vo = t < M && kUnitK * u + 8 * ch < K ? (t * K + kUnitK * u + 8 * ch) * 4 : M * K * 4;
  floatx4 v0 = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, vo, 0, 0));
  floatx4 v1 = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, vo + 16, 0, 0));
  if constexpr (RMS) {
    const float4 *gp = reinterpret_cast<const float4 *>(gamma + kUnitK * u + 8 * ch);
    const float4 g0 = gp[0], g1 = gp[1];
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) q += v0[c] * v0[c] + v1[c] * v1[c];
    q = GroupSum<32>(q);
    if (ch == 0) sq[u * kTok + t] = q;
    v0 *= floatx4{g0.x, g0.y, g0.z, g0.w};
    v1 *= floatx4{g1.x, g1.y, g1.z, g1.w};
  }
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) amax = fmaxf(amax, fmaxf(fabsf(v0[c]), fabsf(v1[c])));
  amax = HalfMax(amax);
  // The largest magnitude times 2^e in [2^14, 2^15); ldexp is exact for
  // every e this gives (|e| <= 163), subnormal inputs included. A zero, inf
  // or NaN maximum gives e = 0 (inf and NaN then propagate).
  const int e = RangeExponent(amax, 14);
  if (ch == 0) exps[u * kTok + t] = e;
  half8 h[kTerms];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int o = (i & 3) * 2 + (i >> 2);  // k order [0,4,1,5,2,6,3,7]
    const float x = ldexpf(i < 4 ? v0[i] : v1[i - 4], e);
    const _Float16 h0 = static_cast<_Float16>(x);
    h[0][o] = h0;
    h[1][o] = static_cast<_Float16>(__builtin_isfinite(x) ? x - static_cast<float>(h0) : 0.f);
  }
#pragma unroll
  for (int term = 0; term < kTerms; ++term) {
    if constexpr (TOKS == 16)
      img[((u * kUnitSteps + (ch >> 2)) * kTerms + term) * 64 + 16 * (ch & 3) + t] =
          __builtin_bit_cast(uint4, h[term]);
    else  // lane 16 quarter + 2 t + term of the step's one operand
      img[(u * kUnitSteps + (ch >> 2)) * 64 + 16 * (ch & 3) + 2 * t + term] =
          __builtin_bit_cast(uint4, h[term]);
  }
}

// Group g of 64 weight rows, run `seg` of WPG * U units. SPB = 32-k steps
// per quantization block within a unit (bs / 32, at most 8).
// RMS: the image holds A * gamma; every run scales its sums by each token's
// 1 / rms = 1 / sqrt(sum_k A^2 / K + eps), from SplitActKernel's per-unit
// sums of squares added in unit order.
template <bool HAS_ZP, int SPB, int U, int WIN, bool RMS, int TOKS>
__global__ __launch_bounds__(64 * kMaxWaves) void DecodeFragKernel(
    const uint8_t *__restrict__ Bp, const float *__restrict__ Sd, const uint32_t *__restrict__ Zd,
    const uint4 *__restrict__ img, const int *__restrict__ exps, float *__restrict__ Y,
    float *__restrict__ partials, float *__restrict__ H, const float *__restrict__ bias, int M,
    int N, int K, int nb, int log2_bs, int segs, int wpg, const float *__restrict__ sq,
    float eps) {
  __shared__ float red[kMaxWaves * 16 * 64];  // 32 KiB: [wave][slice * 4 + v][lane]
  __shared__ float rinv[kTok];                // RMS: each token's 1 / rms
  __shared__ float sqs[RMS ? kMaxSqUnits * kTok : 1];  // RMS: the per-unit sums of squares
  constexpr int kSteps = U * kUnitSteps;
  constexpr int kSB = StepBytesT<TOKS>();
  constexpr int kTPL = TOKS / 4;     // tokens per lane in the MFMA result
  constexpr int kItems = 4 * kTPL;   // (slice, token) results per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int c = lane & 15, qd = lane >> 4;
  const int g = static_cast<int>(blockIdx.x) / segs;
  const int seg = static_cast<int>(blockIdx.x) - g * segs;
  const int T = K / 32;
  const int Tp = (K + kUnitK - 1) / kUnitK * kUnitSteps;  // steps of whole units (image, exponents)
  const int u0 = (seg * wpg + wave) * U;  // first unit of this wavefront
  const int s0 = u0 * kUnitSteps;         // first step

  // Per-group bases (wave-uniform), per-lane offsets below 2^31.
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(Bp + static_cast<size_t>(g) * T * 1024), 0, T * 1024, 0x00020000);
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4 *>(img), 0, Tp * kSB, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(Sd + static_cast<size_t>(g) * nb * 64), 0, nb * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(HAS_ZP ? Zd + static_cast<size_t>(g) * nb * 16 : Zd), 0,
      HAS_ZP ? nb * 64 : 0, 0x00020000);

  // RMS: wavefront 0 copies the per-unit sums of squares ([unit][token],
  // 64 bytes per unit, L2-resident) straight into LDS first, with no
  // registers held, and adds them up after the stream. Lanes past the end
  // copy the last 16 bytes again (in bounds; those LDS bytes are not read).
  if constexpr (RMS) {
    if (wave == 0) {
      const int bytes = (T / kUnitSteps) * kTok * 4;
      const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sqs));
      for (int i = 0; i * 1024 < bytes; ++i)
        CopyToLds16(reinterpret_cast<const char *>(sq) + min(i * 1024 + 16 * lane, bytes - 16),
                    base + static_cast<uint32_t>(i * 1024));
    }
  }

  // Each unit's token exponents: lane quarter qd holds tokens kTPL qd ..
  // kTPL qd + kTPL - 1.
  int4 ue[U];
  const __amdgpu_buffer_rsrc_t re = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int *>(exps), 0, (Tp / kUnitSteps) * 64, 0x00020000);
#pragma unroll
  for (int uu = 0; uu < U; ++uu) {
    if constexpr (TOKS == 16) {
      ue[uu] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(re, (u0 + uu) * 64 + 16 * qd, 0, 0));
    } else {
      typedef int i32x2 __attribute__((ext_vector_type(2)));
      const i32x2 e2 = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(re, (u0 + uu) * 64 + 8 * qd, 0, 0));
      ue[uu] = int4{e2[0], e2[1], 0, 0};
    }
  }

  struct Slot {
    u32x4 w, a0, a1;
    floatx4 s;
    uint32_t z;
  };
  Slot ring[WIN];
  auto issue = [&](int i) __attribute__((always_inline)) {
    Slot &sl = ring[i % WIN];
    const int s = s0 + i;
    sl.w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, s * 1024 + 16 * lane, 0,
                                                                           kNonTemporal));
    sl.a0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ri, s * kSB + 16 * lane, 0, 0));
    if constexpr (TOKS == 16)
      sl.a1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ri, s * kSB + 1024 + 16 * lane, 0, 0));
    if (i % SPB == 0) {
      const int blk = (s * 32) >> log2_bs;
      sl.s = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, blk * 256 + 16 * c, 0, 0));
      if constexpr (HAS_ZP) sl.z = __builtin_amdgcn_raw_buffer_load_b32(rz, blk * 64 + 4 * c, 0, 0);
    }
  };
#pragma unroll
  for (int i = 0; i < WIN && i < kSteps; ++i) issue(i);
  __builtin_amdgcn_sched_barrier(0);

  const Masks mk = MakeMasks();
  floatx4 acc[4], racc[4], tmp[4];
  floatx4 bsc = floatx4{0.f, 0.f, 0.f, 0.f};
  uint32_t neg_lo[4], neg_hi[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    neg_lo[j] = 0xE408E408u;  // fp16 -(1024 + 8)
    neg_hi[j] = 0xD480D480u;  // fp16 -(64 + 8)
  }
  auto step = [&](int i) __attribute__((always_inline)) {
    Slot &sl = ring[i % WIN];
    // Pins the step's arithmetic here: left free, the compiler hoists work
    // on later steps' registers into this one and waits for their loads.
    __asm__ volatile("" : "+v"(sl.w), "+v"(sl.a0), "+v"(sl.a1));
    if (i % kUnitSteps == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) racc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    if (i % SPB == 0) {
      bsc = sl.s;
      if constexpr (HAS_ZP) {
        const uint32_t z = sl.z;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // byte j is the zero point of row 16 j + c: fp16 -(1024 + zp) =
          // 0xE400 | zp, -(64 + zp) = 0xD400 | zp << 4
          const uint32_t zz = ((z >> (8 * j)) & 0xFu) * 0x10001u;
          neg_lo[j] = zz | 0xE400E400u;
          neg_hi[j] = (zz << 4) | 0xD400D400u;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) tmp[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    half8 q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = DecodeQ(sl.w[j], neg_lo[j], neg_hi[j], mk);
    const half8 a0 = __builtin_bit_cast(half8, sl.a0);
#pragma unroll
    for (int j = 0; j < 4; ++j) tmp[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, q[j], tmp[j], 0, 0, 0);
    if constexpr (TOKS == 16) {
      const half8 a1 = __builtin_bit_cast(half8, sl.a1);
#pragma unroll
      for (int j = 0; j < 4; ++j) tmp[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, q[j], tmp[j], 0, 0, 0);
    }
    if ((i + 1) % SPB == 0) {
      // TOKS = 8: result rows 4 qd + v hold term v & 1 of token 2 qd + v / 2
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < kTPL; ++v)
          racc[j][v] = fmaf(bsc[j], TOKS == 16 ? tmp[j][v] : tmp[j][2 * v] + tmp[j][2 * v + 1],
                            racc[j][v]);
    }
    if ((i + 1) % kUnitSteps == 0) {
      const int4 e4 = ue[i / kUnitSteps];
      const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < kTPL; ++v) acc[j][v] += __builtin_amdgcn_ldexpf(racc[j][v], -ev[v]);
    }
  };
  // Straight-line code (no loop, no branch around a load) keeps the
  // compiler's waits exact; the scheduling barriers keep each load where it
  // is issued.
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    step(i);
    __builtin_amdgcn_sched_barrier(0);
    if (i + WIN < kSteps) issue(i + WIN);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The wavefronts' sums meet in LDS; wavefront w then finishes the (slice,
  // token) pairs x = w, w + wpg, ...: added in wavefront order.
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < kTPL; ++v) red[(wave * kItems + j * kTPL + v) * 64 + lane] = acc[j][v];
  if constexpr (RMS) {
    if (wave == 0) {
      // the copies have landed (vmcnt counts them), then lane t adds token
      // t's units in order
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
      __asm__ volatile("" ::: "memory");
      if (lane < kTok) {
        float tot = 0.f;
        for (int u = 0; u < T / kUnitSteps; ++u) tot += sqs[u * kTok + lane];
        rinv[lane] = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
      }
    }
  }
  __syncthreads();
  float *out = seg == 0 ? Y : partials + static_cast<size_t>(seg - 1) * M * N;
  const int y_end = M * N * 4;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(out, 0, y_end, 0x00020000);
  for (int x = wave; x < kItems; x += wpg) {
    float sum = red[x * 64 + lane];
    for (int w = 1; w < wpg; ++w) sum += red[(w * kItems + x) * 64 + lane];
    const int j = x / kTPL, v = x % kTPL;
    const int n = 64 * g + 16 * j + c;
    const int tok = kTPL * qd + v;
    if constexpr (RMS) sum *= rinv[tok];
    if (H != nullptr) {
      // gate/up pairs (rows 2 n', 2 n' + 1 in lanes c, c ^ 1; N even)
      const float other = PairSwap(sum);
      const int half_n = N >> 1;
      if ((c & 1) == 0 && tok < M && n < N) H[tok * half_n + (n >> 1)] = SiluMul(sum, other);
    } else {
      if (bias != nullptr) sum += bias[min(n, N - 1)];  // one run: the bias input is added here
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum), ry,
                                            tok < M && n < N ? (tok * N + n) * 4 : y_end, 0, 0);
    }
  }
}

// Plan-time re-layout of the block scales and zero points for the kernel
// above: for group g (64 rows) and block b, Sd[g][b][c][j] is the fp32 scale
// of row 64 g + 16 j + c (0 past N) and byte j of Zd[g][b][c] its zero point
// (8 when absent or past N).
__global__ __launch_bounds__(256) void RelayoutDecodeScalesKernel(
    const float *__restrict__ S, const uint8_t *__restrict__ Z, float *__restrict__ Sd,
    uint32_t *__restrict__ Zd, int64_t N, int64_t nb, int64_t zp_row_bytes, int64_t items) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // (g, b, c)
  if (idx >= items) return;
  const int c = static_cast<int>(idx & 15);
  const int64_t gb = idx >> 4;
  const int64_t b = gb % nb, g = gb / nb;
  float4 s;
  uint32_t z = 0;
  float *sv = reinterpret_cast<float *>(&s);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = 64 * g + 16 * j + c;
    sv[j] = n < N ? S[n * nb + b] : 0.0f;
    const uint32_t zj =
        n < N && Z != nullptr ? (Z[n * zp_row_bytes + (b >> 1)] >> (4 * (b & 1))) & 0xFu : 8u;
    z |= zj << (8 * j);
  }
  reinterpret_cast<float4 *>(Sd)[idx] = s;
  if (Zd != nullptr) Zd[idx] = z;
}

struct Shape {
  int wpg, units_per_wave, segs;
};

// Runs per group (segs), wavefronts per workgroup (wpg) and units per
// wavefront (U), segs * wpg * U = K / 256: the fewest runs (partial sums)
// whose workgroups still cover 85% of the CUs, then U = 2 before U = 1 and
// the largest wpg of at least 4 (else any). Measured on MI355X at M = 16
// (kernel alone): c2 one run of 8 x 2 units 10.5 us (two runs of 4 x 2:
// 10.7); c1 four runs of 4 x 1 5.7 us (two runs of 4 x 2: 7.1); c3 (56
// units) four runs of 7 x 2, one workgroup per CU, 17.9 us per call
// against 18.5 for seven runs of 4 x 2 (1.75 workgroups per CU).
// Unit counts with no such division into at most 16 runs (a prime 43 at
// K = 11008, 74 = 2 x 37 at K = 18944, which the search above would give one
// run per unit) take runs of one length with a shorter last run: the fewest
// runs covering 85% of the CUs, each ceil(units / runs) units rounded up to
// whole wavefronts (U = 2 before 1, at least 4 wavefronts before any). The
// wavefronts past the last unit read only beyond the buffers of the weights,
// scales, zero points, image and exponents (bounds-checked buffer loads:
// zeros) and add exactly zero.
// Units of 256 k; a K that is not a whole number of them ends in a last
// unit whose steps past K read zero weights (beyond the group's records) and
// zero activations (masked by SplitActKernel).
inline int Units(const WeightView &w) { return static_cast<int>((w.K + kUnitK - 1) / kUnitK); }

// Four units per wavefront (U = 4) give wide weights with 4096 < K <= 8192
// one run where two units need two (K = 5120: 5 x 4 units, not 10 x 2 past
// the 8-wavefront bound). Taken where it lowers the busiest CU's work,
// ceil(workgroups / CUs) x 8 U steps plus 12 for the partial-sum pass of a
// split run, fewer runs on a tie: measured (us, M = 5 / 8 / 16) K = 5120,
// N = 27648 26.2 / 26.4 / 34.8 -> 20.2 / 21.0 / 29.2; K = 6144, N = 16384
// at M = 8 17.9 -> 15.5; K = 8192, N = 28672 at M = 16 43.4 -> 39.2;
// K = 14336, N = 24576 (two runs instead of four) at M = 8 / 16 47.1 /
// 62.4 -> 43.0 / 57.5. Not where one run leaves a second round on a few
// CUs (K = 7168, N = 18432, 288 groups: 22.3 / 30.8 at M = 5 / 16 with two
// runs of two units against 24.6 / 31.9).
inline int64_t ShapeCost(const Shape &sh, int64_t groups, int64_t cus) {
  return (groups * sh.segs + cus - 1) / cus * (sh.units_per_wave * kUnitSteps) +
         (sh.segs > 1 ? 12 : 0);
}

inline Shape PickShapeU12(const WeightView &w, int wpg_req, int u_req);

inline Shape PickShape(const WeightView &w, int wpg_req, int u_req) {
  Shape best = PickShapeU12(w, wpg_req, u_req);
  if (wpg_req > 0 || u_req > 0) return best;
  const int64_t groups = (w.N + 63) / 64, cus = std::max<int64_t>(1, w.num_cus);
  const int units = Units(w);
  for (int segs = 1; segs <= std::min(units, 16); ++segs) {
    if (units % segs != 0 || (units / segs) % 4 != 0) continue;
    const int wpg = units / segs / 4;
    if (wpg < 4 || wpg > kMaxWaves) continue;
    if (segs < units && groups * segs * 100 < cus * 85) continue;
    const Shape u4{wpg, 4, segs};
    const int64_t c4 = ShapeCost(u4, groups, cus), cb = ShapeCost(best, groups, cus);
    if (c4 < cb || (c4 == cb && segs < best.segs)) best = u4;
    break;  // the fewest runs
  }
  return best;
}

inline Shape PickShapeU12(const WeightView &w, int wpg_req, int u_req) {
  const int64_t groups = (w.N + 63) / 64;
  const int units = Units(w);
  Shape sh{1, 1, units};
  if (wpg_req > 0 || u_req > 0) {
    sh.units_per_wave = u_req > 0 ? u_req : 1;
    sh.wpg = wpg_req > 0 ? wpg_req : 1;
    sh.segs = units / (sh.units_per_wave * sh.wpg);
    return sh;
  }
  for (int segs = 1; segs <= std::min(units, 16); ++segs) {
    if (units % segs != 0) continue;
    const int per = units / segs;  // units per workgroup
    if (segs < units && groups * segs * 100 < static_cast<int64_t>(w.num_cus) * 85) continue;
    for (int min_wpg : {4, 1})
      for (int U : {2, 1})
        for (int wpg : {8, 7, 6, 5, 4, 3, 2, 1})
          if (wpg >= min_wpg && wpg * U == per) return Shape{wpg, U, segs};
  }
  for (int segs = 2; segs <= units; ++segs) {
    if (segs < units && groups * segs * 100 < static_cast<int64_t>(w.num_cus) * 85) continue;
    for (int min_wpg : {4, 1})
      for (int U : {2, 1}) {
        const int per = ((units + segs - 1) / segs + U - 1) / U * U;  // units per run
        const int wpg = per / U;
        if (wpg < min_wpg || wpg > kMaxWaves || (units + per - 1) / per != segs) continue;
        return Shape{wpg, U, segs};
      }
  }
  return sh;
}

inline size_t ImageBytes(const WeightView &w) {
  return static_cast<size_t>(Units(w)) * kUnitSteps * kStepBytes;
}
inline size_t ExpBytes(const WeightView &w) {
  return (static_cast<size_t>(Units(w)) * kTok * 4 + 255) / 256 * 256;
}
// The per-unit sums of squares of a fused RMSNorm input: the same size.
inline size_t SqBytes(const WeightView &w) { return ExpBytes(w); }

// The workspace's image, exponents, per-unit sums of squares (RMS) and
// partial sums; sq is null without RMSNorm.
struct Work {
  const uint4 *img;
  const int *exps;
  const float *sq;
  float *P;
  float eps;
};

template <bool HAS_ZP, int SPB, int U, int TOKS>
hipError_t LaunchMain(const WeightView &w, int64_t M, const Work &wk, float *Y, float *H,
                      const float *bias, const Shape &sh, hipStream_t s) {
  const int64_t groups = (w.N + 63) / 64;
  constexpr int kWin = 4;
  const dim3 grid(static_cast<unsigned>(groups * sh.segs)), block(64 * sh.wpg);
  const int m = static_cast<int>(M), n = static_cast<int>(w.N), k = static_cast<int>(w.K),
            nb = static_cast<int>(w.nb);
  if (wk.sq != nullptr)
    hipLaunchKernelGGL((DecodeFragKernel<HAS_ZP, SPB, U, kWin, true, TOKS>), grid, block, 0, s, w.Bp,
                       w.Sd, w.Zd, wk.img, wk.exps, Y, wk.P, H, bias, m, n, k, nb, w.log2_bs,
                       sh.segs, sh.wpg, wk.sq, wk.eps);
  else
    hipLaunchKernelGGL((DecodeFragKernel<HAS_ZP, SPB, U, kWin, false, TOKS>), grid, block, 0, s, w.Bp,
                       w.Sd, w.Zd, wk.img, wk.exps, Y, wk.P, H, bias, m, n, k, nb, w.log2_bs,
                       sh.segs, sh.wpg, nullptr, 0.0f);
  return hipGetLastError();
}

template <bool HAS_ZP, int SPB>
hipError_t LaunchU(const WeightView &w, int64_t M, const Work &wk, float *Y, float *H,
                   const float *bias, const Shape &sh, hipStream_t s) {
  if (M <= 8)
    return sh.units_per_wave == 4   ? LaunchMain<HAS_ZP, SPB, 4, 8>(w, M, wk, Y, H, bias, sh, s)
           : sh.units_per_wave == 2 ? LaunchMain<HAS_ZP, SPB, 2, 8>(w, M, wk, Y, H, bias, sh, s)
                                    : LaunchMain<HAS_ZP, SPB, 1, 8>(w, M, wk, Y, H, bias, sh, s);
  return sh.units_per_wave == 4   ? LaunchMain<HAS_ZP, SPB, 4, 16>(w, M, wk, Y, H, bias, sh, s)
         : sh.units_per_wave == 2 ? LaunchMain<HAS_ZP, SPB, 2, 16>(w, M, wk, Y, H, bias, sh, s)
                                  : LaunchMain<HAS_ZP, SPB, 1, 16>(w, M, wk, Y, H, bias, sh, s);
}

template <bool HAS_ZP>
hipError_t LaunchZp(const WeightView &w, int64_t M, const Work &wk, float *Y, float *H,
                    const float *bias, const Shape &sh, hipStream_t s) {
  switch (std::min(w.block_size / 32, kUnitSteps)) {
  case 1: return LaunchU<HAS_ZP, 1>(w, M, wk, Y, H, bias, sh, s);
  case 2: return LaunchU<HAS_ZP, 2>(w, M, wk, Y, H, bias, sh, s);
  case 4: return LaunchU<HAS_ZP, 4>(w, M, wk, Y, H, bias, sh, s);
  default: return LaunchU<HAS_ZP, 8>(w, M, wk, Y, H, bias, sh, s);
  }
}

} // namespace df

bool DecodeFragLayoutWanted(const WeightView &w) {
  return (w.K % 32) == 0 && w.block_size >= 32 &&
         (w.block_size & (w.block_size - 1)) == 0 && w.K <= (int64_t{1} << 24) &&
         w.N < (int64_t{1} << 22) && w.nb * 256 < (int64_t{1} << 31);
}

size_t DecodeFragScaleBytes(const WeightView &w, size_t *zd_bytes) {
  const int64_t items = (w.N + 63) / 64 * w.nb * 16;
  if (zd_bytes != nullptr) *zd_bytes = w.has_zp ? static_cast<size_t>(items) * 4 : 0;
  return static_cast<size_t>(items) * 16;
}

hipError_t LaunchDecodeFragRelayout(const WeightView &w, float *Sd, uint32_t *Zd, hipStream_t s) {
  const int64_t items = (w.N + 63) / 64 * w.nb * 16;
  hipLaunchKernelGGL(df::RelayoutDecodeScalesKernel, dim3(static_cast<unsigned>((items + 255) / 256)),
                     dim3(256), 0, s, w.scales, w.zp, Sd, Zd, w.N, w.nb, w.zp_row_bytes, items);
  return hipGetLastError();
}

bool DecodeFragSupports(const WeightView &w, int64_t M) {
  return M >= 2 && M <= 16 && w.Bp != nullptr && w.Sd != nullptr &&
         (!w.has_zp || w.Zd != nullptr) && DecodeFragLayoutWanted(w) &&
         M * w.K * 4 + 4096 < (int64_t{1} << 31) && M * w.N * 4 < (int64_t{1} << 31) &&
         (w.K / 32) * df::kStepBytes < (int64_t{1} << 31);
}

bool DecodeFragTakesRms(const WeightView &w) {
  return w.K <= df::kMaxSqUnits * df::kUnitK && (w.K % df::kUnitK) == 0;
}

size_t DecodeFragWorkspaceBytes(const WeightView &w, int64_t M, int wpg, int units_per_wave) {
  const df::Shape sh = df::PickShape(w, wpg, units_per_wave);
  return df::ImageBytes(w) + df::ExpBytes(w) + df::SqBytes(w) +
         static_cast<size_t>(std::max(sh.segs, 1) - 1) * static_cast<size_t>(M) * w.N * 4;
}

hipError_t LaunchDecodeFrag(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                            hipStream_t s, float *H, int wpg, int units_per_wave,
                            const float *bias, const float *gamma, float eps) {
  const df::Shape sh = df::PickShape(w, wpg, units_per_wave);
  const int units = df::Units(w);
  // every unit in a run, no run empty (the last may be shorter)
  if (sh.wpg < 1 || sh.wpg > df::kMaxWaves || sh.segs < 1 ||
      sh.segs * sh.wpg * sh.units_per_wave < units ||
      (sh.segs - 1) * sh.wpg * sh.units_per_wave >= units ||
      (sh.units_per_wave != 1 && sh.units_per_wave != 2 && sh.units_per_wave != 4))
    return hipErrorInvalidValue;
  if (gamma != nullptr && !DecodeFragTakesRms(w)) return hipErrorInvalidValue;
  if (gamma != nullptr && (reinterpret_cast<uintptr_t>(gamma) % 16) != 0) return hipErrorInvalidValue;
  char *base = static_cast<char *>(work);
  uint4 *img = reinterpret_cast<uint4 *>(base);
  int *exps = reinterpret_cast<int *>(base + df::ImageBytes(w));
  float *sq = reinterpret_cast<float *>(base + df::ImageBytes(w) + df::ExpBytes(w));
  float *P = reinterpret_cast<float *>(base + df::ImageBytes(w) + df::ExpBytes(w) + df::SqBytes(w));
  // up to 8 rows: both terms of a token in one MFMA operand (half the image)
  const bool t8 = M <= 8;
  const dim3 sgrid(static_cast<unsigned>(units * (t8 ? 4 : 8))), sblock(64);
  if (gamma != nullptr && t8)
    hipLaunchKernelGGL((df::SplitActKernel<true, 8>), sgrid, sblock, 0, s, A, img, exps, sq, gamma,
                       static_cast<int>(M), static_cast<int>(w.K));
  else if (gamma != nullptr)
    hipLaunchKernelGGL((df::SplitActKernel<true, 16>), sgrid, sblock, 0, s, A, img, exps, sq, gamma,
                       static_cast<int>(M), static_cast<int>(w.K));
  else if (t8)
    hipLaunchKernelGGL((df::SplitActKernel<false, 8>), sgrid, sblock, 0, s, A, img, exps, nullptr,
                       nullptr, static_cast<int>(M), static_cast<int>(w.K));
  else
    hipLaunchKernelGGL((df::SplitActKernel<false, 16>), sgrid, sblock, 0, s, A, img, exps, nullptr,
                       nullptr, static_cast<int>(M), static_cast<int>(w.K));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // One run per group: the kernel writes Y (or H) itself and adds the bias.
  float *Hk = sh.segs == 1 ? H : nullptr;
  const float *bk = sh.segs == 1 ? bias : nullptr;
  const df::Work wk{img, exps, gamma != nullptr ? sq : nullptr, P, eps};
  e = w.has_zp ? df::LaunchZp<true>(w, M, wk, Y, Hk, bk, sh, s)
                      : df::LaunchZp<false>(w, M, wk, Y, Hk, bk, sh, s);
  if (e != hipSuccess || sh.segs == 1) return e;
  return LaunchSumPartials(Y, P, M * w.N, sh.segs - 1, H, s, bias, w.N);
}

} // namespace mnb
