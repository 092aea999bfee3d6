// Decode GEMV for 2 <= M <= 16 activation rows (fp32 FMA).
//
// Role in the reference: the roadmap's `int4_gemv` / `int4_small_m` decode
// side (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-221): fp32
// accumulation, weights never expanded, each weight byte streamed once per
// group of up to 4 activation rows ("tokens").
//
// Per nibble the work is one FMA per token, so from M of about 2 on the path
// is bound by the fp32 VALU rate (one wave64 FMA per clock per CU, measured),
// not by HBM; everything else is arranged to stay off that pipe:
//  - the nibble decode is shared by all tokens of the group: masking a packed
//    word w and w >> 8 with 0x000F000F / 0x00F000F0 gives two nibbles per mask
//    as the exact fp16 subnormals q * 2^-24 or q * 2^-20, and one packed fp16
//    add of -zp * 2^-24 (or -zp * 2^-20) makes (q - zp) * 2^-24 (* 16) exactly
//    (|q - zp| <= 15): nine operations per eight nibbles and row, then
//    v_fma_mix_f32 multiplies fp32 activations by those fp16 values directly.
//    This relies on fp16 subnormals being kept (the gfx950 HIP default FP16
//    denormal mode), as the parity tests check;
//  - A is staged in LDS one slice of 64 chunks (2048 k) per token at a time,
//    double-buffered: slice i + 1 is loaded into registers while slice i is
//    multiplied and written (swizzled) to the other buffer behind it; one
//    barrier per slice. Plain register loads keep every wait exact (the
//    compiler counts them; direct global->LDS copies made it either wait for
//    everything or, hidden from it, over-wait);
//  - each wavefront stages the (scale, zp) pairs of its own rows in a
//    wave-private LDS region (no workgroup barrier), as the M = 1 kernel does.
//
// Mapping: a workgroup of W wavefronts owns a band of G = W * R consecutive
// weight rows; lane l takes chunk c = 64 i + l of each row in slice i (1 KiB
// coalesced per load instruction). Per (row, token) the lane accumulates
//   acc += (scale 2^24) * sum_j a_j (q_j - zp) 2^-24
// and a DPP + readlane reduction gives each output.
#include "mnb_decode_common.h"

#include <algorithm>

namespace mnb {
namespace sm {

using namespace dec;

constexpr int kMaxTokens = 8;  // tokens per launch group (largest instantiated)

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
// Native 4-float vector for the A staging copies (float4 is a struct whose
// copies become memcpy calls that keep the staging array in scratch).
typedef float f32x4 __attribute__((ext_vector_type(4)));

// LDS layout: two slice buffers of MT * 512 float4 (per token 64 chunks of 8
// float4, float4 v of chunk c stored at c * 8 + (v ^ ((c ^ c >> 3) & 7))),
// then per wavefront its R * nb pairs (scale, zp), plus 4 spare pairs. In the
// token loop lanes l and l + 8 read chunks 1 KiB apart; an XOR by c & 7 alone
// would leave their reads in the same banks.
__host__ __device__ inline size_t SliceF4(int mt) { return static_cast<size_t>(mt) * 512; }
inline size_t LdsBytes(int mt, int waves, int R, int64_t nb) {
  return 2 * SliceF4(mt) * 16 + (static_cast<size_t>(waves) * R * nb + 4) * 8;
}

// (h + negc) per fp16 half: h holds q * 2^-24 (or * 2^-20), negc -zp at the
// same scale; the result (q - zp) * scale is exact.
__device__ __forceinline__ uint32_t SubZp(uint32_t h, uint32_t negc) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, h) + __builtin_bit_cast(half2v, negc));
}

// Decoded nibbles of one 16-byte chunk for one row: hz[4t + u] holds the two
// nibbles u | u + 4 of word t as (q - zp) 2^-24 (u even) or (q - zp) 2^-20
// (u odd).
__device__ __forceinline__ void Decode(const uint4 &w4, uint32_t n24, uint32_t n20, uint32_t *hz) {
  const uint32_t words[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t w = words[t];
    const uint32_t w8 = w >> 8;
    hz[4 * t + 0] = SubZp(w & 0x000F000Fu, n24);   // nibbles 0 | 4
    hz[4 * t + 1] = SubZp(w & 0x00F000F0u, n20);   // nibbles 1 | 5
    hz[4 * t + 2] = SubZp(w8 & 0x000F000Fu, n24);  // nibbles 2 | 6
    hz[4 * t + 3] = SubZp(w8 & 0x00F000F0u, n20);  // nibbles 3 | 7
  }
}

// e += sum over words t0, t0 + 1 of the even-scaled products, o of the odd
// ones (a holds the 16 activations of those two words, k order).
__device__ __forceinline__ void DotHalf(const float *a, const uint32_t *hz, int t0, float &e,
                                        float &o, bool first) {
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint32_t *h = hz + 4 * (t0 + tt);
    const float *x = a + 8 * tt;
    if (first && tt == 0) {
      e = MixLo0(x[0], h[0]);
      o = MixLo0(x[1], h[1]);
    } else {
      MixLo(e, x[0], h[0]);
      MixLo(o, x[1], h[1]);
    }
    MixHi(e, x[4], h[0]);
    MixHi(o, x[5], h[1]);
    MixLo(e, x[2], h[2]);
    MixHi(e, x[6], h[2]);
    MixLo(o, x[3], h[3]);
    MixHi(o, x[7], h[3]);
  }
}

// Slice i of A: MT * 512 float4, thread t of the W-wavefront workgroup holds
// slots s = 64 W p + t (W divides 8 MT):
// token s / 512, chunk 64 i + (s / 8) % 64 (zeros past the last chunk: the
// load re-reads the last chunk in bounds, and its values, an infinity among
// them, must not reach the products that the zero scale of those lanes
// multiplies), float4 v = s % 8 of it; stored at LDS slot (token, chunk c,
// v ^ ((c ^ c >> 3) & 7)).
template <int MT, int W>
__device__ __forceinline__ void LoadSlice(f32x4 (&st)[MT * 8 / W], const f32x4 *a4, int K4, int i,
                                          int nchunks) {
#pragma unroll
  for (int p = 0; p < MT * 8 / W; ++p) {
    const int sl = 64 * W * p + threadIdx.x;
    const int m = sl >> 9, cl = (sl >> 3) & 63, v = sl & 7;
    const int c = min(64 * i + cl, nchunks - 1);
    const f32x4 x = a4[static_cast<size_t>(m) * K4 + c * 8 + v];
    st[p] = 64 * i + cl < nchunks ? x : f32x4{0.f, 0.f, 0.f, 0.f};
  }
}
template <int MT, int W>
__device__ __forceinline__ void StoreSlice(const f32x4 (&st)[MT * 8 / W], float4 *lds) {
  f32x4 *dst = reinterpret_cast<f32x4 *>(lds);
#pragma unroll
  for (int p = 0; p < MT * 8 / W; ++p) {
    const int sl = 64 * W * p + threadIdx.x;
    const int m = sl >> 9, cl = (sl >> 3) & 63, v = sl & 7;
    dst[m * 512 + cl * 8 + (v ^ ((cl ^ (cl >> 3)) & 7))] = st[p];
  }
}

template <int MT, int R, int W, bool HAS_ZP, int PW>
__global__ __launch_bounds__(64 * W) void GemvSmallMKernel(const float *__restrict__ A,
                                                        const uint8_t *__restrict__ B,
                                                        const float *__restrict__ S,
                                                        const uint8_t *__restrict__ Z,
                                                        float *__restrict__ Y, int K, int N,
                                                        int nb, int chunk_shift, int row_bytes,
                                                        int zp_row_bytes, int G) {
  extern __shared__ float4 lds4[];
  const int nchunks = K >> 5;
  const int nslices = (nchunks + 63) >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform
  const int row0 = blockIdx.x * G;    // first row of the band
  const int rows = min(G, N - row0);  // rows in the band
  const int wr0 = wave * R;           // first band row of this wavefront
  const int last_row = row0 + rows - 1;
  const int K4 = K >> 2;              // float4 per token row of A

  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(B), 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(S), 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(HAS_ZP ? Z : B), 0, 0x7FFFFFFF, 0x00020000);

  float2 *pair_lds = reinterpret_cast<float2 *>(lds4 + 2 * SliceF4(MT));
  float2 *wpairs = pair_lds + wr0 * nb;  // this wavefront's pairs
  const int spare_rel = W * R * nb - wr0 * nb;
  const f32x4 *a4 = reinterpret_cast<const f32x4 *>(A);

  auto load_w = [&](uint4 *w, int i) __attribute__((always_inline)) {
    const int c = min(64 * i + lane, nchunks - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = __builtin_amdgcn_readfirstlane(min(row0 + wr0 + r, last_row));
      w[r] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, c * 16, row * row_bytes, kNonTemporal));
    }
  };

  // 1. slice 0, this wavefront's (scale, zp) pairs, weights of slice 0
  {
    f32x4 st0[MT * 8 / W];
    LoadSlice<MT, W>(st0, a4, K4, 0, nchunks);
    StoreSlice<MT, W>(st0, lds4);
  }
  const int nitems = R * nb / PW;
  const float rnb = 1.0f / static_cast<float>(nb);
  PairItem<PW, HAS_ZP> pi[2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    pi[q].Load(64 * q + lane, nitems, nb, rnb, row0 + wr0, last_row, zp_row_bytes, rsc, rz);
  uint4 w[R];
  load_w(w, 0);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 2; ++q) pi[q].Store(wpairs, spare_rel);
  for (int i0 = 128; i0 < nitems; i0 += 64) {
    PairItem<PW, HAS_ZP> it;
    it.Load(i0 + lane, nitems, nb, rnb, row0 + wr0, last_row, zp_row_bytes, rsc, rz);
    it.Store(wpairs, spare_rel);
  }

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  // One slice step: decode this slice's weights, put slice i + 1 in flight
  // (A into registers, then weights), the token loop from LDS and registers,
  // then slice i + 1 into the other LDS buffer and the barrier that
  // publishes it.
  const int sw = (lane ^ (lane >> 3)) & 7;  // chunk lane's slot swizzle
  auto step = [&](int i, int b, const uint4 *cur, uint4 *nxt) __attribute__((always_inline)) {
    const int c = 64 * i + lane;
    const int blk = min(c, nchunks - 1) >> chunk_shift;
    uint32_t hz[R][16];
    float s24[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float2 sz = wpairs[r * nb + blk];
      const uint32_t zp = static_cast<uint32_t>(sz.y * 16777216.f + 0.5f);
      const uint32_t n24 = (zp * 0x00010001u) | 0x80008000u;
      const uint32_t n20 = ((zp << 4) * 0x00010001u) | 0x80008000u;
      s24[r] = c < nchunks ? sz.x : 0.f;  // chunks past K contribute nothing
      Decode(cur[r], n24, n20, hz[r]);
    }
    // Unconditional (the last step re-reads the last slice): a staging array
    // filled under a branch is not promoted to registers.
    const int in = min(i + 1, nslices - 1);
    f32x4 st[MT * 8 / W];
    LoadSlice<MT, W>(st, a4, K4, in, nchunks);
    load_w(nxt, in);
    // Keep the order: the scheduler would otherwise hoist the slice stores
    // (provably another buffer) right behind their loads, each then waiting
    // for its load.
    __builtin_amdgcn_sched_barrier(0);
    const float4 *ab = lds4 + b * SliceF4(MT) + lane * 8;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float e[R], o[R];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float a[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float4 t = ab[m * 512 + ((4 * half + v) ^ sw)];
          a[4 * v] = t.x;
          a[4 * v + 1] = t.y;
          a[4 * v + 2] = t.z;
          a[4 * v + 3] = t.w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) DotHalf(a, hz[r], 2 * half, e[r], o[r], half == 0);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][m] = fmaf(s24[r], fmaf(o[r], 0.0625f, e[r]), acc[r][m]);
    }
    __builtin_amdgcn_sched_barrier(0);
    StoreSlice<MT, W>(st, lds4 + (b ^ 1) * SliceF4(MT));
    __syncthreads();
  };
  uint4 wb[R];
  for (int i = 0; i < nslices; i += 2) {
    step(i, 0, w, wb);
    if (i + 1 < nslices) step(i + 1, 1, wb, w);
  }

  // one total per (row, token); lane r * MT + m stores it
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float t = WaveTotal(acc[r][m]);
      mine = lane == r * MT + m ? t : mine;
    }
  const int r = lane / MT, m = lane - r * MT;
  if (lane < R * MT && wr0 + r < rows) Y[static_cast<size_t>(m) * N + row0 + wr0 + r] = mine;
}

struct Shape {
  int G, R, W, grid, max_tokens;
  size_t lds;
};

// Bands as the M = 1 kernel: the same number of rows on every CU, in
// workgroups of W wavefronts x R rows. Arguments <= 0 take the defaults.
// The A values a lane reads from LDS serve R rows, so at R = 2 the LDS
// bandwidth (128 B per clock per CU) is about as busy as the FMA pipe.
inline Shape PickShape(const WeightView &w, int max_tokens, int W, int R) {
  const int rows_per_cu = static_cast<int>((w.N + w.num_cus - 1) / w.num_cus);
  Shape sh{};
  // Defaults from the MI355X sweep (c2 M = 4, 16; c3 M = 2, 8): 4-token
  // groups, 8 wavefronts x 2 rows.
  sh.max_tokens = max_tokens > 0 ? max_tokens : 4;
  sh.W = W > 0 ? W : 8;
  sh.R = R > 0 ? R : 2;
  const int per_wg = sh.W * sh.R;
  const int k = (rows_per_cu + per_wg - 1) / per_wg;
  sh.G = (rows_per_cu + k - 1) / k;
  sh.grid = static_cast<int>((w.N + sh.G - 1) / sh.G);
  sh.lds = LdsBytes(sh.max_tokens, sh.W, sh.R, w.nb);
  return sh;
}

template <int MT, int R, int W, bool HAS_ZP>
hipError_t LaunchT(const WeightView &w, const float *A, float *Y, hipStream_t s, const Shape &sh) {
  const dim3 grid(static_cast<unsigned>(sh.grid)), block(static_cast<unsigned>(W * 64));
  const int K = static_cast<int>(w.K), N = static_cast<int>(w.N), nb = static_cast<int>(w.nb);
  const int cs = w.log2_bs - 5, rb = static_cast<int>(w.row_bytes);
  const int zb = static_cast<int>(w.zp_row_bytes);
  const size_t lds = LdsBytes(MT, W, R, w.nb);
  if (w.nb % 4 == 0)
    hipLaunchKernelGGL((GemvSmallMKernel<MT, R, W, HAS_ZP, 4>), grid, block, lds, s, A, w.B,
                       w.scales, w.zp, Y, K, N, nb, cs, rb, zb, sh.G);
  else
    hipLaunchKernelGGL((GemvSmallMKernel<MT, R, W, HAS_ZP, 1>), grid, block, lds, s, A, w.B,
                       w.scales, w.zp, Y, K, N, nb, cs, rb, zb, sh.G);
  return hipGetLastError();
}

template <int MT, bool HAS_ZP>
hipError_t LaunchRW(const WeightView &w, const float *A, float *Y, hipStream_t s, const Shape &sh) {
  if (sh.G > sh.W * sh.R) return hipErrorInvalidValue;
#define MNB_SM_RW(RR, WW) \
  if (sh.R == RR && sh.W == WW) return LaunchT<MT, RR, WW, HAS_ZP>(w, A, Y, s, sh);
  MNB_SM_RW(1, 4) MNB_SM_RW(2, 4) MNB_SM_RW(4, 4)
  MNB_SM_RW(1, 8) MNB_SM_RW(2, 8) MNB_SM_RW(4, 8)
#undef MNB_SM_RW
  return hipErrorInvalidValue;
}

template <bool HAS_ZP>
hipError_t LaunchGroup(const WeightView &w, int mt, const float *A, float *Y, hipStream_t s,
                       const Shape &sh) {
  switch (mt) {
  case 1: return LaunchRW<1, HAS_ZP>(w, A, Y, s, sh);
  case 2: return LaunchRW<2, HAS_ZP>(w, A, Y, s, sh);
  case 3: return LaunchRW<3, HAS_ZP>(w, A, Y, s, sh);
  case 4: return LaunchRW<4, HAS_ZP>(w, A, Y, s, sh);
  case 5: return LaunchRW<5, HAS_ZP>(w, A, Y, s, sh);
  case 6: return LaunchRW<6, HAS_ZP>(w, A, Y, s, sh);
  case 7: return LaunchRW<7, HAS_ZP>(w, A, Y, s, sh);
  default: return LaunchRW<8, HAS_ZP>(w, A, Y, s, sh);
  }
}

} // namespace sm

bool GemvSmallMSupports(const WeightView &w, int64_t M) {
  // 32-bit buffer offsets; 16-byte scale loads (nb % 4 == 0 path) and 2-byte
  // zero-point loads need aligned bases; the default shape must fit the LDS.
  if (w.B == nullptr || M < 2 || M > 16 || (w.K % 32) != 0 || w.block_size < 32 ||
      (w.row_bytes % 16) != 0)
    return false;
  if ((reinterpret_cast<uintptr_t>(w.B) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(w.scales) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(w.zp) % 2) != 0)
    return false;
  if (w.row_bytes * w.N >= (int64_t{1} << 31) || w.nb * 4 * w.N >= (int64_t{1} << 31) ||
      w.K * 4 * M >= (int64_t{1} << 31))
    return false;
  return sm::PickShape(w, 0, 0, 0).lds <= 160 * 1024;
}

hipError_t LaunchGemvSmallMShape(const WeightView &w, int64_t M, const float *A, float *Y,
                                 hipStream_t s, int max_tokens, int waves, int rows_per_wave) {
  const sm::Shape sh = sm::PickShape(w, max_tokens, waves, rows_per_wave);
  if (sh.max_tokens < 1 || sh.max_tokens > sm::kMaxTokens || sh.lds > 160 * 1024)
    return hipErrorInvalidValue;
  // Balanced groups of at most max_tokens tokens, one launch each.
  const int groups = static_cast<int>((M + sh.max_tokens - 1) / sh.max_tokens);
  int64_t m0 = 0;
  for (int g = 0; g < groups; ++g) {
    const int mt = static_cast<int>((M - m0) / (groups - g));
    const float *Ag = A + m0 * w.K;
    float *Yg = Y + m0 * w.N;
    const hipError_t e = w.zp ? sm::LaunchGroup<true>(w, mt, Ag, Yg, s, sh)
                              : sm::LaunchGroup<false>(w, mt, Ag, Yg, s, sh);
    if (e != hipSuccess) return e;
    m0 += mt;
  }
  return hipSuccess;
}

hipError_t LaunchGemvSmallM(const WeightView &w, int64_t M, const float *A, float *Y,
                            hipStream_t s) {
  return LaunchGemvSmallMShape(w, M, A, Y, s, 0, 0, 0);
}

} // namespace mnb
