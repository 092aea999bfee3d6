// Decode GEMV for 2 <= M <= 16 activation rows on fp16 MFMA with fp32-exact
// products.
//
// Role in the reference: the roadmap's `int4_gemv` / `int4_small_m` decode
// side (docs/next_steps/2026/2026_08_qwen3_inference.rst:208-221): every
// product a * (q - zp) is formed exactly and the products are summed in fp32,
// as on the fp32 FMA paths, but on the matrix cores:
//  - each activation row (token) is scaled by a power of two 2^e that puts
//    its largest magnitude in the workgroup's k range in [2^14, 2^15), and
//    every scaled value is split into three fp16 terms, a 2^e = a0 + a1 + a2
//    (each difference is exact in fp32 and 3 x 11 significand bits cover
//    fp32's 24; only parts below about 2^-39 of that largest magnitude fall
//    under fp16's subnormal range and are rounded);
//  - q - zp is an integer in [-15, 15], exact in fp16 (exponent-constant
//    decode, no rounding), so each v_mfma_f32_16x16x32_f16 of a term forms
//    exact products and sums them in fp32;
//  - each MFMA covers 32 k of one quantization block; its three terms'
//    results accumulate into one fp32 tile, which is multiplied by the
//    block's fp32 scale into the output accumulator; 2^-e is applied at the
//    end (exact unless the output is an fp32 subnormal).
// Why: the fp32 FMA paths do one FMA per nibble and token, so at M = 16 they
// run at 5 % of HBM bandwidth (VALU and LDS bound). Three 16x16x32 fp16 MFMAs
// cover 16 tokens x 16 weight rows x 32 k, and the VALU work per nibble no
// longer depends on M.
//
// Mapping (16x16x32 f16 layout as in the prefill GEMM: lane l supplies A row
// l & 15 / B column l & 15 with 8 k of unit l >> 4; value v of lane l is
// D[4 (l >> 4) + v][l & 15]):
//  - MFMA rows are the 16 tokens (rows past M are zero), columns 16 weight
//    rows; a wavefront owns RB blocks of 16 weight rows, a workgroup 4
//    wavefronts, over one range of 512 k (K is split over workgroups in
//    ranges of 512);
//  - k runs in groups of 128: lane (c = l & 15, g = l >> 4) loads the 16
//    bytes at 64 group + 16 g of weight row c (one 32-k chunk). With blocks
//    of 128 k or more, MFMA j of the group takes dword j of every lane (k =
//    128 group + 32 g + 8 j + 0..7, one block). With blocks of 32 or 64 k the
//    four lanes of a row first transpose their dwords (v_permlane32_swap and
//    v_permlane16_swap), so that MFMA j covers chunk j of the group (k = 128
//    group + 32 j + 8 g + 0..7) and needs one scale;
//  - decode is a streaming problem (each weight byte is used once), and only
//    bytes in flight hide HBM latency: every wavefront issues all the loads of
//    its range (per 16-row block: four 16-byte weight loads, one scale and
//    one zero-point load per lane) at once, right after its activation
//    loads, and splits the activations into LDS (in the operand order above)
//    while they are in flight;
//  - the partial sums of the ranges are added in range order (split 0 writes
//    Y, the others a workspace, SumPartialsKernel adds them to Y), so results
//    do not depend on scheduling.
#include "mnb_decode_common.h"

#include <algorithm>
#include <type_traits>

namespace mnb {
namespace mf {

using namespace dec;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTok = 16;                              // tokens per MFMA tile (M padded)
constexpr int kWaves = 4;                             // wavefronts per workgroup
constexpr int kKR = 512;                              // k per workgroup
constexpr int kSteps = kKR / 32;                      // 32-k MFMA steps per range
constexpr int kStepUnits = 4 * kTok;                  // 16-byte A units per step and term
constexpr int kTermUnits = kSteps * kStepUnits;       // 1024
constexpr int kMaxSplits = 64;

__device__ __forceinline__ uint32_t PkAddF16(uint32_t a, uint32_t b) {
  const half2v r = __builtin_bit_cast(half2v, a) + __builtin_bit_cast(half2v, b);
  return __builtin_bit_cast(uint32_t, r);
}

struct Masks {
  uint32_t lo, hi, e1024, e64;  // 0x000F000F, 0x00F000F0, fp16 pairs 1024.0, 64.0
};
__device__ __forceinline__ Masks MakeMasks() {
  Masks c{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  // Held in VGPRs: v_and_or_b32 (VOP3) takes no literal operand on gfx9.
  __asm__ volatile("" : "+v"(c.lo), "+v"(c.hi), "+v"(c.e1024), "+v"(c.e64));
  return c;
}

// 8 nibbles (k order) of one word -> q - zp as fp16 in [0,4,1,5,2,6,3,7]
// order, exact: (w & 0x000F000F) | 0x6400.. is the fp16 pair 1024 + q of
// nibbles 0 | 4 (ulp 1 at 1024), (w & 0x00F000F0) | 0x5400.. the pair 64 + q
// of nibbles 1 | 5 (ulp 1/16 at 64); the same of w >> 8 gives nibbles 2 | 6
// and 3 | 7. neg_lo / neg_hi are the fp16 pairs -(1024 + zp) / -(64 + zp).
__device__ __forceinline__ half8 DecodeQ(uint32_t w, uint32_t neg_lo, uint32_t neg_hi,
                                         const Masks &c) {
  const uint32_t w8 = w >> 8;
  const uint4 r = make_uint4(PkAddF16((w & c.lo) | c.e1024, neg_lo),
                             PkAddF16((w & c.hi) | c.e64, neg_hi),
                             PkAddF16((w8 & c.lo) | c.e1024, neg_lo),
                             PkAddF16((w8 & c.hi) | c.e64, neg_hi));
  return __builtin_bit_cast(half8, r);
}

// Transposes the 4 x 4 dwords held by lanes c, c + 16, c + 32, c + 48 in
// v[0..3] (lane group g, register j -> lane group j, register g): one
// v_permlane32_swap per pair (0, 2), (1, 3) exchanges the off-diagonal 2 x 2
// blocks, one v_permlane16_swap per pair (0, 1), (2, 3) the elements inside
// them.
__device__ __forceinline__ void Transpose4(u32x4 &v) {
  auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  v = u32x4{c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ uint32_t FromLane(int byte_addr, uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(byte_addr, static_cast<int>(v)));
}

// Per (row, range) scales and zero points, loaded cooperatively by the 4
// lanes of a row (lane group g covers the 128 k of group g) and handed to the
// other lanes with ds_bpermute when group g is multiplied. BSC = 32-k chunks
// per block, capped at 4: BSC = 4 (block_size >= 128): the scale and
// zero-point byte of group g's block; BSC = 2 (64): the 2 scales (8 B) and the
// zero-point byte of group g's 2 blocks; BSC = 1 (32): the 4 scales (16 B)
// and the 2 zero-point bytes of group g's 4 blocks.
template <int BSC>
struct RowConsts {
  using ST = typename std::conditional<BSC == 4, uint32_t,
                                       typename std::conditional<BSC == 2, u32x2, u32x4>::type>::type;
  ST s;
  uint32_t z;
};

// A wavefront's item t (t < 2 PAIRS): row blocks RB (wis + t * waves_per_split)
// + r (16 rows each) of its split's k range. Rows past N load past the end of
// their buffers (zeros, no memory traffic) and store nothing. Split 0 writes
// Y; split p > 0 writes partials[p - 1].
template <int BSC, int RB, int PAIRS, int WIN, bool HAS_ZP>
__global__ __launch_bounds__(64 * kWaves) void GemvMfmaKernel(
    const float *__restrict__ A, const uint8_t *__restrict__ B, const float *__restrict__ S,
    const uint8_t *__restrict__ Z, float *__restrict__ Y, float *__restrict__ partials, int M,
    int K, int N, int nb, int log2_bs, int row_bytes, int zp_row_bytes, int splits,
    int waves_per_split) {
  constexpr bool kTr = BSC < 4;        // blocks shorter than 128 k: transpose each group
  constexpr int kGroups = kKR / 128;   // 128-k groups per range
  constexpr int kSegs = 4 / BSC;       // scale segments (blocks) per group
  __shared__ uint4 lds_a[3 * kTermUnits];  // 48 KiB: [term][step][g][token]
  __shared__ int4 lds_e[kTok / 4];         // scale exponent e per token
  const int lane = threadIdx.x & 63;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lc = lane & 15, lg = lane >> 4;
  const int split = blockIdx.x % splits;
  const int wis = (blockIdx.x / splits) * kWaves + wave;  // wavefront index within the split
  const int k0 = split * kKR;

  // Activations: thread (t, c) loads the 32 values k0 + 32 c .. + 31 of token
  // t, first, so that waiting for them does not wait for the weight loads
  // issued after them. Tokens past M read past the end of the buffer: zeros,
  // and no memory traffic.
  const int at = tid >> 4, ac = tid & 15;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, M * K * 4, 0x00020000);
  floatx4 av[8];
  {
    const int vo = at < M ? (at * K + k0 + 32 * ac) * 4 : M * K * 4;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      av[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ra, vo + 16 * i, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);

  // Exact buffer sizes: loads at or past the end return zero without a
  // memory access. Every offset is in the per-lane voffset.
  const int b_end = N * row_bytes, s_end = N * nb * 4, z_end = N * zp_row_bytes;
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(B), 0, b_end, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(S), 0, s_end, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(HAS_ZP ? Z : B), 0, HAS_ZP ? z_end : 0, 0x00020000);
  // This lane's group (g) block within the range, and the range's first
  // 128-k group.
  const int gblk = (k0 + 128 * lg) >> log2_bs;
  const int grp0 = k0 / 128;

  // Per-lane offsets of item 0; item t is row_step rows further on (uniform
  // strides, unsigned: offsets of rows past N are never used).
  const uint32_t row_step = static_cast<uint32_t>(waves_per_split) * RB * 16;
  int row_base[RB];
  uint32_t vb0[RB], vs0[RB], vz0[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    row_base[r] = (RB * wis + r) * 16 + lc;
    vb0[r] = static_cast<uint32_t>(row_base[r]) * row_bytes + 64 * grp0 + 16 * lg;
    vs0[r] = (static_cast<uint32_t>(row_base[r]) * nb + gblk) * 4;
    vz0[r] = static_cast<uint32_t>(row_base[r]) * zp_row_bytes + (gblk >> 1);
  }
  const uint32_t db = row_step * row_bytes, ds = row_step * nb * 4, dz = row_step * zp_row_bytes;
  auto row_ok = [&](int r, int t) __attribute__((always_inline)) {
    return row_base[r] + t * static_cast<int>(row_step) < N;
  };

  // Scales and zero points of every item, right behind the activations: the
  // wait for the activations covers them, and only weights stay in flight
  // while items are multiplied (a register copy of a value still in flight
  // would wait for it). One scale load and one zero-point load per lane and
  // row block.
  constexpr int kItems = 2 * PAIRS;
  RowConsts<BSC> rc[kItems][RB];
#pragma unroll
  for (int t = 0; t < kItems; ++t)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const bool ok = row_ok(r, t);
      const int vs = ok ? static_cast<int>(vs0[r] + t * ds) : s_end;
      const int vz = ok ? static_cast<int>(vz0[r] + t * dz) : z_end;
      if constexpr (BSC == 4) {
        rc[t][r].s = __builtin_amdgcn_raw_buffer_load_b32(rsc, vs, 0, 0);
        rc[t][r].z = HAS_ZP ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz, 0, 0) : 0x88u;
      } else if constexpr (BSC == 2) {
        rc[t][r].s = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsc, vs, 0, 0));
        rc[t][r].z = HAS_ZP ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz, 0, 0) : 0x88u;
      } else {
        rc[t][r].s = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsc, vs, 0, 0));
        rc[t][r].z = HAS_ZP ? __builtin_amdgcn_raw_buffer_load_b16(rz, vz, 0, 0) : 0x8888u;
      }
    }
  __builtin_amdgcn_sched_barrier(0);

  // The wavefront's weights as a sequence of kSeq group loads (item t =
  // g / 4, group q = g % 4: one 16-byte load per lane and row block), kWin of
  // them in flight in a ring of registers: the oldest is multiplied, then
  // the one kWin further on is issued. A wavefront that finds the memory
  // queue full blocks on that issue only after it has multiplied what it has.
  constexpr int kSeq = kItems * kGroups;
  constexpr int kWin = WIN;
  u32x4 ring[kWin][RB];
  auto issue = [&](int g) __attribute__((always_inline)) {
    const int t = g / kGroups, q = g % kGroups;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      // Past the end, + 64 q keeps the offset past the end.
      const int vb = row_ok(r, t) ? static_cast<int>(vb0[r] + static_cast<uint32_t>(t) * db) : b_end;
      ring[g % kWin][r] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb + 64 * q, 0, kNonTemporal));
    }
  };
#pragma unroll
  for (int g = 0; g < kWin; ++g) issue(g);
  __builtin_amdgcn_sched_barrier(0);

  // Split the activations into LDS while the weights are in flight: the
  // token's largest magnitude over the range (the 16 lanes of one wavefront
  // that hold the token), its power-of-two scale, three fp16 terms per value.
  // MFMA j of group q reads step 4 q + j; lane group g of it holds k-unit
  // 16 q + 4 j + g when the group is transposed, else 16 q + 4 g + j.
  {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) amax = fmaxf(amax, fabsf(av[i][c]));
    amax = RowMax16(amax);
    // e puts the largest magnitude in [2^14, 2^15); applied with ldexp, which
    // is exact for every e this gives (|e| <= 163), subnormal inputs included.
    int e = 0;
    if (amax > 0.f && __builtin_isfinite(amax)) {
      int ex;
      frexpf(amax, &ex);  // amax < 2^ex
      e = 15 - ex;
    }
    if (ac == 0) reinterpret_cast<int *>(lds_e)[at] = e;
#pragma unroll
    for (int u = 0; u < 4; ++u) {  // k-unit 4 c + u of the range (8 values)
      half8 h[3];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int o = (i & 3) * 2 + (i >> 2);  // k order [0,4,1,5,2,6,3,7]
        const float x = ldexpf(av[2 * u + (i >> 2)][i & 3], e);
        const _Float16 h0 = static_cast<_Float16>(x);
        const float r1 = __builtin_isfinite(x) ? x - static_cast<float>(h0) : 0.f;
        const _Float16 h1 = static_cast<_Float16>(r1);
        h[0][o] = h0;
        h[1][o] = h1;
        h[2][o] = static_cast<_Float16>(r1 - static_cast<float>(h1));
      }
      const int ku = 4 * ac + u;
      const int st = kTr ? ku >> 2 : (ku >> 4) * 4 + (ku & 3);
      const int g = kTr ? ku & 3 : (ku >> 2) & 3;
#pragma unroll
      for (int term = 0; term < 3; ++term)
        lds_a[term * kTermUnits + st * kStepUnits + g * kTok + at] =
            __builtin_bit_cast(uint4, h[term]);
    }
  }
  __syncthreads();

  const Masks mk = MakeMasks();
  const int4 ex4 = lds_e[lg];
  const int tok_e[4] = {ex4.x, ex4.y, ex4.z, ex4.w};
  // Outputs through a buffer as well: stores for tokens past M or rows past N
  // go past its end and are dropped, with no branch in the loop.
  const int y_end = M * N * 4;
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
      split == 0 ? Y : partials + static_cast<size_t>(split - 1) * M * N, 0, y_end, 0x00020000);

  // Multiply group q of item t into acc; at the item's last group store its
  // outputs: value v of this lane is token 4 g + v of weight row 16 (block)
  // + c; ldexp by -e undoes the token's scaling (exact unless the output is
  // an fp32 subnormal).
  floatx4 acc[RB];
  auto step = [&](int g) __attribute__((always_inline)) {
    const int t = g / kGroups, q = g % kGroups;
    u32x4 (&w)[RB] = ring[g % kWin];
    // Pins the group's decode here: left free, the compiler hoists the
    // arithmetic on later groups' weights into this one and then waits for
    // their loads.
#pragma unroll
    for (int r = 0; r < RB; ++r) __asm__ volatile("" : "+v"(w[r]));
    if (q == 0) {
#pragma unroll
      for (int r = 0; r < RB; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const int src = (lc + 16 * q) * 4;  // the lane of this row that loaded group q's constants
    float s[RB][kSegs];
    uint32_t zq[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if constexpr (BSC == 4) {
        s[r][0] = __builtin_bit_cast(float, FromLane(src, rc[t][r].s));
        // Nibble of this group's block in the byte its lane loaded.
        const int zsh = (((k0 + 128 * q) >> log2_bs) & 1) * 4;
        zq[r] = (FromLane(src, rc[t][r].z) >> zsh) & 0xFu;
      } else {
#pragma unroll
        for (int sg = 0; sg < kSegs; ++sg)
          s[r][sg] = __builtin_bit_cast(float, FromLane(src, rc[t][r].s[sg]));
        zq[r] = FromLane(src, rc[t][r].z);  // kSegs nibbles, low first
      }
      if constexpr (kTr) Transpose4(w[r]);
    }
#pragma unroll
    for (int sg = 0; sg < kSegs; ++sg) {
      uint32_t neg_lo[RB], neg_hi[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const uint32_t zp = HAS_ZP ? (BSC == 4 ? zq[r] : (zq[r] >> (4 * sg)) & 0xFu) : 8u;
        // fp16 -(1024 + zp) = 0xE400 | zp and -(64 + zp) = 0xD400 | zp << 4.
        const uint32_t zz = zp * 0x10001u;
        neg_lo[r] = zz | 0xE400E400u;
        neg_hi[r] = (zz << 4) | 0xD400D400u;
      }
      floatx4 tmp[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) tmp[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < BSC; ++jj) {
        const int j = sg * BSC + jj;
        half8 bq[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) bq[r] = DecodeQ(w[r][j], neg_lo[r], neg_hi[r], mk);
#pragma unroll
        for (int term = 0; term < 3; ++term) {
          const half8 af = __builtin_bit_cast(
              half8, lds_a[term * kTermUnits + (4 * q + j) * kStepUnits + lane]);
#pragma unroll
          for (int r = 0; r < RB; ++r)
            tmp[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bq[r], tmp[r], 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[r][v] = fmaf(s[r][sg], tmp[r][v], acc[r][v]);
    }
    if (q == kGroups - 1) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int n = row_base[r] + t * static_cast<int>(row_step);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int tok = 4 * lg + v;
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ldexpf(acc[r][v], -tok_e[v])),
                                                ry, tok < M && n < N ? (tok * N + n) * 4 : y_end,
                                                0, 0);
        }
      }
    }
  };

  // Straight-line code (no loop, no branch around a load or store) keeps the
  // compiler's waits exact; the output stores count in the same counter as
  // the loads. The scheduling barriers keep each load where it is issued.
#pragma unroll
  for (int g = 0; g < kSeq; ++g) {
    step(g);
    __builtin_amdgcn_sched_barrier(0);
    if (g + kWin < kSeq) issue(g + kWin);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Y += P[0] + P[1] + ... + P[parts - 1], added in that order. VEC: four
// consecutive outputs per thread (Y, P 16-byte aligned, M N % 4 == 0); the
// parts' loads are issued sixteen at a time.
template <bool VEC>
__global__ __launch_bounds__(256) void SumPartialsKernel(float *__restrict__ Y,
                                                         const float *__restrict__ P, int64_t mn,
                                                         int parts, float *__restrict__ H,
                                                         const float *__restrict__ bias,
                                                         int64_t N) {
  constexpr int kBatch = 16;
  if constexpr (VEC) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    // the bias is loaded with the sums (added after them: a separate bias
    // pass; N % 4 == 0 here)
    floatx4 b = floatx4{0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr) {
      const int64_t n = i % N;
      b = floatx4{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]};
    }
    floatx4 y = *reinterpret_cast<const floatx4 *>(Y + i);
    for (int p = 0; p < parts; p += kBatch) {
      floatx4 v[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        if (p + q < parts)
          v[q] = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(P + (p + q) * mn + i));
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        if (p + q < parts) y += v[q];
    }
    if (bias != nullptr) y += b;
    if (H != nullptr) {
      // gate/up pairs (N even, so a pair never straddles rows)
      *reinterpret_cast<float2 *>(H + i / 2) = make_float2(SiluMul(y[0], y[1]), SiluMul(y[2], y[3]));
    } else {
      *reinterpret_cast<floatx4 *>(Y + i) = y;
    }
  } else {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= mn) return;
    const float b = bias != nullptr ? bias[i % N] : 0.f;
    float y = Y[i];
    for (int p = 0; p < parts; p += kBatch) {
      float v[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        if (p + q < parts) v[q] = __builtin_nontemporal_load(P + (p + q) * mn + i);
#pragma unroll
      for (int q = 0; q < kBatch; ++q)
        if (p + q < parts) y += v[q];
    }
    if (bias != nullptr) y += b;
    if (H != nullptr) {
      // mn is even: lanes i and i ^ 1 are both in range, in the same wavefront
      const float other = PairSwap(y);
      if ((i & 1) == 0) H[i / 2] = SiluMul(y, other);
    } else {
      Y[i] = y;
    }
  }
}

struct Shape {
  int bsc, rb, splits, wgs_per_split, waves_per_split, pairs;
};

// Row blocks of 16 per item (RB) and the grid: a target number of
// workgroups per CU (a whole number of them per split), each wavefront with
// one or two pairs of items (more workgroups when the rows need it).
// Defaults from a sweep of RB in {1, 2} against 1..4 workgroups per CU on
// MI355X (c2, c3, c5 shapes, M = 8 and 16): one row block for long rows
// (K >= 8192: c3 and c5 down 13% faster than two), two for short ones; one
// workgroup per CU (c5 qkv 20%, c2 3-5% faster than two) except for weights
// at least six times wider than deep (c5 gate+up: two).
inline Shape PickShape(const WeightView &w, int rb, int wgs_per_cu) {
  Shape sh;
  sh.bsc = std::min(4, w.block_size / 32);
  sh.splits = static_cast<int>(w.K / kKR);
  sh.rb = rb > 0 ? rb : (w.K >= 8192 ? 1 : 2);
  const int64_t items = (w.N + 16 * sh.rb - 1) / (16 * sh.rb);  // per split
  const int wpc = wgs_per_cu > 0 ? wgs_per_cu : (w.N >= 6 * w.K ? 2 : 1);
  const int64_t target = static_cast<int64_t>(w.num_cus) * wpc;
  int64_t wps = std::max<int64_t>(1, (target + sh.splits - 1) / sh.splits);
  wps = std::min(wps, (items + kWaves - 1) / kWaves);       // no workgroup without an item
  wps = std::max(wps, (items + 4 * kWaves - 1) / (4 * kWaves));  // at most two pairs
  sh.wgs_per_split = static_cast<int>(wps);
  sh.waves_per_split = sh.wgs_per_split * kWaves;
  sh.pairs = static_cast<int>((items + 2 * sh.waves_per_split - 1) / (2 * sh.waves_per_split));
  return sh;
}

// Group loads in flight per wavefront: 8 KiB of weights with two row blocks.
constexpr int kWinFor(int rb) { return rb == 1 ? 8 : 4; }

template <int BSC, int RB, int PAIRS>
hipError_t LaunchMain(const WeightView &w, int64_t M, const float *A, float *Y, float *P,
                      const Shape &sh, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(sh.splits * sh.wgs_per_split)), block(64 * kWaves);
  if (w.zp != nullptr)
    hipLaunchKernelGGL((GemvMfmaKernel<BSC, RB, PAIRS, kWinFor(RB), true>), grid, block, 0, s, A, w.B,
                       w.scales, w.zp, Y, P, static_cast<int>(M), static_cast<int>(w.K),
                       static_cast<int>(w.N), static_cast<int>(w.nb), w.log2_bs,
                       static_cast<int>(w.row_bytes), static_cast<int>(w.zp_row_bytes),
                       sh.splits, sh.waves_per_split);
  else
    hipLaunchKernelGGL((GemvMfmaKernel<BSC, RB, PAIRS, kWinFor(RB), false>), grid, block, 0, s, A, w.B,
                       w.scales, w.zp, Y, P, static_cast<int>(M), static_cast<int>(w.K),
                       static_cast<int>(w.N), static_cast<int>(w.nb), w.log2_bs,
                       static_cast<int>(w.row_bytes), static_cast<int>(w.zp_row_bytes),
                       sh.splits, sh.waves_per_split);
  return hipGetLastError();
}

template <int BSC>
hipError_t LaunchBsc(const WeightView &w, int64_t M, const float *A, float *Y, float *P,
                     const Shape &sh, hipStream_t s) {
  if (sh.rb == 1)
    return sh.pairs == 1 ? LaunchMain<BSC, 1, 1>(w, M, A, Y, P, sh, s)
                         : LaunchMain<BSC, 1, 2>(w, M, A, Y, P, sh, s);
  return sh.pairs == 1 ? LaunchMain<BSC, 2, 1>(w, M, A, Y, P, sh, s)
                       : LaunchMain<BSC, 2, 2>(w, M, A, Y, P, sh, s);
}

} // namespace mf

bool GemvMfmaSupports(const WeightView &w, int64_t M) {
  // K in whole 512-k ranges (at most 64); power-of-two blocks of 32 or more;
  // every buffer offset (including one past the end) below 2^31.
  return w.B != nullptr && M >= 2 && M <= 16 && (w.K % mf::kKR) == 0 &&
         w.K / mf::kKR <= mf::kMaxSplits &&
         w.block_size >= 32 && (w.block_size & (w.block_size - 1)) == 0 &&
         w.row_bytes * w.N + w.K < (int64_t{1} << 31) && w.nb * 4 * w.N < (int64_t{1} << 31) &&
         M * w.K * 4 + 512 < (int64_t{1} << 31) && M * w.N * 4 < (int64_t{1} << 31);
}

size_t GemvMfmaWorkspaceBytes(const WeightView &w, int64_t M) {
  return static_cast<size_t>(w.K / mf::kKR - 1) * M * w.N * 4;
}

hipError_t LaunchGemvMfmaShape(const WeightView &w, int64_t M, const float *A, float *Y,
                               void *work, hipStream_t s, int rows_per_wave, int wgs_per_cu,
                               float *H) {
  const mf::Shape sh = mf::PickShape(w, rows_per_wave, wgs_per_cu);
  if (!(sh.rb == 1 || sh.rb == 2) || sh.pairs < 1 || sh.pairs > 2) return hipErrorInvalidValue;
  float *P = static_cast<float *>(work);
  hipError_t e;
  switch (sh.bsc) {
  case 1: e = mf::LaunchBsc<1>(w, M, A, Y, P, sh, s); break;
  case 2: e = mf::LaunchBsc<2>(w, M, A, Y, P, sh, s); break;
  default: e = mf::LaunchBsc<4>(w, M, A, Y, P, sh, s); break;
  }
  if (e != hipSuccess) return e;
  // One 512-k range: Y is complete, only the gate/up activation is left.
  if (sh.splits == 1) return H != nullptr ? LaunchSiluMul(Y, H, M, w.N, s) : hipSuccess;
  return LaunchSumPartials(Y, P, M * w.N, sh.splits - 1, H, s);
}

hipError_t LaunchSumPartials(float *Y, const float *P, int64_t mn, int parts, float *H,
                             hipStream_t s, const float *bias, int64_t N) {
  const bool vec = (mn % 4) == 0 && (reinterpret_cast<uintptr_t>(Y) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(P) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(H) % 8) == 0 && (bias == nullptr || N % 4 == 0);
  if (vec)
    hipLaunchKernelGGL(mf::SumPartialsKernel<true>,
                       dim3(static_cast<unsigned>((mn / 4 + 255) / 256)), dim3(256), 0, s, Y, P,
                       mn, parts, H, bias, N);
  else
    hipLaunchKernelGGL(mf::SumPartialsKernel<false>, dim3(static_cast<unsigned>((mn + 255) / 256)),
                       dim3(256), 0, s, Y, P, mn, parts, H, bias, N);
  return hipGetLastError();
}

hipError_t LaunchGemvMfma(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                          hipStream_t s, float *H) {
  return LaunchGemvMfmaShape(w, M, A, Y, work, s, 0, 0, H);
}

} // namespace mnb
