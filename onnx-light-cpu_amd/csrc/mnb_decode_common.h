// Device helpers shared by the decode GEMV kernels (M = 1 and small M).
#pragma once

#include "mnb_kernels.h"

namespace mnb {
namespace dec {

constexpr uint32_t kNonTemporal = 2;  // buffer-load cache policy: NT

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
// a * f16(lo half of h), a fresh accumulator
__device__ __forceinline__ float MixLo0(float a, uint32_t h) {
  float r;
  __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(h));
  return r;
}
// a * f16(hi half of h), a fresh accumulator
__device__ __forceinline__ float MixHi0(float a, uint32_t h) {
  float r;
  __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(h));
  return r;
}

// The reference engine's fp32 product of one activation row with one weight
// row: each weight dequantized on its own, w = float(q - zp) * scale, and
// acc = acc + a * w with the product rounded, k ascending (MatMulPlan<float>
// over the dequantized weights, onnx_light_cpu/impl/math/gemm_kernel.cc:
// 1208-1258). The fast decode kernels apply the zero point through each
// block's activation sum (y += scale (sum a q - zp sum a)), so an infinite
// activation meets inf - inf there and gives NaN where the reference gives
// +-inf (NaN only where q == zp or the signs differ). Each kernel therefore
// recomputes an output whose fast result is not finite with this function;
// finite activations never take it unless the fast sum overflows, and then
// the reference's own overflow is the answer. One thread reads the whole
// row: slow, and only on non-finite outputs.
//   nib(k8)  -> the packed word of nibbles k = 8 k8 .. 8 k8 + 7 (low first)
//   blk(b)   -> float2(scale, zero point) of block b
template <class Nibbles, class Block>
__device__ __forceinline__ float ReferenceRowDot(const float *__restrict__ a, int K, int log2_bs,
                                                 Nibbles nib, Block blk) {
#pragma clang fp contract(off)
  float acc = 0.0f;
  for (int k8 = 0; k8 < (K >> 3); ++k8) {
    const uint32_t word = nib(k8);
    const float2 sz = blk((k8 << 3) >> log2_bs);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float w = static_cast<float>(static_cast<int>((word >> (4 * i)) & 0xFu) -
                                         static_cast<int>(sz.y)) *
                      sz.x;
      const float p = a[8 * k8 + i] * w;
      acc = acc + p;
    }
  }
  return acc;
}

// ReferenceRowDot over one weight row in the MatMulNBits layout: its packed
// nibbles brow (4-byte aligned), block scales srow and packed zero points
// zrow (nullptr: 8).
__device__ __forceinline__ float ReferenceRowDotPlain(const float *__restrict__ a, int K,
                                                      int log2_bs, const uint8_t *brow,
                                                      const float *srow, const uint8_t *zrow) {
  return ReferenceRowDot(
      a, K, log2_bs, [&](int k8) { return *reinterpret_cast<const uint32_t *>(brow + 4 * k8); },
      [&](int b) {
        const float zp =
            zrow != nullptr ? static_cast<float>((zrow[b >> 1] >> (4 * (b & 1))) & 0xFu) : 8.0f;
        return make_float2(srow[b], zp);
      });
}

template <int CTRL>
__device__ __forceinline__ float DppAdd(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false);
  return v + __int_as_float(moved);
}

template <int CTRL>
__device__ __forceinline__ float DppMax(float v) {
  const int moved = __builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true);
  return fmaxf(v, __int_as_float(moved));
}

// Largest value over each aligned 16-lane row, every lane of the row holding
// it (the xor butterfly over 1, 2, 4 and 8 lanes with DPP moves).
__device__ __forceinline__ float RowMax16(float v) {
  v = DppMax<0xB1>(v);   // quad_perm [1,0,3,2]
  v = DppMax<0x4E>(v);   // quad_perm [2,3,0,1]
  v = DppMax<0x141>(v);  // row_half_mirror
  return DppMax<0x140>(v);  // row_mirror
}

// Largest value over each 32-lane half of the wavefront, every lane of the
// half holding it: the xor butterfly over 1, 2, 4, 8 and 16 lanes with DPP
// moves (row_half_mirror and row_mirror pair the same lanes' values as xor 4
// and xor 8 once the smaller groups agree) instead of LDS permutes.
__device__ __forceinline__ float HalfMax(float v) {
  v = RowMax16(v);
  return fmaxf(v, Xor16(v));
}

// Sum over aligned groups of LANES (4, 8, 16 or 32) lanes, every lane of a
// group holding it: the same additions, in the same order, as the xor
// butterfly over 1, 2, ... LANES / 2 (so bit-identical to it).
template <int LANES>
__device__ __forceinline__ float GroupSum(float v) {
  static_assert(LANES == 4 || LANES == 8 || LANES == 16 || LANES == 32, "group size");
  v = DppAdd<0xB1>(v);
  v = DppAdd<0x4E>(v);
  if constexpr (LANES >= 8) v = DppAdd<0x141>(v);
  if constexpr (LANES >= 16) v = DppAdd<0x140>(v);
  if constexpr (LANES >= 32) v += Xor16(v);
  return v;
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

// q = j / nb and r = j % nb for 0 <= j < 2^16 through the fp32 reciprocal
// (error below one, corrected once).
__device__ __forceinline__ int DivNb(int j, int nb, float rnb, int &r) {
  int q = static_cast<int>(static_cast<float>(j) * rnb);
  r = j - q * nb;
  if (r >= nb) { ++q; r -= nb; }
  if (r < 0) { --q; r += nb; }
  return q;
}

// One work item of a wavefront's (scale, zp) staging: PW consecutive pairs of
// one of its rows (PW = 4 needs nb % 4 == 0: one 16-byte scale load, one
// 2-byte zero-point load). Pair j = PW * item of the wavefront, row-major
// [wave row][block]; rows past the band re-read the band's last row.
template <int PW, bool HAS_ZP>
struct PairItem {
  float s[PW];
  uint32_t z;
  int j, shift;

  // Loads are unconditional (item clamped to the last one) so that no branch
  // forces the compiler to wait for them early; Store skips clamped items.
  __device__ __forceinline__ void Load(int item, int nitems, int nb, float rnb, int wrow0,
                                       int last_row, int zp_row_bytes,
                                       __amdgpu_buffer_rsrc_t rsc, __amdgpu_buffer_rsrc_t rz) {
    j = item < nitems ? item * PW : -1;
    const int jl = min(item, nitems - 1) * PW;
    int blk;
    const int row = min(wrow0 + DivNb(jl, nb, rnb, blk), last_row);
    if (PW == 4) {
      const float4 v = __builtin_bit_cast(
          float4, __builtin_amdgcn_raw_buffer_load_b128(rsc, (row * nb + blk) * 4, 0, 0));
      s[0] = v.x;
      s[1 % PW] = v.y;
      s[2 % PW] = v.z;
      s[3 % PW] = v.w;
    } else {
      s[0] = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(rsc, (row * nb + blk) * 4, 0, 0));
    }
    z = 0x8888u;
    shift = 0;
    if (HAS_ZP) {
      const int off = row * zp_row_bytes + (blk >> 1);
      if (PW == 4) {
        z = __builtin_amdgcn_raw_buffer_load_b16(rz, off, 0, 0);
      } else {
        z = __builtin_amdgcn_raw_buffer_load_b8(rz, off, 0, 0);
        shift = (blk & 1) * 4;
      }
    }
  }

  // spare: index of the 4 spare pairs
  __device__ __forceinline__ void Store(float2 *pairs, int spare) const {
    const int base = j >= 0 ? j : spare;
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const uint32_t zp = (z >> (shift + 4 * u)) & 0xFu;
      pairs[base + u] = make_float2(s[u] * 16777216.f, static_cast<float>(zp) * 5.9604644775390625e-8f);
    }
  }
};

} // namespace dec
} // namespace mnb
