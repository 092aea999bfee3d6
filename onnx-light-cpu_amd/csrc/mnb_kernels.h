// Internal launch interface shared by the C ABI (mnb_capi.hip) and the kernel
// translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mnb {

// Global -> LDS copy of 16 bytes per lane: lane L's 16 bytes at gsrc land at
// LDS byte lds_base + 16 L (global_load_lds_dwordx4). Issued through inline
// asm on purpose: the compiler cannot tell which LDS bytes such a copy writes,
// so for the builtin it orders every later LDS access behind all outstanding
// vector-memory loads (an s_waitcnt vmcnt(0) before each LDS read or write),
// which serialises the prefetch pipeline. Hidden from it, the copy still
// counts in the hardware vmcnt, so the compiler's own waits for register
// loads stay correct (loads complete in issue order; at worst they also wait
// for an older copy); callers wait for the copy themselves (s_waitcnt vmcnt
// counting the loads issued after it, then a barrier) before reading its
// destination. One wait state separates the M0 write from the copy. M0 is
// listed as clobbered for the reader; clang warns that it does not track M0
// across inline asm, and nothing else in the kernels that use this helper
// reads M0 (checked in their gfx950 assembly).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void CopyToLds16(const void *gsrc, uint32_t lds_base) {
  __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                   :
                   : "s"(lds_base), "v"(gsrc)
                   : "memory", "m0");
}
// The same copy from sbase + voff: a wave-uniform 64-bit base in SGPRs and a
// per-lane 32-bit byte offset, so the address costs no 64-bit VGPR pair and
// no vector arithmetic per copy.
__device__ __forceinline__ void CopyToLds16S(const void *sbase, uint32_t voff, uint32_t lds_base) {
  __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :
                   : "s"(lds_base), "v"(voff), "s"(sbase)
                   : "memory", "m0");
}
#pragma clang diagnostic pop

// Gated-MLP activation of one gate/up pair, in the order of the ONNX subgraph
// it replaces: s = Sigmoid(g) = 1 / (1 + exp(-g)), then Mul(g, s), then
// Mul(., u), each rounded to fp32. exp is the device library's expf (at most
// 1 ulp, arguments reduced in extended precision, so its error does not grow
// with |g|) and the reciprocal v_rcp_f32 (1 ulp). Error contract, against the
// exact g * sigmoid(g) * u of the fp32 g and u: at most 2^-20 relative, plus
// 2^-126 * |g * u| absolute where sigmoid(g) falls below fp32's normal range
// (g < -87). Special values follow the subgraph: g = +inf gives +-inf * u,
// g = -inf gives NaN (-inf * 0), NaN propagates. Every kernel that applies
// the activation (fused epilogues and the separate SiluMulKernel) uses this
// one expression, so a fused result equals the unfused one bit for bit.
__device__ __forceinline__ float SiluMul(float g, float u) {
  const float s = __builtin_amdgcn_rcpf(1.0f + expf(-g));
  return (g * s) * u;
}

// The value of lane ^ 1 (DPP quad_perm [1,0,3,2]: one VALU move, no LDS
// round trip). Both lanes of each pair must be active.
__device__ __forceinline__ float PairSwap(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}

// The value of lane ^ 16 (ds_swizzle, bit mode: and 0x1F, or 0, xor 0x10;
// no memory access, a shorter path than an LDS permute).
__device__ __forceinline__ float Xor16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}

// Power-of-two exponent f that brings a largest magnitude amax into
// [2^target, 2^(target+1)), so that values up to amax times 2^f stay in fp16's
// range; the scaling itself is exact in fp32. 0 for a zero, infinite or NaN
// maximum (those then propagate as they would in fp32).
__device__ __forceinline__ int RangeExponent(float amax, int target) {
  if (!(amax > 0.0f) || !(amax <= 3.402823466e38f)) return 0;
  int e;
  (void)frexpf(amax, &e);  // amax = m * 2^e, m in [0.5, 1): floor(log2 amax) = e - 1
  return target - (e - 1);
}

// Exponent target of the plan's per-weight-row scale exponents: the largest
// block scale of row n times 2^col_exp[n] lies in [2^11, 2^12), so every
// block scale down to 2^-25 of it is a normal fp16 number and
// (q - zp) * scale, |q - zp| <= 15, stays below 65504.
constexpr int kScaleExpTarget = 11;
// Exponent target of the prefill path's per-row activation exponents: the
// row's largest magnitude times 2^f lies in [2^14, 2^15).
constexpr int kRowExpTarget = 14;

// Everything a kernel needs to address one plan's constants.
// B, scales and zp are null on a compact plan, which keeps only the re-laid
// copies (see the plan's description in mnb_capi.hip); kernels on the
// original layout then report themselves unsupported.
struct WeightView {
  const uint8_t *B;       // [N, nb, bs/2] packed nibbles, low nibble first, or nullptr
  const float *scales;    // [N, nb], or nullptr
  const uint8_t *zp;      // [N, zp_row_bytes] packed nibbles, or nullptr (zp = 8 or compact)
  const int32_t *col_exp; // [N] RangeExponent(max_b |scales[n][b]|, kScaleExpTarget)
  const uint8_t *Bp;      // the prefill kernel's fragment-ordered weights, or nullptr
  const uint8_t *Sp;      // its per-block scale / zero-point words, or nullptr
  const float *Sd;        // DecodeFragKernel's block scales per 64-row group, or nullptr
  const uint32_t *Zd;     // its zero points per 64-row group, or nullptr
  int64_t K;
  int64_t N;
  int64_t nb;             // ceil(K / bs)
  int64_t row_bytes;      // nb * bs / 2
  int64_t zp_row_bytes;   // ceil(nb / 2)
  int32_t block_size;
  int32_t log2_bs;
  int32_t num_cus;        // compute units of the plan's device
  int32_t has_zp;         // MatMulNBits input 3 present (Zd holds it on a compact plan)
};

// Decode GEMV, M in [1, 16], K % 32 == 0, block_size >= 32.
hipError_t LaunchGemv(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s);
bool GemvSupports(const WeightView &w, int64_t M);

// Decode GEMV for 2 <= M <= 16 (fp32 FMA on fp16-subnormal decoded nibbles),
// in groups of at most 4 tokens, one launch per group.
hipError_t LaunchGemvSmallM(const WeightView &w, int64_t M, const float *A, float *Y,
                            hipStream_t s);
bool GemvSmallMSupports(const WeightView &w, int64_t M);
// Same with an explicit shape (tuning): tokens per group (<= 8), wavefronts
// per workgroup (4 or 8), rows per wavefront (1, 2 or 4); 0 = default.
hipError_t LaunchGemvSmallMShape(const WeightView &w, int64_t M, const float *A, float *Y,
                                 hipStream_t s, int max_tokens, int waves, int rows_per_wave);

// Decode GEMV for 1 <= M <= 4 on fp16 MFMA (activations split into three fp16
// terms in LDS, nibbles masked into fp16 subnormals, fp32 sums within about
// 2^-22 of sum |a w| per output),
// streaming the plan's fragment-ordered weights: one workgroup per 64-row
// group, `steps_per_wave` (8, 16 or 32; 8 or 16 when M > 1) 32-k steps per
// wavefront with `window` (4 or 8; 8 when M > 1) weight records in flight; 0
// picks either. Needs Bp / Sd (/ Zd) and 32 <= block_size <= 256. H, bias and
// the RMSNorm input (gamma, window 8) as below.
bool GemvFragSupports(const WeightView &w, int64_t M);
bool GemvFragShapeOk(const WeightView &w, int64_t M, int steps_per_wave, int window);
// Whether the auto path takes it: its groups cover most CUs (with `rms`, for
// a fused RMSNorm input).
bool GemvFragPreferred(const WeightView &w, int64_t M, bool rms = false);
// Whether the 64-row groups cover 85% of the CUs (one workgroup per group).
bool GemvFragWide(const WeightView &w);
hipError_t LaunchGemvFrag(const WeightView &w, int64_t M, const float *A, float *Y, hipStream_t s,
                          int steps_per_wave, int window, float *H, const float *bias,
                          const float *gamma = nullptr, float eps = 0.0f);
// The same GEMV for 1 or 2 rows too long for one workgroup per group (K >
// 16384 at M = 1, K > 8192 at M = 2): K split into segments of whole 256-k
// units, one workgroup per (group, segment), the segments' partial sums in
// `work` (GemvFragSegWorkspaceBytes) added in order by SumPartialsKernel with
// the bias. No gate/up epilogue and no RMSNorm input.
bool GemvFragSegSupports(const WeightView &w, int64_t M);
size_t GemvFragSegWorkspaceBytes(const WeightView &w, int64_t M);
hipError_t LaunchGemvFragSeg(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                             hipStream_t s, const float *bias);

// Decode GEMV for M == 1 (fp16-subnormal mixed FMA): one workgroup per band
// of `band_rows` weight rows, `rows_per_wave` (1, 2, 4 or 8) rows per
// wavefront; 0 picks both from the shape and the device's CU count.
//
// Gate/up epilogue (this and the MFMA decode and GEMM launches below): when
// H is not null, the plan's rows are gate/up pairs (row 2n the gate of output
// n, row 2n + 1 its up) and the launch writes H[m][n] = SiluMul(y[m][2n],
// y[m][2n + 1]) instead of the product y; Y is then scratch (M x N floats)
// for the launches that need an intermediate sum, unused by the others.
//
// RMSNorm input (M = 1 GEMV, the M <= 4 fragment GEMV, the small-M MFMA
// decode on the fragment-ordered copy, GEMM): with gamma (K floats, 16-byte aligned)
// the launch multiplies RMSNorm(A) = A / sqrt(mean_k(A^2) + eps) * gamma
// instead of A; both compute the rows' mean squares themselves.
// bias (N floats, MatMulNBits input 5, not with H) is added to each row's sum
// before its store.
hipError_t LaunchGemvM1(const WeightView &w, const float *A, float *Y, hipStream_t s,
                        int band_rows, int rows_per_wave, float *H = nullptr,
                        const float *gamma = nullptr, float eps = 0.0f,
                        const float *bias = nullptr);
bool GemvM1Supports(const WeightView &w);

// Decode GEMV for 2 <= M <= 16 on fp16 MFMA with exact products (each
// activation split into three fp16 terms after a power-of-two scaling); K a
// multiple of 512 (at most 32768), power-of-two block_size >= 32. `work`
// holds GemvMfmaWorkspaceBytes(w, M) bytes: the partial sums of K ranges 1..
hipError_t LaunchGemvMfma(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                          hipStream_t s, float *H = nullptr);
bool GemvMfmaSupports(const WeightView &w, int64_t M);
size_t GemvMfmaWorkspaceBytes(const WeightView &w, int64_t M);
// Same with an explicit shape (tuning): 16-row blocks per item (1 or 2) and
// workgroups per CU; 0 picks.
hipError_t LaunchGemvMfmaShape(const WeightView &w, int64_t M, const float *A, float *Y,
                               void *work, hipStream_t s, int rows_per_wave, int wgs_per_cu,
                               float *H = nullptr);

// Decode GEMV for 2 <= M <= 16 on fp16 MFMA with exact products over the
// plan's fragment-ordered weights (Bp) and re-laid block scales / zero points
// (Sd, Zd); K % 256 == 0, power-of-two block_size >= 32. `work` holds
// DecodeFragWorkspaceBytes(w, M, 0, 0) bytes: the split activation image, the
// per-unit exponents, the per-unit sums of squares of an RMSNorm input and
// the partial sums of runs 1.. (one pre-pass kernel, the main kernel, and the
// ordered partial-sum pass when K is split over several workgroups). wpg
// (wavefronts per workgroup, 1 to 8) and units_per_wave (1 or 2; a unit is
// 256 k): 0 picks. bias (N floats, not with H) is added by the main kernel's
// stores or the partial-sum pass. gamma: the RMSNorm input as above (the
// pre-pass multiplies by gamma and sums A^2 per unit; each run scales its
// sums by 1 / rms).
bool DecodeFragLayoutWanted(const WeightView &w);
size_t DecodeFragScaleBytes(const WeightView &w, size_t *zd_bytes);
hipError_t LaunchDecodeFragRelayout(const WeightView &w, float *Sd, uint32_t *Zd, hipStream_t s);
bool DecodeFragSupports(const WeightView &w, int64_t M);
// Whether the launch takes an RMSNorm input (gamma): K <= 16384.
bool DecodeFragTakesRms(const WeightView &w);
size_t DecodeFragWorkspaceBytes(const WeightView &w, int64_t M, int wpg = 0,
                                int units_per_wave = 0);
hipError_t LaunchDecodeFrag(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                            hipStream_t s, float *H = nullptr, int wpg = 0,
                            int units_per_wave = 0, const float *bias = nullptr,
                            const float *gamma = nullptr, float eps = 0.0f);
// Y += P[0] + ... + P[parts - 1] over mn elements, in that order (then the
// gate/up activation into H when H is not null).
hipError_t LaunchSumPartials(float *Y, const float *P, int64_t mn, int parts, float *H,
                             hipStream_t s, const float *bias = nullptr, int64_t N = 1);

// Prefill GEMM on fp16 MFMA, any M, K % 64 == 0, block_size >= 32. `work`
// holds GemmWorkspaceBytes(w, M) bytes of device memory: A scaled per row by
// a power of two and rounded to fp16, the rows' exponents, then the partial
// sums of a split-K launch.
// On a plan holding the re-laid weights, StreamKernel serves 17 <= M <= 64
// and the prefill kernel (128 x 256 tiles) M >= 65 where its tiles fill the
// CUs; both add `bias` (N floats) themselves and then set *bias_done.
// Otherwise GemmKernel (BM x 128 tiles over the original layout) serves.
hipError_t LaunchGemm(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                      hipStream_t s, float *H = nullptr, const float *gamma = nullptr,
                      float eps = 0.0f, const float *bias = nullptr, bool *bias_done = nullptr);
bool GemmUsesPrefill(const WeightView &w, int64_t M);
bool GemmUsesStream(const WeightView &w, int64_t M);
// The prefill kernel forced (any M >= 1 on a plan holding the re-laid
// weights; split-K when its tiles alone do not fill the CUs); adds `bias`
// in its epilogue and sets *bias_done.
hipError_t LaunchPrefill(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                         hipStream_t s, float *H = nullptr, const float *gamma = nullptr,
                         float eps = 0.0f, const float *bias = nullptr, bool *bias_done = nullptr);
bool PrefillSupports(const WeightView &w, int64_t M);
// Small-M prefill (17 <= M <= 64) streaming the prefill kernel's re-laid
// weights once: ConvertA, StreamKernel over (64-row group, K segment)
// workgroups, and the ordered reduction of the segments when K is split.
// segs / spw (K segments, 32-k steps per wavefront) pick the shape, 0 for
// the default; `work` holds StreamWorkspaceBytes(w, M, segs, spw) bytes.
// Adds `bias` itself.
bool StreamSupports(const WeightView &w, int64_t M);
size_t StreamWorkspaceBytes(const WeightView &w, int64_t M, int segs, int spw);
// Whether (segs, spw) gives a launch the kernel serves (4 to 8 wavefronts per
// workgroup, whole steps per wavefront).
bool StreamShapeOk(const WeightView &w, int64_t M, int segs, int spw);
hipError_t LaunchStream(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                        hipStream_t s, float *H, const float *gamma, float eps, const float *bias,
                        int segs, int spw);
// The prefill kernel's weight layout: whether the plan's shape can use it,
// its byte sizes (Bp returned, Sp through sp_bytes), and the plan-time
// re-layout from B, scales, zero points and col_exp.
bool PrefillLayoutWanted(const WeightView &w);
size_t PrefillLayoutBytes(const WeightView &w, size_t *sp_bytes);
hipError_t LaunchPrefillRelayout(const WeightView &w, uint8_t *Bp, uint8_t *Sp, hipStream_t s);
// The GEMM path (path 2): GemmKernel on the original layout, or the prefill
// / streaming kernels on the re-laid copy.
bool GemmSupports(const WeightView &w, int64_t M);
// GemmKernel itself (the original layout).
bool GemmKernelSupports(const WeightView &w, int64_t M);
size_t GemmWorkspaceBytes(const WeightView &w, int64_t M);
// Same with an explicit tile height (32, 64 or 128; 0 picks both;
// kPrefillTileCode = the prefill kernel) and split count (1..16), for
// tuning; `work` then holds GemmShapeWorkspaceBytes(w, M, splits) bytes.
constexpr int kPrefillTileCode = 256;
hipError_t LaunchGemmShape(const WeightView &w, int64_t M, const float *A, float *Y, void *work,
                           hipStream_t s, int bm, int splits, float *H = nullptr,
                           const float *gamma = nullptr, float eps = 0.0f);
size_t GemmShapeWorkspaceBytes(const WeightView &w, int64_t M, int splits);

// H[m][n] = SiluMul(Y[m][2n], Y[m][2n + 1]) for an M x N (N even) Y: the
// gate/up activation after a kernel without the fused epilogue.
hipError_t LaunchSiluMul(const float *Y, float *H, int64_t M, int64_t N, hipStream_t s);

// RMSNorm over the rows of X [M, K] (K % 4 == 0, X 16-byte aligned):
// Xn[m][k] = X[m][k] * inv_rms[m] * gamma[k], inv_rms[m] =
// 1 / sqrt(mean_k(X[m]^2) + eps).
hipError_t LaunchRmsNorm(const float *X, const float *gamma, float *Xn, int64_t M, int64_t K,
                         float eps, hipStream_t s);

// col_exp[n] = RangeExponent(max_b |scales[n][b]|, kScaleExpTarget) for the
// plan's N weight rows (run once, at plan creation).
hipError_t LaunchColExp(const float *scales, int32_t *col_exp, int64_t N, int64_t nb,
                        hipStream_t s);

// Generic fallback: any K, any block_size, any M. Slow; for odd shapes and
// cross-checks.
hipError_t LaunchGeneric(const WeightView &w, int64_t M, const float *A, float *Y,
                         hipStream_t s);

} // namespace mnb
