// QDQ front-end of the C ABI: a constant weight-only DequantizeLinear feeding
// MatMul, repacked on the host into MatMulNBits inputs (mnb_qdq_repack in
// include/mnb.h). Host code only: it runs once, when the plan is prepared,
// and reads every nibble once (no float weight is formed).
#include "../../include/mnb.h"

#include <cstring>

namespace {

// Element i of an ONNX-packed 4-bit tensor as an unsigned nibble; signed
// elements are shifted by 8 (two's complement x in [-8, 7] -> x + 8).
inline uint32_t Nibble(const uint8_t *p, int64_t i, bool is_signed) {
  const uint32_t v = (p[i >> 1] >> ((i & 1) * 4)) & 0xFu;
  return is_signed ? (v ^ 0x8u) : v;  // (v - 16 if v >= 8) + 8 == v ^ 8
}

} // namespace

extern "C" int mnb_qdq_repack(int64_t K, int64_t N, int32_t block_size, int32_t is_signed,
                              const uint8_t *x, const float *x_scale,
                              const uint8_t *x_zero_point, uint8_t *B, float *scales,
                              uint8_t *zero_points, int32_t *has_zero_points) {
  if (x == nullptr || x_scale == nullptr || B == nullptr || scales == nullptr ||
      zero_points == nullptr || has_zero_points == nullptr)
    return MNB_ERR_NULL_POINTER;
  if (K <= 0 || N <= 0 || K > (int64_t{1} << 31) || N > (int64_t{1} << 31))
    return MNB_ERR_BAD_SHAPE;
  if (block_size < 16 || (block_size & (block_size - 1)) != 0) return MNB_ERR_BAD_ATTRIBUTE;
  const bool sgn = is_signed != 0;
  const int64_t bs = block_size, nb = (K + bs - 1) / bs, row_bytes = nb * bs / 2;
  const int64_t zrow = (nb + 1) / 2;
  std::memset(B, 0, static_cast<size_t>(N * row_bytes));
  // B[n][k / bs][(k % bs) / 2], nibble k & 1 (bs is even, so k % bs and k have
  // the same parity). x is row-major [K][N]: walk it in storage order.
  for (int64_t k = 0; k < K; ++k) {
    const int64_t base = (k / bs) * (bs / 2) + (k % bs) / 2;
    const int shift = static_cast<int>(k & 1) * 4;
    for (int64_t n = 0; n < N; ++n)
      B[n * row_bytes + base] |= static_cast<uint8_t>(Nibble(x, k * N + n, sgn) << shift);
  }
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t n = 0; n < N; ++n) scales[n * nb + b] = x_scale[b * N + n];
  if (x_zero_point == nullptr && sgn) {
    *has_zero_points = 0;  // ONNX zero point 0 on signed nibbles == MatMulNBits' default 8
    return MNB_OK;
  }
  std::memset(zero_points, 0, static_cast<size_t>(N * zrow));
  if (x_zero_point != nullptr)
    for (int64_t b = 0; b < nb; ++b)
      for (int64_t n = 0; n < N; ++n)
        zero_points[n * zrow + b / 2] |=
            static_cast<uint8_t>(Nibble(x_zero_point, b * N + n, sgn) << ((b & 1) * 4));
  *has_zero_points = 1;  // UINT4 without x_zero_point: explicit zeros
  return MNB_OK;
}
