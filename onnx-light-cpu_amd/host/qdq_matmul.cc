#include "qdq_matmul.h"

#include "mnb.h"

#include <stdexcept>
#include <string>

namespace onnx_light_cpu_amd {
namespace {

[[noreturn]] void Fail(const std::string &what) {
  throw std::invalid_argument("onnx_light_cpu_amd::DequantizeLinearToMatMulNBits: " + what);
}

bool PowerOfTwoAtLeast16(int64_t v) { return v >= 16 && (v & (v - 1)) == 0; }

// Element i of an ONNX-packed 4-bit tensor (low nibble first).
uint8_t Nibble(const uint8_t *p, int64_t i) { return (p[i >> 1] >> ((i & 1) * 4)) & 0xF; }

} // namespace

MatMulNBitsWeights DequantizeLinearToMatMulNBits(const DequantizeLinearWeight &w) {
  const TensorView &x = w.x;
  if (x.type != DataType::kInt4 && x.type != DataType::kUint4)
    Fail("x must be INT4 or UINT4");
  if (x.shape.size() != 2) Fail("x must be a 2-D [K, N] MatMul weight");
  if (x.device != Device::kCPU || w.x_scale.device != Device::kCPU ||
      (w.x_zero_point && w.x_zero_point->device != Device::kCPU))
    Fail("the constant inputs must be in host memory");
  if (w.x_scale.type != DataType::kFloat) Fail("x_scale must be float");
  if (w.x_zero_point && w.x_zero_point->type != x.type)
    Fail("x_zero_point must have x's type");
  const int64_t K = x.shape[0], N = x.shape[1];
  if (K <= 0 || N <= 0) Fail("x must not be empty");
  const int64_t rank = 2;
  int64_t axis = w.attrs.GetInt("axis").value_or(1);
  if (axis < 0) axis += rank;
  const int64_t block = w.attrs.GetInt("block_size").value_or(0);

  // Bring the scales (and zero points) to the blocked [nb, N] form.
  int64_t bs = 0;
  std::vector<float> scale_rows;
  std::vector<uint8_t> zp_rows;  // ONNX-packed [nb, N]
  const float *scale = static_cast<const float *>(w.x_scale.data);
  const uint8_t *zp = w.x_zero_point ? static_cast<const uint8_t *>(w.x_zero_point->data) : nullptr;
  if (block > 0) {
    if (axis != 0) Fail("blocked quantization must run along K (axis 0), got axis " +
                        std::to_string(axis));
    if (!PowerOfTwoAtLeast16(block))
      Fail("block_size must be a power of two >= 16, got " + std::to_string(block));
    bs = block;
    const int64_t nb = (K + bs - 1) / bs;
    if (w.x_scale.shape != std::vector<int64_t>{nb, N})
      Fail("x_scale must be [ceil(K/block_size), N] = [" + std::to_string(nb) + ", " +
           std::to_string(N) + "]");
    if (w.x_zero_point && w.x_zero_point->shape != w.x_scale.shape)
      Fail("x_zero_point must have x_scale's shape");
  } else {
    const int64_t ns = w.x_scale.numel();
    if (ns == N && w.x_scale.shape.size() == 1) {
      if (axis != 1) Fail("per-axis scales must run along N (axis 1) for a MatMul weight");
    } else if (ns != 1) {
      Fail("x_scale must be blocked [ceil(K/block_size), N], per column [N] or per tensor");
    }
    if (w.x_zero_point && w.x_zero_point->numel() != ns)
      Fail("x_zero_point must have x_scale's shape");
    if (!PowerOfTwoAtLeast16(K))
      Fail("per-column and per-tensor scales map to one block of K, so K must be a power of "
           "two >= 16, got " + std::to_string(K));
    bs = K;
    if (ns == 1) {  // broadcast one scale (and zero point) to every column
      scale_rows.assign(static_cast<size_t>(N), scale[0]);
      scale = scale_rows.data();
      if (zp != nullptr) {
        const uint8_t z = Nibble(zp, 0);
        zp_rows.assign(static_cast<size_t>((N + 1) / 2), static_cast<uint8_t>(z | (z << 4)));
        zp = zp_rows.data();
      }
    }
  }

  const int64_t nb = (K + bs - 1) / bs;
  MatMulNBitsWeights out;
  out.attrs.ints = {{"K", K}, {"N", N}, {"bits", 4}, {"block_size", bs}};
  out.B.resize(static_cast<size_t>(N * nb * (bs / 2)));
  out.scales.resize(static_cast<size_t>(N * nb));
  out.zero_points.resize(static_cast<size_t>(N * ((nb + 1) / 2)));
  int32_t has_zp = 0;
  const int st = mnb_qdq_repack(K, N, static_cast<int32_t>(bs), x.type == DataType::kInt4,
                                static_cast<const uint8_t *>(x.data), scale, zp, out.B.data(),
                                out.scales.data(), out.zero_points.data(), &has_zp);
  if (st != MNB_OK) Fail(std::string("mnb_qdq_repack failed: ") + mnb_status_str(st));
  if (!has_zp) out.zero_points.clear();
  return out;
}

} // namespace onnx_light_cpu_amd
