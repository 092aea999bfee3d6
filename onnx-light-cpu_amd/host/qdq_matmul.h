// Constant DequantizeLinear -> MatMul recognition: the roadmap's
// qwen3-int4-qdq export contract (docs/next_steps/2026/
// 2026_08_qwen3_inference.rst:96-101, 262), "recognize the constant QDQ
// pattern and pass packed weights directly to an internal weight-only plan;
// never materialize a complete float weight tensor". The weight input of
// MatMul(A, W), W = DequantizeLinear(x, x_scale, x_zero_point), is turned
// into the attributes and constant inputs of one com.microsoft::MatMulNBits
// node, which the registered MatMulNBitsKernel then serves.
#pragma once

#include "kernel_registration.h"

#include <cstdint>
#include <optional>
#include <vector>

namespace onnx_light_cpu_amd {

// DequantizeLinear's constant inputs and attributes, in host memory.
struct DequantizeLinearWeight {
  TensorView x;                            // INT4 or UINT4 [K, N], ONNX 4-bit packing
  TensorView x_scale;                      // float: [ceil(K/bs), N] blocked along K,
                                           // [N] per column, or one value per tensor
  std::optional<TensorView> x_zero_point;  // x's type, x_scale's shape; absent = 0
  NodeAttributes attrs;                    // "axis" (ONNX default 1), "block_size" (default 0)
};

// A MatMulNBits node equivalent to MatMul(A, DequantizeLinear(...)).
struct MatMulNBitsWeights {
  NodeAttributes attrs;               // K, N, bits = 4, block_size
  std::vector<uint8_t> B;             // [N, nb, block_size/2]
  std::vector<float> scales;          // [N, nb]
  std::vector<uint8_t> zero_points;   // [N, ceil(nb/2)]; empty when every zero point is 8
};

// Maps the pattern, or throws std::invalid_argument naming what does not map:
// blocked quantization must run along K (axis 0) with a power-of-two
// block_size >= 16; per-column (axis 1, scale [N]) and per-tensor scales map
// to one block of K, so K must then be a power of two >= 16.
MatMulNBitsWeights DequantizeLinearToMatMulNBits(const DequantizeLinearWeight &w);

} // namespace onnx_light_cpu_amd
