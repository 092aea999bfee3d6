// com.microsoft::MatMulNBits operator adapter over the C ABI of include/mnb.h.
//
// Shaped like the reference's operator wrappers
// (onnx_light_cpu/kernels/math/matmul_kernel.h:14-26, matmul_kernel.cc:117-159;
//  integer_matmul_kernel.cc:298-378): Run() records usage, reads inputs
// (optional zero points), validates dtypes and shapes, allocates Y through the
// runtime and calls the compute operator(). Errors are std::invalid_argument
// with an "onnx_light_cpu_amd::MatMulNBitsKernel: ..." message.
#pragma once

#include "kernel_registration.h"
#include "mnb.h"

#include <mutex>

namespace onnx_light_cpu_amd {

class MatMulNBitsKernel : public KernelBase {
public:
  static constexpr const char *kName = "onnx_light_cpu_amd::MatMulNBitsKernel";

  // Reads attributes K, N, bits, block_size, accuracy_level; throws on
  // missing or invalid ones.
  explicit MatMulNBitsKernel(const NodeAttributes &attrs);
  ~MatMulNBitsKernel() override;

  void Run(RuntimeContext &rt) override;

  // Y = A * W^T (+ bias) for device tensors. B/scales/zero_points are the
  // node's constant initializers: the device plan is prepared on first use
  // and reused while the same buffers are passed. bias (input 5) is fp32 [N]
  // in device memory, or null.
  void operator()(const TensorView &a, const TensorView &b, const TensorView &scales,
                  const TensorView *zero_points, TensorView &y, void *stream,
                  const TensorView *bias = nullptr);

  const mnb_desc &desc() const { return desc_; }

private:
  void EnsurePlan(const TensorView &b, const TensorView &scales, const TensorView *zero_points);

  void *Workspace(int64_t M);

  mnb_desc desc_{};
  std::mutex mu_;
  void *work_ = nullptr;   // device workspace of the prefill path, grown on demand
  size_t work_bytes_ = 0;
  mnb_plan *plan_ = nullptr;
  const void *plan_b_ = nullptr;
  const void *plan_s_ = nullptr;
  const void *plan_z_ = nullptr;
};

} // namespace onnx_light_cpu_amd
