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

#include <map>
#include <mutex>
#include <tuple>

namespace onnx_light_cpu_amd {

class MatMulNBitsKernel : public KernelBase {
public:
  static constexpr const char *kName = "onnx_light_cpu_amd::MatMulNBitsKernel";

  // Reads attributes K, N, bits, block_size, accuracy_level; throws on
  // missing or invalid ones.
  explicit MatMulNBitsKernel(const NodeAttributes &attrs);
  ~MatMulNBitsKernel() override;

  // Reentrant: runs on one kernel object may overlap in time from several
  // host threads (distinct streams, outputs and workspaces).
  void Run(RuntimeContext &rt) override;

  // Y = A * W^T (+ bias) for device tensors. B/scales/zero_points are the
  // node's constant initializers: the device plan for a set of constant
  // buffers is prepared once (on first use, under a lock) and kept, read-only,
  // until the kernel object is destroyed. bias (input 5) is fp32 [N] in
  // device memory, or null. The workspace (size: WorkspaceBytes) comes from
  // the caller; this call allocates no device memory.
  void operator()(const TensorView &a, const TensorView &b, const TensorView &scales,
                  const TensorView *zero_points, TensorView &y, void *stream, void *workspace,
                  size_t workspace_bytes, const TensorView *bias = nullptr);

  // Workspace bytes a run of M rows needs with these constants (prepares the
  // plan if needed).
  size_t WorkspaceBytes(const TensorView &b, const TensorView &scales,
                        const TensorView *zero_points, int64_t M);

  const mnb_desc &desc() const { return desc_; }

private:
  // Input types, shapes and placement against the node's attributes; throws
  // before any device call.
  void Validate(const TensorView &a, const TensorView &b, const TensorView &scales,
                const TensorView *zero_points, const TensorView *bias) const;

  // The plan of these constant buffers, created once and never destroyed
  // before the kernel object (a run on another thread may be using it).
  // Plans are keyed by the buffers' addresses and never evicted: the inputs
  // must be constants that stay allocated and unchanged while the kernel
  // object lives (a graph's initializers over a session). A buffer freed and
  // reallocated at the same address would meet the plan derived from the old
  // contents. Device buffers are read once, when the plan is created, after
  // all work issued on the device so far has finished
  // (mnb_plan_create_device).
  const mnb_plan *Plan(const TensorView &b, const TensorView &scales,
                       const TensorView *zero_points);

  mnb_desc desc_{};
  std::mutex mu_;
  std::map<std::tuple<const void *, const void *, const void *>, mnb_plan *> plans_;
};

} // namespace onnx_light_cpu_amd
