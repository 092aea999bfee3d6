#include "matmul_nbits_kernel.h"

#include "register_kernels.h"

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace onnx_light_cpu_amd {
namespace {

[[noreturn]] void Fail(const std::string &what) {
  throw std::invalid_argument(std::string(MatMulNBitsKernel::kName) + ": " + what);
}

void CheckStatus(int status, const char *what) {
  if (status != MNB_OK) {
    std::string msg = std::string(what) + " failed: " + mnb_status_str(status);
    const char *detail = mnb_last_error();
    if ((status == MNB_ERR_HIP || status == MNB_ERR_NO_DEVICE || status == MNB_ERR_ALLOC) &&
        detail && *detail)
      msg += std::string(" (") + detail + ")";
    Fail(msg);
  }
}

int64_t RequireInt(const NodeAttributes &attrs, const char *name) {
  auto v = attrs.GetInt(name);
  if (!v) Fail(std::string("missing attribute '") + name + "'");
  return *v;
}

} // namespace

MatMulNBitsKernel::MatMulNBitsKernel(const NodeAttributes &attrs) {
  desc_.K = RequireInt(attrs, "K");
  desc_.N = RequireInt(attrs, "N");
  desc_.bits = static_cast<int32_t>(attrs.GetInt("bits").value_or(4));
  desc_.block_size = static_cast<int32_t>(RequireInt(attrs, "block_size"));
  desc_.accuracy_level = static_cast<int32_t>(attrs.GetInt("accuracy_level").value_or(0));
  desc_.has_zero_points = 0;
  if (desc_.bits != 4) Fail("only bits=4 is supported, got " + std::to_string(desc_.bits));
  if (desc_.K <= 0 || desc_.N <= 0) Fail("K and N must be positive");
  if (desc_.block_size < 16 || (desc_.block_size & (desc_.block_size - 1)) != 0)
    Fail("block_size must be a power of two >= 16, got " + std::to_string(desc_.block_size));
  if (desc_.accuracy_level < 0 || desc_.accuracy_level > 4)
    Fail("accuracy_level must be in [0, 4]");
}

MatMulNBitsKernel::~MatMulNBitsKernel() {
  for (auto &kv : plans_) mnb_plan_destroy(kv.second);
}

const mnb_plan *MatMulNBitsKernel::Plan(const TensorView &b, const TensorView &scales,
                                        const TensorView *zero_points) {
  const void *z = zero_points ? zero_points->data : nullptr;
  const auto key = std::make_tuple(static_cast<const void *>(b.data),
                                   static_cast<const void *>(scales.data), z);
  std::lock_guard<std::mutex> lock(mu_);
  auto it = plans_.find(key);
  if (it != plans_.end()) return it->second;
  mnb_desc d = desc_;
  d.has_zero_points = zero_points != nullptr;
  mnb_plan *p = nullptr;
  int st;
  if (b.device == Device::kGPU) {
    st = mnb_plan_create_device(&d, static_cast<const uint8_t *>(b.data),
                                static_cast<const float *>(scales.data),
                                static_cast<const uint8_t *>(z), &p);
  } else {
    st = mnb_plan_create(&d, static_cast<const uint8_t *>(b.data),
                         static_cast<const float *>(scales.data),
                         static_cast<const uint8_t *>(z), &p);
  }
  CheckStatus(st, "plan creation");
  plans_.emplace(key, p);
  return p;
}

size_t MatMulNBitsKernel::WorkspaceBytes(const TensorView &b, const TensorView &scales,
                                         const TensorView *zero_points, int64_t M) {
  size_t need = 0;
  CheckStatus(mnb_workspace_bytes(Plan(b, scales, zero_points), M, &need), "mnb_workspace_bytes");
  return need;
}

void MatMulNBitsKernel::Validate(const TensorView &a, const TensorView &b,
                                 const TensorView &scales, const TensorView *zero_points,
                                 const TensorView *bias) const {
  const int64_t K = desc_.K, N = desc_.N, bs = desc_.block_size;
  const int64_t nb = (K + bs - 1) / bs;
  if (a.type != DataType::kFloat) Fail("input A must be float");
  if (b.type != DataType::kUint8) Fail("input B must be uint8");
  if (scales.type != DataType::kFloat) Fail("input scales must be float");
  if (zero_points && zero_points->type != DataType::kUint8)
    Fail("input zero_points must be uint8 (float zero points are not supported)");
  if (a.shape.empty() || a.shape.back() != K)
    Fail("A's last dimension must equal K=" + std::to_string(K));
  if (a.device != Device::kGPU) Fail("A must be in device memory");
  if (b.numel() != N * nb * (bs / 2))
    Fail("B must have N*ceil(K/block_size)*block_size/2 = " + std::to_string(N * nb * (bs / 2)) +
         " bytes, got " + std::to_string(b.numel()));
  if (scales.numel() != N * nb)
    Fail("scales must have N*ceil(K/block_size) = " + std::to_string(N * nb) + " elements");
  if (zero_points && zero_points->numel() != N * ((nb + 1) / 2))
    Fail("zero_points must have N*ceil(n_blocks/2) = " + std::to_string(N * ((nb + 1) / 2)) +
         " bytes");
  if (bias && bias->type != DataType::kFloat) Fail("input bias must be float");
  if (bias && bias->numel() != N) Fail("bias must have N=" + std::to_string(N) + " elements");
  if (bias && bias->device != Device::kGPU) Fail("bias must be in device memory");
}

void MatMulNBitsKernel::operator()(const TensorView &a, const TensorView &b,
                                   const TensorView &scales, const TensorView *zero_points,
                                   TensorView &y, void *stream, void *workspace,
                                   size_t workspace_bytes, const TensorView *bias) {
  Validate(a, b, scales, zero_points, bias);
  const int64_t K = desc_.K;
  const mnb_plan *plan = Plan(b, scales, zero_points);
  const int64_t M = a.numel() / K;
  CheckStatus(mnb_run_ex(plan, M, static_cast<const float *>(a.data),
                         bias ? static_cast<const float *>(bias->data) : nullptr,
                         static_cast<float *>(y.data), workspace, workspace_bytes, stream, 0),
              "mnb_run_ex");
}

void MatMulNBitsKernel::Run(RuntimeContext &rt) {
  RecordKernelUsage(kName);
  if (rt.inputs.size() < 3 || rt.inputs.size() > 6)
    Fail("expects 3 to 6 inputs, got " + std::to_string(rt.inputs.size()));
  const TensorView *a = rt.GetInput(0);
  const TensorView *b = rt.GetInput(1);
  const TensorView *scales = rt.GetInput(2);
  const TensorView *zp = rt.GetInput(3);
  if (!a || !b || !scales) Fail("inputs A, B and scales are required");
  if (rt.GetInput(4)) Fail("input g_idx is not supported");
  const TensorView *bias = rt.GetInput(5);
  std::vector<int64_t> shape = a->shape;
  if (shape.empty()) Fail("A must have rank >= 1");
  shape.back() = desc_.N;
  Validate(*a, *b, *scales, zp, bias);
  TensorView &y = rt.MakeOutputTensor(0, DataType::kFloat, shape);
  const int64_t M = a->numel() / desc_.K;
  const size_t need = WorkspaceBytes(*b, *scales, zp, M);
  void *work = rt.Workspace(need);
  (*this)(*a, *b, *scales, zp, y, rt.stream, work, need, bias);
}

void RegisterMatMulNBitsKernel() {
  KernelRegistration info;
  info.domain = "com.microsoft";
  info.op_type = "MatMulNBits";
  info.device = Device::kGPU;
  info.kernel_name = MatMulNBitsKernel::kName;
  info.types = {DataType::kFloat};
  info.since_version = 1;
  RegisterKernel(std::move(info), [](const NodeAttributes &attrs, RuntimeContext &) {
    return std::unique_ptr<KernelBase>(new MatMulNBitsKernel(attrs));
  });
}

void RegisterAllKernels() {
  KernelRegistrationScope scope;
  RegisterMatMulNBitsKernel();
}

} // namespace onnx_light_cpu_amd
