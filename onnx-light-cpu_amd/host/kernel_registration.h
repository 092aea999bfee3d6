// Kernel registration boundary of the MI355X MatMulNBits library.
//
// Mirrors the reference's registration API
// (onnx_light_cpu/kernels/kernel_registration.h:30-123,
//  onnx_light_cpu/kernels/kernel_usage.h) with the same names, the same
// record fields and the same failure behaviour (a duplicate
// (domain, op_type, device) in one pass throws std::invalid_argument;
// inventory mode records without installing). onnx-light's runtime headers
// (KernelDispatchTable, RuntimeContext, Tensor) are not available to this
// build, so the minimal runtime surface the adapter needs is declared here
// and the dispatch table is a process-local one keyed "domain:op_type" as
// onnx-light keys its own (test_onnx_light_kernel_registration.cc:149).
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <set>
#include <string>
#include <string_view>
#include <tuple>
#include <utility>
#include <vector>

namespace onnx_light_cpu_amd {

// Device the kernel runs on. kCPU/kUndefined exist in onnx-light; a GPU
// enumerator there is not pinned by the reference, so kGPU is this build's.
enum class Device : int32_t { kUndefined = 0, kCPU = 1, kGPU = 2 };

// TensorProto::DataType values used by this operator.
enum class DataType : int32_t { kUndefined = 0, kFloat = 1, kUint8 = 2, kInt32 = 6,
                                kFloat16 = 10, kUint4 = 21, kInt4 = 22 };

// A borrowed tensor: pointer, element type, shape and the memory it lives in.
struct TensorView {
  void *data = nullptr;
  DataType type = DataType::kUndefined;
  std::vector<int64_t> shape;
  Device device = Device::kGPU;

  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

// Integer attributes of one node (K, N, bits, block_size, accuracy_level).
struct NodeAttributes {
  std::map<std::string, int64_t> ints;

  std::optional<int64_t> GetInt(const std::string &name) const {
    auto it = ints.find(name);
    if (it == ints.end()) return std::nullopt;
    return it->second;
  }
};

// Per-run context: optional inputs, outputs, the stream, an output allocator
// (onnx-light's rt->MakeOutputTensor role) and a workspace allocator, all
// supplied by the caller for this one run.
class RuntimeContext {
public:
  using Allocator = std::function<void *(size_t bytes)>;

  std::vector<std::optional<TensorView>> inputs;
  std::vector<TensorView> outputs;
  void *stream = nullptr;
  Allocator allocate_output;
  // Device scratch for this run only, 16-byte aligned, usable in stream
  // order on `stream` until the run's work completes (a session's arena or a
  // caller buffer). Kernels never allocate device memory themselves.
  Allocator allocate_workspace;

  const TensorView *GetInput(size_t i) const {
    return i < inputs.size() && inputs[i].has_value() ? &*inputs[i] : nullptr;
  }
  // Allocates output i with `shape` through allocate_output, or checks a
  // preset output buffer of that shape.
  TensorView &MakeOutputTensor(size_t i, DataType type, std::vector<int64_t> shape);
  // `bytes` of workspace through allocate_workspace (nullptr for 0 bytes);
  // throws std::invalid_argument when there is no workspace allocator.
  void *Workspace(size_t bytes);
};

class KernelBase {
public:
  virtual ~KernelBase() = default;
  virtual void Run(RuntimeContext &rt) = 0;
};

using NodeKernelFn =
    std::function<std::unique_ptr<KernelBase>(const NodeAttributes &, RuntimeContext &)>;

struct KernelRegistration {
  std::string domain;
  std::string op_type;
  Device device = Device::kGPU;
  std::string kernel_name;
  std::vector<DataType> types;
  std::optional<int64_t> since_version;
  std::optional<int64_t> until_version;
};

class KernelRegistrationScope {
public:
  explicit KernelRegistrationScope(std::vector<KernelRegistration> *inventory = nullptr);
  ~KernelRegistrationScope();
  KernelRegistrationScope(const KernelRegistrationScope &) = delete;
  KernelRegistrationScope &operator=(const KernelRegistrationScope &) = delete;

private:
  friend void RegisterKernel(KernelRegistration info, NodeKernelFn fn);
  std::set<std::tuple<std::string, std::string, Device>> seen_;
  std::vector<KernelRegistration> *inventory_ = nullptr;
  bool owns_ = false;
};

// "" -> "ai.onnx", as onnx-light's NormaliseDomain (kernel_registration.cc:57).
std::string NormaliseDomain(std::string_view domain);

void RegisterKernel(KernelRegistration info, NodeKernelFn fn);
std::vector<KernelRegistration> CollectRegisteredKernels();

// The process-local dispatch table standing in for onnx-light's.
NodeKernelFn LookupKernel(const std::string &domain, const std::string &op_type, Device device);
std::vector<std::string> DispatchTableKeys();
void ClearDispatchTable();

// Usage log (onnx_light_cpu/kernels/kernel_usage.h).
void RecordKernelUsage(std::string_view name);
std::vector<std::string> UsedKernelNames();
void ClearUsedKernelNames();
void SetKernelUsageRecording(bool enabled) noexcept;
const std::vector<std::pair<std::string, std::string>> &RegisteredKernelNames();

} // namespace onnx_light_cpu_amd
