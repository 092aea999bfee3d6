// Registration boundary and usage log; behaviour follows
// onnx_light_cpu/kernels/kernel_registration.cc:56-100 and kernel_usage.cc:36-56.
#include "kernel_registration.h"

#include "register_kernels.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdexcept>

namespace onnx_light_cpu_amd {
namespace {

KernelRegistrationScope *&CurrentScope() {
  thread_local KernelRegistrationScope *scope = nullptr;
  return scope;
}

struct DispatchTable {
  std::mutex mu;
  std::map<std::string, NodeKernelFn> fns;  // "domain:op_type@device"
};

DispatchTable &Table() {
  static DispatchTable t;
  return t;
}

std::string Key(const std::string &domain, const std::string &op, Device device) {
  return domain + ":" + op + "@" + std::to_string(static_cast<int32_t>(device));
}

struct UsageLog {
  std::mutex mu;
  std::vector<std::string> names;
  std::atomic<bool> enabled{true};
};

UsageLog &Usage() {
  static UsageLog u;
  return u;
}

} // namespace

TensorView &RuntimeContext::MakeOutputTensor(size_t i, DataType type, std::vector<int64_t> shape) {
  if (outputs.size() <= i) outputs.resize(i + 1);
  TensorView &out = outputs[i];
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const size_t elem = type == DataType::kFloat16 ? 2 : (type == DataType::kUint8 ? 1 : 4);
  if (out.data != nullptr) {
    if (out.numel() != n || out.type != type)
      throw std::invalid_argument("onnx_light_cpu_amd::RuntimeContext: preset output " +
                                  std::to_string(i) + " does not match the computed shape");
  } else {
    if (!allocate_output)
      throw std::invalid_argument("onnx_light_cpu_amd::RuntimeContext: no output allocator");
    out.data = allocate_output(static_cast<size_t>(n) * elem);
    if (out.data == nullptr && n != 0)
      throw std::runtime_error("onnx_light_cpu_amd::RuntimeContext: output allocation failed");
  }
  out.type = type;
  out.shape = std::move(shape);
  out.device = Device::kGPU;
  return out;
}

void *RuntimeContext::Workspace(size_t bytes) {
  if (bytes == 0) return nullptr;
  if (!allocate_workspace)
    throw std::invalid_argument("onnx_light_cpu_amd::RuntimeContext: no workspace allocator (" +
                                std::to_string(bytes) + " bytes needed)");
  void *p = allocate_workspace(bytes);
  if (p == nullptr)
    throw std::runtime_error("onnx_light_cpu_amd::RuntimeContext: workspace allocation failed");
  return p;
}

KernelRegistrationScope::KernelRegistrationScope(std::vector<KernelRegistration> *inventory) {
  if (CurrentScope() == nullptr) {
    CurrentScope() = this;
    inventory_ = inventory;
    owns_ = true;
  }
}

KernelRegistrationScope::~KernelRegistrationScope() {
  if (owns_) CurrentScope() = nullptr;
}

std::string NormaliseDomain(std::string_view domain) {
  return domain.empty() ? std::string("ai.onnx") : std::string(domain);
}

void RegisterKernel(KernelRegistration info, NodeKernelFn fn) {
  info.domain = NormaliseDomain(info.domain);
  std::optional<KernelRegistrationScope> fallback;
  if (CurrentScope() == nullptr) fallback.emplace();
  KernelRegistrationScope *scope = CurrentScope();
  const auto key = std::make_tuple(info.domain, info.op_type, info.device);
  if (!scope->seen_.insert(key).second) {
    throw std::invalid_argument("onnx_light_cpu_amd::RegisterKernel: duplicate registration for "
                                "domain '" + info.domain + "', operator '" + info.op_type +
                                "', device " +
                                std::to_string(static_cast<int32_t>(info.device)) + ".");
  }
  if (scope->inventory_ != nullptr) {
    scope->inventory_->push_back(std::move(info));
    return;
  }
  DispatchTable &t = Table();
  std::lock_guard<std::mutex> lock(t.mu);
  t.fns[Key(info.domain, info.op_type, info.device)] = std::move(fn);
}

std::vector<KernelRegistration> CollectRegisteredKernels() {
  std::vector<KernelRegistration> inventory;
  {
    KernelRegistrationScope scope(&inventory);
    RegisterAllKernels();
  }
  std::sort(inventory.begin(), inventory.end(),
            [](const KernelRegistration &a, const KernelRegistration &b) {
              return std::tie(a.domain, a.op_type, a.device, a.kernel_name) <
                     std::tie(b.domain, b.op_type, b.device, b.kernel_name);
            });
  return inventory;
}

NodeKernelFn LookupKernel(const std::string &domain, const std::string &op_type, Device device) {
  DispatchTable &t = Table();
  std::lock_guard<std::mutex> lock(t.mu);
  auto it = t.fns.find(Key(NormaliseDomain(domain), op_type, device));
  return it == t.fns.end() ? NodeKernelFn() : it->second;
}

std::vector<std::string> DispatchTableKeys() {
  DispatchTable &t = Table();
  std::lock_guard<std::mutex> lock(t.mu);
  std::vector<std::string> keys;
  for (const auto &kv : t.fns) keys.push_back(kv.first);
  return keys;
}

void ClearDispatchTable() {
  DispatchTable &t = Table();
  std::lock_guard<std::mutex> lock(t.mu);
  t.fns.clear();
}

void RecordKernelUsage(std::string_view name) {
  UsageLog &u = Usage();
  if (!u.enabled.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(u.mu);
  u.names.emplace_back(name);
}

std::vector<std::string> UsedKernelNames() {
  UsageLog &u = Usage();
  std::lock_guard<std::mutex> lock(u.mu);
  return u.names;
}

void ClearUsedKernelNames() {
  UsageLog &u = Usage();
  std::lock_guard<std::mutex> lock(u.mu);
  u.names.clear();
}

void SetKernelUsageRecording(bool enabled) noexcept {
  Usage().enabled.store(enabled, std::memory_order_relaxed);
}

const std::vector<std::pair<std::string, std::string>> &RegisteredKernelNames() {
  static const std::vector<std::pair<std::string, std::string>> names = [] {
    std::vector<std::pair<std::string, std::string>> out;
    for (const auto &r : CollectRegisteredKernels()) out.emplace_back(r.op_type, r.kernel_name);
    return out;
  }();
  return names;
}

} // namespace onnx_light_cpu_amd
