// C entry points over the C++ host side, for the Python mirror
// (the role of onnx_light_cpu/onnx_py/_cpuregister.cc:62-114: register,
// inventory, usage log) plus a node runner that goes through the dispatch
// table the way onnx-light's RunNode would. Exceptions never cross this
// boundary: failures return -1 and leave a message for olc_amd_last_error().
#include "kernel_registration.h"
#include "qdq_matmul.h"
#include "register_kernels.h"

#include <algorithm>
#include <cstring>
#include <exception>
#include <sstream>
#include <string>

namespace {

thread_local std::string g_error;

size_t CopyOut(const std::string &s, char *buf, size_t cap) {
  if (buf != nullptr && cap > 0) {
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return s.size() + 1;
}

template <typename F> int Guard(F &&f) {
  try {
    f();
    g_error.clear();
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  } catch (...) {
    g_error = "unknown exception";
    return -1;
  }
}

} // namespace

using namespace onnx_light_cpu_amd;

extern "C" {

const char *olc_amd_last_error(void) { return g_error.c_str(); }

int olc_amd_register_all_kernels(void) {
  return Guard([] { RegisterAllKernels(); });
}

int olc_amd_register_matmul_nbits_kernel(void) {
  return Guard([] { RegisterMatMulNBitsKernel(); });
}

// Runs one registration pass that registers the listed operators
// (comma-separated op_type names) in order, as RegisterAllKernels does for the
// full list; a repeated name fails the pass with the duplicate error.
int olc_amd_register_pass(const char *op_types) {
  return Guard([&] {
    KernelRegistrationScope scope;
    std::string list = op_types ? op_types : "";
    size_t pos = 0;
    while (pos <= list.size()) {
      const size_t end = std::min(list.find(',', pos), list.size());
      const std::string op = list.substr(pos, end - pos);
      if (op == "MatMulNBits")
        RegisterMatMulNBitsKernel();
      else if (!op.empty())
        throw std::invalid_argument("onnx_light_cpu_amd::RegisterKernel: unknown operator '" +
                                    op + "'");
      pos = end + 1;
    }
  });
}

// One line per registration: domain, op_type, device, kernel_name, types
// (comma separated TensorProto values), since, until (-1 = none); tab separated.
size_t olc_amd_registered_kernels(char *buf, size_t cap) {
  std::ostringstream os;
  try {
    for (const auto &r : CollectRegisteredKernels()) {
      os << r.domain << '\t' << r.op_type << '\t' << static_cast<int32_t>(r.device) << '\t'
         << r.kernel_name << '\t';
      for (size_t i = 0; i < r.types.size(); ++i)
        os << (i ? "," : "") << static_cast<int32_t>(r.types[i]);
      os << '\t' << r.since_version.value_or(-1) << '\t' << r.until_version.value_or(-1) << '\n';
    }
  } catch (const std::exception &e) {
    g_error = e.what();
    return 0;
  }
  return CopyOut(os.str(), buf, cap);
}

size_t olc_amd_used_kernel_names(char *buf, size_t cap) {
  std::string s;
  for (const auto &n : UsedKernelNames()) s += n + "\n";
  return CopyOut(s, buf, cap);
}

void olc_amd_clear_used_kernel_names(void) { ClearUsedKernelNames(); }

void olc_amd_set_usage_recording(int enabled) { SetKernelUsageRecording(enabled != 0); }

size_t olc_amd_dispatch_keys(char *buf, size_t cap) {
  std::string s;
  for (const auto &k : DispatchTableKeys()) s += k + "\n";
  return CopyOut(s, buf, cap);
}

void olc_amd_clear_dispatch_table(void) { ClearDispatchTable(); }

} // extern "C"

namespace {

// The RuntimeContext of one run from the C arrays: inputs given as parallel
// arrays (a NULL input pointer means the optional input is absent; dims holds
// every input's dimensions back to back), a caller-provided device output of
// output_numel floats, and a caller-provided device workspace that the
// context hands out when it is large enough.
RuntimeContext MakeContext(int n_inputs, void *const *input_ptrs, const int32_t *input_types,
                           const int32_t *input_devices, const int32_t *input_ranks,
                           const int64_t *dims, void *output, int64_t output_numel,
                           void *workspace, size_t workspace_bytes, void *stream) {
  RuntimeContext rt;
  rt.stream = stream;
  const int64_t *d = dims;
  for (int i = 0; i < n_inputs; ++i) {
    if (input_ptrs[i] == nullptr) {
      rt.inputs.emplace_back(std::nullopt);
      d += input_ranks[i];
      continue;
    }
    TensorView t;
    t.data = input_ptrs[i];
    t.type = static_cast<DataType>(input_types[i]);
    t.device = static_cast<Device>(input_devices[i]);
    t.shape.assign(d, d + input_ranks[i]);
    d += input_ranks[i];
    rt.inputs.emplace_back(std::move(t));
  }
  TensorView y;
  y.data = output;
  y.type = DataType::kFloat;
  y.shape = {output_numel};
  rt.outputs.push_back(y);
  rt.allocate_workspace = [workspace, workspace_bytes](size_t bytes) -> void * {
    if (bytes > workspace_bytes)
      throw std::invalid_argument("onnx_light_cpu_amd::RunNode: workspace of " +
                                  std::to_string(workspace_bytes) + " bytes, " +
                                  std::to_string(bytes) + " needed");
    return workspace;
  };
  return rt;
}

NodeAttributes MakeAttributes(int n_attrs, const char *const *attr_names,
                              const int64_t *attr_values) {
  NodeAttributes attrs;
  for (int i = 0; i < n_attrs; ++i) attrs.ints[attr_names[i]] = attr_values[i];
  return attrs;
}

NodeKernelFn Lookup(const char *domain, const char *op_type, int device) {
  NodeKernelFn fn = LookupKernel(domain ? domain : "", op_type ? op_type : "",
                                 static_cast<Device>(device));
  if (!fn)
    throw std::invalid_argument("onnx_light_cpu_amd::RunNode: no kernel for '" +
                                NormaliseDomain(domain ? domain : "") + ":" +
                                (op_type ? op_type : "") + "'");
  return fn;
}

} // namespace

extern "C" {

// Runs one node through the dispatch table (a kernel object created for this
// run). The workspace is a caller device buffer of workspace_bytes (NULL/0
// when the run needs none).
int olc_amd_run_node(const char *domain, const char *op_type, int device, int n_attrs,
                     const char *const *attr_names, const int64_t *attr_values, int n_inputs,
                     void *const *input_ptrs, const int32_t *input_types,
                     const int32_t *input_devices, const int32_t *input_ranks,
                     const int64_t *dims, void *output, int64_t output_numel, void *workspace,
                     size_t workspace_bytes, void *stream) {
  return Guard([&] {
    NodeKernelFn fn = Lookup(domain, op_type, device);
    RuntimeContext rt = MakeContext(n_inputs, input_ptrs, input_types, input_devices,
                                    input_ranks, dims, output, output_numel, workspace,
                                    workspace_bytes, stream);
    std::unique_ptr<KernelBase> kernel = fn(MakeAttributes(n_attrs, attr_names, attr_values), rt);
    kernel->Run(rt);
  });
}

// One kernel object kept across runs, as a session keeps a node's kernel:
// created from the dispatch table once, run any number of times (also from
// several threads at once, each with its own stream, output and workspace),
// destroyed once. Returns NULL on failure (message in olc_amd_last_error).
void *olc_amd_kernel_create(const char *domain, const char *op_type, int device, int n_attrs,
                            const char *const *attr_names, const int64_t *attr_values) {
  KernelBase *out = nullptr;
  const int rc = Guard([&] {
    NodeKernelFn fn = Lookup(domain, op_type, device);
    RuntimeContext rt;
    out = fn(MakeAttributes(n_attrs, attr_names, attr_values), rt).release();
  });
  return rc == 0 ? out : nullptr;
}

int olc_amd_kernel_run(void *kernel, int n_inputs, void *const *input_ptrs,
                       const int32_t *input_types, const int32_t *input_devices,
                       const int32_t *input_ranks, const int64_t *dims, void *output,
                       int64_t output_numel, void *workspace, size_t workspace_bytes,
                       void *stream) {
  return Guard([&] {
    if (kernel == nullptr) throw std::invalid_argument("onnx_light_cpu_amd::RunNode: null kernel");
    RuntimeContext rt = MakeContext(n_inputs, input_ptrs, input_types, input_devices,
                                    input_ranks, dims, output, output_numel, workspace,
                                    workspace_bytes, stream);
    static_cast<KernelBase *>(kernel)->Run(rt);
  });
}

void olc_amd_kernel_destroy(void *kernel) { delete static_cast<KernelBase *>(kernel); }

// DequantizeLinearToMatMulNBits for the Python mirror: x is INT4 (x_type 22)
// or UINT4 (21) [K, N], x_scale fp32 with scale_rank dims, x_zero_point of
// x's type or NULL; axis_set = 0 means the ONNX default axis. Outputs go to
// caller buffers of the given capacities (elements); *out_block_size and
// *has_zero_points describe the MatMulNBits node.
int olc_amd_dequantize_linear_to_matmul_nbits(
    int x_type, int64_t K, int64_t N, const uint8_t *x, const float *x_scale, int scale_rank,
    const int64_t *scale_dims, const uint8_t *x_zero_point, int axis_set, int64_t axis,
    int64_t block_size, int64_t *out_block_size, uint8_t *B, size_t B_cap, float *scales,
    size_t scales_cap, uint8_t *zero_points, size_t zero_points_cap, int *has_zero_points) {
  return Guard([&] {
    DequantizeLinearWeight w;
    w.x.data = const_cast<uint8_t *>(x);
    w.x.type = static_cast<DataType>(x_type);
    w.x.shape = {K, N};
    w.x.device = Device::kCPU;
    w.x_scale.data = const_cast<float *>(x_scale);
    w.x_scale.type = DataType::kFloat;
    w.x_scale.shape.assign(scale_dims, scale_dims + scale_rank);
    w.x_scale.device = Device::kCPU;
    if (x_zero_point != nullptr) {
      TensorView z = w.x_scale;
      z.data = const_cast<uint8_t *>(x_zero_point);
      z.type = w.x.type;
      w.x_zero_point = z;
    }
    if (axis_set) w.attrs.ints["axis"] = axis;
    if (block_size > 0) w.attrs.ints["block_size"] = block_size;
    MatMulNBitsWeights m = DequantizeLinearToMatMulNBits(w);
    if (m.B.size() > B_cap || m.scales.size() > scales_cap ||
        m.zero_points.size() > zero_points_cap)
      throw std::invalid_argument("olc_amd_dequantize_linear_to_matmul_nbits: buffer too small");
    std::copy(m.B.begin(), m.B.end(), B);
    std::copy(m.scales.begin(), m.scales.end(), scales);
    std::copy(m.zero_points.begin(), m.zero_points.end(), zero_points);
    *out_block_size = *m.attrs.GetInt("block_size");
    *has_zero_points = m.zero_points.empty() ? 0 : 1;
  });
}

} // extern "C"
