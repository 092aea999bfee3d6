// C ABI of the MatMulNBits library: plan lifetime, validation, dispatch.
//
// Validation mirrors the reference operator wrappers' argument checks
// (onnx_light_cpu/kernels/math/matmul_kernel.cc:38-41, 118-133;
// integer_matmul_kernel.cc:153-174) but reports status codes instead of
// throwing, and it runs before any HIP call.
#include "../../include/mnb.h"
#include "mnb_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <new>
#include <vector>

struct mnb_plan {
  mnb_desc desc;  // desc.N = weight rows the kernels see (2 I for a gate/up plan)
  mnb::WeightView view;
  int device;
  bool owns;
  bool gate_up;   // rows are gate/up pairs; runs write silu(gate) * up, N / 2 columns
  uint8_t *dB;
  float *dS;
  uint8_t *dZ;
  int32_t *dColExp;  // always plan-owned: per weight row power-of-two scale exponent
  uint8_t *dBp;      // plan-owned prefill layout of the weights (nullptr: shape not served)
  uint8_t *dSp;
  float *dSd;        // plan-owned decode layout of the block scales (nullptr: not served)
  uint32_t *dZd;     // and of the zero points (nullptr without zero points)
};

namespace {

thread_local char g_last_error[256] = "";

void SetLastError(const char *what, hipError_t e) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(e));
}

bool IsPow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int Log2(int64_t v) {
  int r = 0;
  while ((int64_t{1} << r) < v) ++r;
  return r;
}

int ValidateDesc(const mnb_desc *d) {
  if (d == nullptr) return MNB_ERR_NULL_POINTER;
  if (d->bits != 4) return MNB_ERR_UNSUPPORTED;
  if (!IsPow2(d->block_size) || d->block_size < 16) return MNB_ERR_BAD_ATTRIBUTE;
  if (d->accuracy_level < 0 || d->accuracy_level > 4) return MNB_ERR_BAD_ATTRIBUTE;
  if (d->K <= 0 || d->N <= 0) return MNB_ERR_BAD_SHAPE;
  if (d->K > (int64_t{1} << 30) || d->N > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  if (d->has_zero_points != 0 && d->has_zero_points != 1) return MNB_ERR_BAD_ATTRIBUTE;
  return MNB_OK;
}

void Sizes(const mnb_desc *d, int64_t *nb, int64_t *row_bytes, int64_t *zp_row_bytes) {
  *nb = (d->K + d->block_size - 1) / d->block_size;
  *row_bytes = *nb * d->block_size / 2;
  *zp_row_bytes = (*nb + 1) / 2;
}

int CheckDevice(int *device) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    SetLastError("hipGetDevice", e);
    return MNB_ERR_NO_DEVICE;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    SetLastError("hipGetDeviceProperties", e);
    return MNB_ERR_NO_DEVICE;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    std::snprintf(g_last_error, sizeof(g_last_error), "device %d is %s, this library is gfx950",
                  dev, prop.gcnArchName);
    return MNB_ERR_NO_DEVICE;
  }
  *device = dev;
  return MNB_OK;
}

int DeviceCUs(int dev) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  return cus;
}

void FillView(mnb_plan *p) {
  int64_t nb, row_bytes, zp_row_bytes;
  Sizes(&p->desc, &nb, &row_bytes, &zp_row_bytes);
  p->view.B = p->dB;
  p->view.scales = p->dS;
  p->view.zp = p->desc.has_zero_points ? p->dZ : nullptr;
  p->view.has_zp = p->desc.has_zero_points;
  p->view.col_exp = p->dColExp;
  p->view.Bp = p->dBp;
  p->view.Sp = p->dSp;
  p->view.Sd = p->dSd;
  p->view.Zd = p->dZd;
  p->view.K = p->desc.K;
  p->view.N = p->desc.N;
  p->view.nb = nb;
  p->view.row_bytes = row_bytes;
  p->view.zp_row_bytes = zp_row_bytes;
  p->view.block_size = p->desc.block_size;
  p->view.log2_bs = Log2(p->desc.block_size);
  p->view.num_cus = DeviceCUs(p->device);
}

void FreePlanMemory(mnb_plan *p) {
  if (p->owns) {
    if (p->dB) (void)hipFree(p->dB);
    if (p->dS) (void)hipFree(p->dS);
    if (p->dZ) (void)hipFree(p->dZ);
  }
  if (p->dColExp) (void)hipFree(p->dColExp);
  if (p->dBp) (void)hipFree(p->dBp);
  if (p->dSp) (void)hipFree(p->dSp);
  if (p->dSd) (void)hipFree(p->dSd);
  if (p->dZd) (void)hipFree(p->dZd);
  p->dSd = nullptr;
  p->dZd = nullptr;
  p->dB = nullptr;
  p->dS = nullptr;
  p->dZ = nullptr;
  p->dColExp = nullptr;
  p->dBp = nullptr;
  p->dSp = nullptr;
}

// Whether a plan can serve every path from the re-laid copies alone: the
// fragment-ordered GEMV for every M <= 4 (the decode path without a
// workspace runs it on groups of up to 4 rows) and as the M = 1 choice (its
// 64-row groups cover most CUs), the small-M MFMA decode up to 16 rows, and
// the prefill kernel for the GEMM path. Plans whose M = 1 decode is faster on
// the original layout (narrow weights: GemvM1Kernel) keep both copies.
bool CompactEligible(const mnb::WeightView &w) {
  if (w.Bp == nullptr || w.Sp == nullptr || w.Sd == nullptr || (w.has_zp && w.Zd == nullptr))
    return false;
  for (int64_t m = 1; m <= 4; ++m)
    if (!mnb::GemvFragSupports(w, m)) return false;
  return mnb::GemvFragPreferred(w, 1) && mnb::DecodeFragSupports(w, 16) &&
         mnb::PrefillSupports(w, 1);
}

// Plan-time constants derived from the device copies of the weights (run
// once, synchronously, on the null stream): the per-row scale exponents and,
// for shapes the prefill kernel serves, its fragment-ordered copy of the
// weights with per-block scale / zero-point words (1.06x the packed B bytes
// at block size 128, 1.25x at 32).
// Fills the plan's view.
int DerivePlanConstants(mnb_plan *p) {
  FillView(p);
  hipError_t e = hipMalloc(reinterpret_cast<void **>(&p->dColExp),
                           static_cast<size_t>(p->desc.N) * sizeof(int32_t));
  if (e != hipSuccess) {
    SetLastError("hipMalloc", e);
    return MNB_ERR_ALLOC;
  }
  e = mnb::LaunchColExp(p->dS, p->dColExp, p->desc.N, p->view.nb, nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) {
    SetLastError("plan constants", e);
    return MNB_ERR_HIP;
  }
  FillView(p);
  if (mnb::PrefillLayoutWanted(p->view)) {
    size_t sp_bytes = 0;
    const size_t bp_bytes = mnb::PrefillLayoutBytes(p->view, &sp_bytes);
    e = hipMalloc(reinterpret_cast<void **>(&p->dBp), bp_bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&p->dSp), sp_bytes);
    if (e != hipSuccess) {
      SetLastError("hipMalloc", e);
      return MNB_ERR_ALLOC;
    }
    e = mnb::LaunchPrefillRelayout(p->view, p->dBp, p->dSp, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
      SetLastError("prefill re-layout", e);
      return MNB_ERR_HIP;
    }
    FillView(p);
    // The small-M decode kernel reads the same fragment-ordered weights with
    // fp32 block scales and zero points re-laid per 64-row group.
    if (mnb::DecodeFragLayoutWanted(p->view)) {
      size_t zd_bytes = 0;
      const size_t sd_bytes = mnb::DecodeFragScaleBytes(p->view, &zd_bytes);
      e = hipMalloc(reinterpret_cast<void **>(&p->dSd), sd_bytes);
      if (e == hipSuccess && zd_bytes > 0) e = hipMalloc(reinterpret_cast<void **>(&p->dZd), zd_bytes);
      if (e != hipSuccess) {
        SetLastError("hipMalloc", e);
        return MNB_ERR_ALLOC;
      }
      e = mnb::LaunchDecodeFragRelayout(p->view, p->dSd, p->dZd, nullptr);
      if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
      if (e != hipSuccess) {
        SetLastError("decode re-layout", e);
        return MNB_ERR_HIP;
      }
      FillView(p);
    }
  }
  // Compact plan: where every automatic route reads only the re-laid copies,
  // a plan that owns its weights drops the original layout (about 2.07x the
  // weights' bytes become 1.07x at bs = 128 with zero points).
  if (p->owns && CompactEligible(p->view)) {
    (void)hipFree(p->dB);
    (void)hipFree(p->dS);
    if (p->dZ) (void)hipFree(p->dZ);
    p->dB = nullptr;
    p->dS = nullptr;
    p->dZ = nullptr;
    FillView(p);
  }
  return MNB_OK;
}

int CheckInputs(const mnb_desc *desc, const void *B, const void *scales, const void *zp,
                mnb_plan **out_plan) {
  if (out_plan == nullptr) return MNB_ERR_NULL_POINTER;
  *out_plan = nullptr;
  int st = ValidateDesc(desc);
  if (st != MNB_OK) return st;
  if (B == nullptr || scales == nullptr) return MNB_ERR_NULL_POINTER;
  if (desc->has_zero_points && zp == nullptr) return MNB_ERR_NULL_POINTER;
  if (!desc->has_zero_points && zp != nullptr) return MNB_ERR_UNSUPPORTED;
  return MNB_OK;
}

} // namespace

namespace mnb {

__global__ __launch_bounds__(256) void SiluMulKernel(const float *__restrict__ Y,
                                                     float *__restrict__ H, int64_t half_mn) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < half_mn) {
    const float2 gu = reinterpret_cast<const float2 *>(Y)[i];
    H[i] = SiluMul(gu.x, gu.y);
  }
}

hipError_t LaunchSiluMul(const float *Y, float *H, int64_t M, int64_t N, hipStream_t s) {
  const int64_t half_mn = M * N / 2;
  hipLaunchKernelGGL(SiluMulKernel, dim3(static_cast<unsigned>((half_mn + 255) / 256)), dim3(256),
                     0, s, Y, H, half_mn);
  return hipGetLastError();
}

// Sum over the 256 threads of a workgroup (4 wavefronts); every thread gets it.
__device__ __forceinline__ float BlockSum256(float v, float *red) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row: the normalized row x * inv_rms * gamma,
// inv_rms = 1 / sqrt(mean(x^2) + eps).
__global__ __launch_bounds__(256) void RmsNormKernel(const float *__restrict__ X,
                                                     const float *__restrict__ gamma,
                                                     float *__restrict__ Xn, int64_t K,
                                                     float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float4 *x = reinterpret_cast<const float4 *>(X + row * K);
  const int64_t n4 = K / 4;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < n4; i += 256) {
    const float4 v = x[i];
    s += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
  }
  const float inv = 1.0f / sqrtf(BlockSum256(s, red) / static_cast<float>(K) + eps);
  const float4 *g = reinterpret_cast<const float4 *>(gamma);
  float4 *y = reinterpret_cast<float4 *>(Xn + row * K);
  for (int64_t i = threadIdx.x; i < n4; i += 256) {
    const float4 v = x[i], gg = g[i];
    y[i] = make_float4(v.x * inv * gg.x, v.y * inv * gg.y, v.z * inv * gg.z, v.w * inv * gg.w);
  }
}

__global__ __launch_bounds__(256) void ColExpKernel(const float *__restrict__ S,
                                                    int32_t *__restrict__ E, int64_t N,
                                                    int64_t nb) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (n >= N) return;
  float m = 0.0f;
  for (int64_t b = 0; b < nb; ++b) m = fmaxf(m, fabsf(S[n * nb + b]));
  E[n] = RangeExponent(m, kScaleExpTarget);
}

hipError_t LaunchColExp(const float *scales, int32_t *col_exp, int64_t N, int64_t nb,
                        hipStream_t s) {
  hipLaunchKernelGGL(ColExpKernel, dim3(static_cast<unsigned>((N + 255) / 256)), dim3(256), 0, s,
                     scales, col_exp, N, nb);
  return hipGetLastError();
}

hipError_t LaunchRmsNorm(const float *X, const float *gamma, float *Xn, int64_t M, int64_t K,
                         float eps, hipStream_t s) {
  hipLaunchKernelGGL(RmsNormKernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, s, X, gamma,
                     Xn, K, eps);
  return hipGetLastError();
}

} // namespace mnb

static size_t Round256(size_t v) { return (v + 255) / 256 * 256; }

// Workspace of mnb_run_no_alloc: a file-scope device array, one copy per GPU
// the library runs on, held until the process ends. In host code `scratch`
// names a host-side stand-in, never the device memory: host code uses only
// the per-device address from hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t{MNB_NO_ALLOC_SCRATCH_BYTES};
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with
// that device current) and kept. Returns MNB_OK or MNB_ERR_HIP.
int ScratchAddress(int device, void **out) {
  if (device < 0 || device >= kMaxScratchDevices) {
    std::snprintf(g_last_error, sizeof(g_last_error), "device %d: no scratch slot", device);
    return MNB_ERR_NO_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      SetLastError("hipGetSymbolAddress(scratch)", e);
      return MNB_ERR_HIP;
    }
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return MNB_OK;
}

} // namespace

// Bytes of the gate/up plans' scratch sum y = A * W^T (M x N floats, N = 2 I)
// at the front of the workspace, rounded up to keep what follows aligned.
static size_t GateUpScratchBytes(const mnb_plan *plan, int64_t M) {
  if (!plan->gate_up) return 0;
  return (static_cast<size_t>(M) * static_cast<size_t>(plan->view.N) * 4 + 255) / 256 * 256;
}

// Y[m][n] += bias[n]: MatMulNBits' optional bias input, an epilogue over the
// finished Y on the same stream (every path's kernels have completed their
// writes of Y when it starts).
__global__ __launch_bounds__(256) void AddBiasKernel(float *__restrict__ Y,
                                                     const float *__restrict__ bias, int64_t mn,
                                                     int64_t N) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < mn) Y[i] += bias[i % N];
}

static hipError_t LaunchAddBias(float *Y, const float *bias, int64_t M, int64_t N,
                                hipStream_t s) {
  const int64_t mn = M * N;
  hipLaunchKernelGGL(AddBiasKernel, dim3(static_cast<unsigned>((mn + 255) / 256)), dim3(256), 0,
                     s, Y, bias, mn, N);
  return hipGetLastError();
}

extern "C" {

const char *mnb_version(void) { return "mnb-gfx950 0.1.0"; }

const char *mnb_last_error(void) { return g_last_error; }

const char *mnb_status_str(int status) {
  switch (status) {
  case MNB_OK: return "ok";
  case MNB_ERR_NULL_POINTER: return "null pointer";
  case MNB_ERR_BAD_SHAPE: return "bad shape";
  case MNB_ERR_BAD_ATTRIBUTE: return "bad attribute";
  case MNB_ERR_UNSUPPORTED: return "unsupported";
  case MNB_ERR_WORKSPACE: return "workspace too small";
  case MNB_ERR_HIP: return "HIP runtime error";
  case MNB_ERR_NO_DEVICE: return "no gfx950 device";
  case MNB_ERR_ALLOC: return "device allocation failed";
  default: return "unknown status";
  }
}

int mnb_weight_bytes(const mnb_desc *desc, size_t *bytes) {
  if (bytes == nullptr) return MNB_ERR_NULL_POINTER;
  int st = ValidateDesc(desc);
  if (st != MNB_OK) return st;
  int64_t nb, row_bytes, zp_row_bytes;
  Sizes(desc, &nb, &row_bytes, &zp_row_bytes);
  *bytes = static_cast<size_t>(desc->N) *
           static_cast<size_t>(row_bytes + 4 * nb + (desc->has_zero_points ? zp_row_bytes : 0));
  return MNB_OK;
}

int mnb_plan_create(const mnb_desc *desc, const uint8_t *B, const float *scales,
                    const uint8_t *zero_points, mnb_plan **out_plan) {
  int st = CheckInputs(desc, B, scales, zero_points, out_plan);
  if (st != MNB_OK) return st;
  int dev = -1;
  st = CheckDevice(&dev);
  if (st != MNB_OK) return st;

  mnb_plan *p = new (std::nothrow) mnb_plan();
  if (p == nullptr) return MNB_ERR_ALLOC;
  p->desc = *desc;
  p->device = dev;
  p->owns = true;
  int64_t nb, row_bytes, zp_row_bytes;
  Sizes(desc, &nb, &row_bytes, &zp_row_bytes);
  const size_t b_bytes = static_cast<size_t>(desc->N) * static_cast<size_t>(row_bytes);
  const size_t s_bytes = static_cast<size_t>(desc->N) * static_cast<size_t>(nb) * sizeof(float);
  const size_t z_bytes = static_cast<size_t>(desc->N) * static_cast<size_t>(zp_row_bytes);

  hipError_t e = hipMalloc(reinterpret_cast<void **>(&p->dB), b_bytes);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&p->dS), s_bytes);
  if (e == hipSuccess && desc->has_zero_points)
    e = hipMalloc(reinterpret_cast<void **>(&p->dZ), z_bytes);
  if (e != hipSuccess) {
    SetLastError("hipMalloc", e);
    FreePlanMemory(p);
    delete p;
    return MNB_ERR_ALLOC;
  }
  e = hipMemcpy(p->dB, B, b_bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(p->dS, scales, s_bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess && desc->has_zero_points)
    e = hipMemcpy(p->dZ, zero_points, z_bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    SetLastError("hipMemcpy", e);
    FreePlanMemory(p);
    delete p;
    return MNB_ERR_HIP;
  }
  st = DerivePlanConstants(p);
  if (st != MNB_OK) {
    FreePlanMemory(p);
    delete p;
    return st;
  }
  *out_plan = p;
  return MNB_OK;
}

int mnb_plan_create_device(const mnb_desc *desc, const uint8_t *dB, const float *dScales,
                           const uint8_t *dZeroPoints, mnb_plan **out_plan) {
  int st = CheckInputs(desc, dB, dScales, dZeroPoints, out_plan);
  if (st != MNB_OK) return st;
  if ((reinterpret_cast<uintptr_t>(dScales) % 4) != 0) return MNB_ERR_BAD_SHAPE;
  int dev = -1;
  st = CheckDevice(&dev);
  if (st != MNB_OK) return st;
  mnb_plan *p = new (std::nothrow) mnb_plan();
  if (p == nullptr) return MNB_ERR_ALLOC;
  p->desc = *desc;
  p->device = dev;
  p->owns = false;
  p->dB = const_cast<uint8_t *>(dB);
  p->dS = const_cast<float *>(dScales);
  p->dZ = const_cast<uint8_t *>(dZeroPoints);
  // The derived copies are made once, on the null stream, which does not wait
  // for non-blocking streams: every write to the borrowed buffers already
  // issued on any stream of the device must land first.
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    SetLastError("hipDeviceSynchronize", e);
    delete p;
    return MNB_ERR_HIP;
  }
  st = DerivePlanConstants(p);
  if (st != MNB_OK) {
    FreePlanMemory(p);
    delete p;
    return st;
  }
  *out_plan = p;
  return MNB_OK;
}

int mnb_plan_create_gate_up(const mnb_desc *desc, const uint8_t *Bg, const float *Sg,
                            const uint8_t *Zg, const uint8_t *Bu, const float *Su,
                            const uint8_t *Zu, mnb_plan **out_plan) {
  int st = CheckInputs(desc, Bg, Sg, Zg, out_plan);
  if (st != MNB_OK) return st;
  st = CheckInputs(desc, Bu, Su, Zu, out_plan);
  if (st != MNB_OK) return st;
  if (desc->N > (int64_t{1} << 29)) return MNB_ERR_BAD_SHAPE;
  // Rows interleaved once, on the host: row 2n = gate row n, 2n + 1 = up row n.
  mnb_desc d2 = *desc;
  d2.N = 2 * desc->N;
  int64_t nb, row_bytes, zp_row_bytes;
  Sizes(desc, &nb, &row_bytes, &zp_row_bytes);
  const size_t I = static_cast<size_t>(desc->N);
  std::vector<uint8_t> b2, z2;
  std::vector<float> s2;
  try {
    b2.resize(2 * I * row_bytes);
    s2.resize(2 * I * nb);
    if (desc->has_zero_points) z2.resize(2 * I * zp_row_bytes);
  } catch (const std::bad_alloc &) {
    return MNB_ERR_ALLOC;
  }
  for (size_t n = 0; n < I; ++n) {
    std::memcpy(&b2[(2 * n) * row_bytes], Bg + n * row_bytes, row_bytes);
    std::memcpy(&b2[(2 * n + 1) * row_bytes], Bu + n * row_bytes, row_bytes);
    std::memcpy(&s2[(2 * n) * nb], Sg + n * nb, nb * sizeof(float));
    std::memcpy(&s2[(2 * n + 1) * nb], Su + n * nb, nb * sizeof(float));
    if (desc->has_zero_points) {
      std::memcpy(&z2[(2 * n) * zp_row_bytes], Zg + n * zp_row_bytes, zp_row_bytes);
      std::memcpy(&z2[(2 * n + 1) * zp_row_bytes], Zu + n * zp_row_bytes, zp_row_bytes);
    }
  }
  mnb_plan *p = nullptr;
  st = mnb_plan_create(&d2, b2.data(), s2.data(), desc->has_zero_points ? z2.data() : nullptr, &p);
  if (st != MNB_OK) return st;
  p->gate_up = true;
  *out_plan = p;
  return MNB_OK;
}

int mnb_plan_destroy(mnb_plan *plan) {
  if (plan == nullptr) return MNB_OK;
  FreePlanMemory(plan);
  delete plan;
  return MNB_OK;
}

int mnb_plan_device_bytes(const mnb_plan *plan, size_t *bytes) {
  if (plan == nullptr || bytes == nullptr) return MNB_ERR_NULL_POINTER;
  int64_t nb, row_bytes, zp_row_bytes;
  Sizes(&plan->desc, &nb, &row_bytes, &zp_row_bytes);
  const size_t N = static_cast<size_t>(plan->desc.N);
  size_t total = N * sizeof(int32_t);  // the per-row scale exponents
  if (plan->owns && plan->dB != nullptr)
    total += N * static_cast<size_t>(row_bytes) + N * static_cast<size_t>(nb) * sizeof(float) +
             (plan->dZ != nullptr ? N * static_cast<size_t>(zp_row_bytes) : 0);
  if (plan->dBp != nullptr) {
    size_t sp = 0;
    total += mnb::PrefillLayoutBytes(plan->view, &sp) + sp;
  }
  if (plan->dSd != nullptr) {
    size_t zd = 0;
    total += mnb::DecodeFragScaleBytes(plan->view, &zd) + (plan->dZd != nullptr ? zd : 0);
  }
  *bytes = total;
  return MNB_OK;
}

// Rows from which the decode path multiplies on the original-layout MFMA
// kernel (GemvMfmaKernel), for plans without the fragment-ordered weight copy
// (N % 4 != 0 or N >= 2^22; when the caller passes the workspace): below it
// the fp32-FMA kernels are faster, their cost
// growing by about one M = 1 pass per token while the MFMA kernel's barely
// changes with M. Where the MFMA kernel starts ahead depends on the shape: it
// splits K into 512-k ranges, so wide, short weights (N large against K) give
// it more rows per range and fewer partial sums. Measured on MI355X (FMA
// against MFMA with its partial-sum pass, c1-c5 shapes, M = 2..5): at M = 4
// it wins for N >= 3K (c2 16.8 against 19.7 us, c5 gate+up 25.6 against
// 32.2) and loses below (c1, c3, c5 qkv, o, down by 20-40%); at M = 3 it wins
// for N >= 6K (gate+up 25.1 against 27.0), ties at c2; from M = 5 it is
// ahead or within 5% everywhere.
static int64_t MfmaDecodeMinRows(const mnb::WeightView &w) {
  if (w.N >= 6 * w.K) return 3;
  if (w.N >= 3 * w.K) return 4;
  return 5;
}

static bool UsesMfmaDecode(const mnb_plan *plan, int64_t M) {
  return M >= MfmaDecodeMinRows(plan->view) && M <= 16 && mnb::GemvMfmaSupports(plan->view, M);
}

// Rows from which plans holding the fragment-ordered weights (and their
// decode scales) take DecodeFragKernel, when the caller passes its
// workspace; the fp32-FMA kernels serve fewer. DecodeFragKernel's cost barely
// changes with M (its pre-pass and, for long K, its partial-sum pass add a
// fixed few us), the FMA kernel's grows by about one M = 1 pass per token, so
// the larger the weights the earlier the crossover. Measured on MI355X
// (HIP-graph replay, us, FMA against DecodeFragKernel with both terms of up
// to 8 tokens in one operand): M = 2 c1 5.3 / 8.7, c3 12.8 / 14.3, c5 qkv
// 7.4 / 9.9, o 5.3 / 8.7, down 11.0 / 13.0; M = 3 c1 6.4 / 8.9, c3 15.9 /
// 14.8, qkv 9.1 / 10.0, o 6.4 / 8.7, down 14.4 / 13.3; M = 4 c1 7.2 / 8.9,
// c3 18.4 / 14.7, qkv 10.6 / 9.9, o 7.2 / 8.8, down 17.0 / 13.3. Wide
// weights (N >= 3K) take the fragment-ordered GEMV up to 4 rows when their
// groups cover the CUs; the thresholds by N / K serve the others (before the
// one-operand split: M = 2 c2 13.4 / 14.4, c5 gate+up 23.3 / 22.7; M = 4 c2
// 20.2 / 13.6, gate+up 32.5 / 22.3).
static int64_t FragDecodeMinRows(const mnb::WeightView &w) {
  const int64_t kn = w.K * w.N;
  if (w.N >= 6 * w.K) return 2;
  if (w.N >= 3 * w.K || kn >= (int64_t{48} << 20)) return 3;  // c3, c5 down: 58.7 M
  if (kn >= (int64_t{20} << 20)) return 4;                     // c5 qkv: 25.2 M
  return 5;                                                    // c1, c5 o: 16.8 M
}

static bool UsesFragDecode(const mnb_plan *plan, int64_t M) {
  return M >= FragDecodeMinRows(plan->view) && mnb::DecodeFragSupports(plan->view, M);
}

// The K-segmented fragment-ordered GEMV (1 or 2 rows too long for one
// workgroup, 2 to 4 long rows on narrow weights): plain plans (its sums pass has no gate/up pairing), no RMSNorm
// input (a segment sees only its part of each row's sum of squares).
static bool UsesFragSegments(const mnb_plan *plan, int64_t M, bool rms) {
  return !rms && !plan->gate_up && mnb::GemvFragSegSupports(plan->view, M);
}

// The decode kernel path 1 launches for M rows with `work_bytes` of workspace
// at `work` (M <= 16).
// kDecFragGroups: a compact plan without the small-M kernel's workspace runs
// the fragment-ordered GEMV on consecutive groups of up to 4 rows.
// kDecGemvFragSeg: the fragment-ordered GEMV with K split into segments, for
// 1 or 2 rows too long for one workgroup (and for GemvM1Kernel), and 2 to 4
// rows of K >= 5120 on weights up to 192 Mi elements (2 rows from 48 Mi).
enum DecodeKernel {
  kDecM1, kDecGemvFrag, kDecFrag, kDecMfma, kDecSmallM, kDecGemv, kDecFragGroups, kDecGemvFragSeg
};

// Rows per launch of the exact route (path 4): the decode kernels' limit.
constexpr int64_t kExactGroupRows = 16;

static bool HasWorkspace(const void *work, size_t bytes, size_t need) {
  return need == 0 ||
         (work != nullptr && bytes >= need && (reinterpret_cast<uintptr_t>(work) % 16) == 0);
}

// Without the kernel's workspace, M >= 2 falls back to the fp32-FMA kernels.
// M <= 4 takes the LDS-staged MFMA kernel on the fragment-ordered copy where
// its 64-row groups cover most CUs (a fused RMSNorm input at M = 1 too); M = 1
// otherwise GemvM1Kernel. Rows too long for both (K > 16384 at M = 1, K >
// 8192 at M = 2) take that MFMA kernel with K segments when the workspace
// holds their partial sums (plain plans, no RMSNorm input), and so do 2 to 4
// rows of K >= 5120 on narrow weights (2 rows from 48 Mi elements), ahead of
// the small-M MFMA decode and the fp32-FMA GEMV, and wide weights whose
// single-workgroup launch would leave a second round on a few CUs. Wide
// weights with rows too long for one workgroup take the segments ahead of
// GemvM1Kernel (K = 11008, N = 17408: 22.9 against 29.5 us; K = 13824,
// N = 20480 31.8 against 38.4; K = 8960, N = 14336 16.4 against 19.4);
// narrower ones keep it (K = 11008, N = 4096 and K = 13824, N = 5120).
static DecodeKernel PickDecodeKernel(const mnb_plan *plan, int64_t M, const void *work,
                                     size_t work_bytes, bool rms = false) {
  const bool segs = UsesFragSegments(plan, M, rms) &&
                    HasWorkspace(work, work_bytes, mnb::GemvFragSegWorkspaceBytes(plan->view, M));
  if (mnb::GemvFragPreferred(plan->view, M, rms)) return segs ? kDecGemvFragSeg : kDecGemvFrag;
  if (segs && mnb::GemvFragWide(plan->view)) return kDecGemvFragSeg;
  if (M == 1 && mnb::GemvM1Supports(plan->view)) return kDecM1;
  if (segs) return kDecGemvFragSeg;
  if (UsesFragDecode(plan, M) &&
      HasWorkspace(work, work_bytes, mnb::DecodeFragWorkspaceBytes(plan->view, M)))
    return kDecFrag;
  if (!mnb::DecodeFragSupports(plan->view, M) && UsesMfmaDecode(plan, M) &&
      HasWorkspace(work, work_bytes, mnb::GemvMfmaWorkspaceBytes(plan->view, M)))
    return kDecMfma;
  if (plan->view.B == nullptr) return kDecFragGroups;
  return mnb::GemvSmallMSupports(plan->view, M) ? kDecSmallM : kDecGemv;
}

// Whether the decode path (path 1) serves M <= 16 rows: the original-layout
// kernels, or on a compact plan the fragment-ordered GEMV (groups of 4 rows).
static bool DecodeSupported(const mnb_plan *plan, int64_t M) {
  if (M < 1 || M > 16) return false;
  return plan->view.B != nullptr ? mnb::GemvSupports(plan->view, M)
                                 : mnb::GemvFragSupports(plan->view, std::min<int64_t>(M, 4));
}

// Decode kernels that multiply a fused RMSNorm input themselves.
static bool DecodeTakesRms(const mnb_plan *plan, DecodeKernel k) {
  return k == kDecGemvFrag || k == kDecM1 || (k == kDecFrag && mnb::DecodeFragTakesRms(plan->view));
}

// Workspace bytes the decode kernel PickDecodeKernel chooses for M rows when
// the caller passes enough: 0 for the kernels that need none.
static size_t DecodeNeed(const mnb_plan *plan, int64_t M, bool rms = false) {
  const bool segs = UsesFragSegments(plan, M, rms);
  if (mnb::GemvFragPreferred(plan->view, M, rms))
    return segs ? mnb::GemvFragSegWorkspaceBytes(plan->view, M) : 0;
  if (segs && mnb::GemvFragWide(plan->view)) return mnb::GemvFragSegWorkspaceBytes(plan->view, M);
  if (M == 1 && mnb::GemvM1Supports(plan->view)) return 0;
  if (segs) return mnb::GemvFragSegWorkspaceBytes(plan->view, M);
  if (UsesFragDecode(plan, M)) return mnb::DecodeFragWorkspaceBytes(plan->view, M);
  if (!mnb::DecodeFragSupports(plan->view, M) && UsesMfmaDecode(plan, M))
    return mnb::GemvMfmaWorkspaceBytes(plan->view, M);
  return 0;
}

// Whether a gate/up plan's run of M rows on `path` applies the activation in
// the fragment-ordered GEMV's epilogue and so needs no scratch sum.
static bool GateUpFusedInGemv(const mnb_plan *plan, int64_t M, int path, bool rms = false) {
  return plan->gate_up && path == 1 && mnb::GemvFragPreferred(plan->view, M, rms);
}


int mnb_workspace_bytes(const mnb_plan *plan, int64_t M, size_t *bytes) {
  if (plan == nullptr || bytes == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 0 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  // The size covers every path mnb_run_path may be asked to take for M rows:
  // the prefill GEMM (A rounded to fp16, tile layout, split-K partial sums)
  // and the MFMA decode kernel (split-K partial sums).
  // A gate/up plan adds the scratch sum in front of either.
  // The exact route (path 4) runs the decode kernels over groups of at most
  // 16 rows, one after another in the same workspace.
  // Decode launches served by the fragment-ordered GEMV need none. The
  // decode kernel of a fused RMSNorm input (mnb_run_rmsnorm passes this
  // size on) may differ from the plain one: the size covers both.
  size_t need = 0;
  if (M > 0 && mnb::GemmSupports(plan->view, M)) need = mnb::GemmWorkspaceBytes(plan->view, M);
  const int64_t md = std::min<int64_t>(M, kExactGroupRows);
  if (md > 0) need = std::max({need, DecodeNeed(plan, md), DecodeNeed(plan, md, true)});
  *bytes = need + GateUpScratchBytes(plan, M);
  return MNB_OK;
}


// accuracy_level is ONNX Runtime's MatMulNBits attribute: the lowest accuracy
// at which A may enter the computation (0 unset, 1 fp32, 2 fp16, 3 bf16,
// 4 int8). Level 1 asks for fp32 activations, so its rows never take the
// fp16 GEMM: above 16 rows they go through the exact-product decode kernels,
// 16 rows at a time (path 4). Levels 0 (unset: the library's default), 2, 3
// and 4 take the fp16 GEMM above 16 rows, whose activations keep an 11-bit
// significand with per-row range scaling: at least the accuracy levels 2-4
// permit. Every level runs the exact decode kernels up to 16 rows.
static bool Fp32ActivationsOnly(const mnb_plan *plan) { return plan->desc.accuracy_level == 1; }

static bool ExactGroupsSupported(const mnb_plan *plan, bool a_aligned) {
  return a_aligned && DecodeSupported(plan, kExactGroupRows);
}

static int SelectPath(const mnb_plan *plan, int64_t M, const float *dA) {
  const bool a_aligned = (reinterpret_cast<uintptr_t>(dA) % 16) == 0;
  if (a_aligned && DecodeSupported(plan, M)) return 1;
  if (Fp32ActivationsOnly(plan)) return ExactGroupsSupported(plan, a_aligned) ? 4 : 3;
  if (a_aligned && mnb::GemmSupports(plan->view, M)) return 2;
  // Rows the GEMM kernels cannot take (K an odd multiple of 32): the decode
  // kernels 16 rows at a time rather than one wavefront per output.
  return ExactGroupsSupported(plan, a_aligned) ? 4 : 3;
}

// Workspace the automatic path (mnb_run) takes for M rows of dA: the chosen
// kernel's own, plus a gate/up plan's scratch sum where its epilogue does not
// apply the activation (the exact route: per group of 16 rows).
static size_t AutoWorkspaceBytes(const mnb_plan *plan, int64_t M, const float *dA) {
  const int path = SelectPath(plan, M, dA);
  switch (path) {
  case 1:
    return DecodeNeed(plan, M) + (GateUpFusedInGemv(plan, M, 1) ? 0 : GateUpScratchBytes(plan, M));
  case 2: return mnb::GemmWorkspaceBytes(plan->view, M) + GateUpScratchBytes(plan, M);
  case 4: {
    const int64_t md = std::min<int64_t>(M, kExactGroupRows);
    return DecodeNeed(plan, md) + GateUpScratchBytes(plan, md);
  }
  default: return GateUpScratchBytes(plan, M);
  }
}

int mnb_select_path(const mnb_plan *plan, int64_t M, int *path) {
  if (plan == nullptr || path == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 0) return MNB_ERR_BAD_SHAPE;
  // Paths are chosen for a 16-byte-aligned activation buffer, as hipMalloc returns.
  *path = SelectPath(plan, M, nullptr);
  return MNB_OK;
}

// One run of the plan. With gamma, dA is the un-normalized input of a fused
// RMSNorm: only the M = 1 GEMV and the GEMM take it (each reduces the rows
// itself); mnb_run_rmsnorm normalizes the input for the rest.
static int RunImpl(const mnb_plan *plan, int64_t M, const float *dA, const float *dBias, float *dY,
                   void *dWorkspace, size_t workspace_bytes, void *stream, int path,
                   const float *gamma, float eps) {
  if (plan == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 0 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  if (M == 0) return MNB_OK;
  if (dA == nullptr || dY == nullptr) return MNB_ERR_NULL_POINTER;
  if (path < 0 || path > 5) return MNB_ERR_UNSUPPORTED;
  const bool a_aligned = (reinterpret_cast<uintptr_t>(dA) % 16) == 0;
  if (path == 0) path = SelectPath(plan, M, dA);
  if (path == 1 && !(a_aligned && DecodeSupported(plan, M))) return MNB_ERR_UNSUPPORTED;
  if (path == 2 && !(a_aligned && mnb::GemmSupports(plan->view, M))) return MNB_ERR_UNSUPPORTED;
  if (path == 4 && !ExactGroupsSupported(plan, a_aligned)) return MNB_ERR_UNSUPPORTED;
  if (path == 5 && !(a_aligned && mnb::PrefillSupports(plan->view, M))) return MNB_ERR_UNSUPPORTED;
  if (plan->gate_up && dBias != nullptr) return MNB_ERR_UNSUPPORTED;
  if (path == 4) {
    // The decode kernels over consecutive groups of rows, in stream order on
    // the one workspace (each group's launches finish reading it before the
    // next group's start writing it).
    const int64_t K = plan->view.K, cols = plan->gate_up ? plan->view.N / 2 : plan->view.N;
    for (int64_t m0 = 0; m0 < M; m0 += kExactGroupRows) {
      const int64_t mg = std::min(kExactGroupRows, M - m0);
      const int st = RunImpl(plan, mg, dA + m0 * K, dBias, dY + m0 * cols, dWorkspace,
                             workspace_bytes, stream, 1, nullptr, 0.0f);
      if (st != MNB_OK) return st;
    }
    return MNB_OK;
  }
  // A gate/up plan's runs start with the scratch sum; the path's own
  // workspace follows it.
  const size_t scratch =
      GateUpFusedInGemv(plan, M, path, gamma != nullptr) ? 0 : GateUpScratchBytes(plan, M);
  if (scratch > 0 && (dWorkspace == nullptr || workspace_bytes < scratch ||
                      (reinterpret_cast<uintptr_t>(dWorkspace) % 16) != 0))
    return MNB_ERR_WORKSPACE;
  float *Ys = scratch > 0 ? static_cast<float *>(dWorkspace) : dY;
  float *H = plan->gate_up ? dY : nullptr;
  void *work = scratch > 0 ? static_cast<void *>(static_cast<char *>(dWorkspace) + scratch)
                           : dWorkspace;
  const size_t work_bytes = scratch > 0 ? workspace_bytes - scratch : workspace_bytes;
  if (path == 2 || path == 5) {
    const size_t need = mnb::GemmWorkspaceBytes(plan->view, M);
    if (work == nullptr || work_bytes < need || (reinterpret_cast<uintptr_t>(work) % 16) != 0)
      return MNB_ERR_WORKSPACE;
  }

  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess || cur != plan->device) {
    std::snprintf(g_last_error, sizeof(g_last_error), "plan lives on device %d, current is %d",
                  plan->device, cur);
    return MNB_ERR_NO_DEVICE;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Kernels with the gate/up epilogue take H and write it themselves; after
  // the others, SiluMulKernel turns the scratch sum into H.
  bool fused = false, bias_done = false;
  switch (path) {
  case 1: {
    const DecodeKernel dk = PickDecodeKernel(plan, M, work, work_bytes, gamma != nullptr);
    // only these kernels take an RMSNorm input (mnb_run_rmsnorm checks first)
    if (gamma != nullptr && !DecodeTakesRms(plan, dk)) return MNB_ERR_UNSUPPORTED;
    switch (dk) {
    case kDecGemvFrag:
      e = mnb::LaunchGemvFrag(plan->view, M, dA, Ys, s, 0, 0, H, dBias, gamma, eps);
      fused = true;
      bias_done = dBias != nullptr;
      break;
    case kDecM1:
      e = mnb::LaunchGemvM1(plan->view, dA, Ys, s, 0, 0, H, gamma, eps, dBias);
      fused = true;
      bias_done = dBias != nullptr;
      if (e == hipErrorInvalidValue && H != nullptr) {
        // no shape with paired rows for this plan: plain launch, then the pass
        e = mnb::LaunchGemvM1(plan->view, dA, Ys, s, 0, 0, nullptr, gamma, eps);
        fused = false;
      }
      break;
    case kDecFrag:
      e = mnb::LaunchDecodeFrag(plan->view, M, dA, Ys, work, s, H, 0, 0, dBias, gamma, eps);
      fused = true;
      bias_done = dBias != nullptr;
      break;
    case kDecMfma:
      e = mnb::LaunchGemvMfma(plan->view, M, dA, Ys, work, s, H);
      fused = true;
      break;
    case kDecGemvFragSeg:
      e = mnb::LaunchGemvFragSeg(plan->view, M, dA, Ys, work, s, dBias);
      bias_done = dBias != nullptr;
      break;
    case kDecSmallM: e = mnb::LaunchGemvSmallM(plan->view, M, dA, Ys, s); break;
    case kDecFragGroups: {
      // consecutive groups of up to 4 rows, in stream order
      const int64_t K = plan->view.K, N = plan->view.N;
      for (int64_t m0 = 0; m0 < M && e == hipSuccess; m0 += 4) {
        const int64_t mg = std::min<int64_t>(4, M - m0);
        e = mnb::LaunchGemvFrag(plan->view, mg, dA + m0 * K, Ys + m0 * N, s, 0, 0,
                                H != nullptr ? H + m0 * (N / 2) : nullptr, dBias);
      }
      fused = true;
      bias_done = dBias != nullptr;
      break;
    }
    default: e = mnb::LaunchGemv(plan->view, M, dA, Ys, s); break;
    }
    break;
  }
  case 2:
    // The GEMM's fused stores address H with 32-bit byte offsets: H's bytes
    // and those of a whole tile of rows (up to 128) must stay below 2^31.
    fused = H != nullptr && M * plan->view.N * 2 < (int64_t{1} << 31) &&
            plan->view.N < (int64_t{1} << 22);
    e = mnb::LaunchGemm(plan->view, M, dA, Ys, work, s, fused ? H : nullptr, gamma, eps, dBias,
                        &bias_done);
    break;
  case 5:
    fused = H != nullptr && M * plan->view.N * 2 < (int64_t{1} << 31) &&
            plan->view.N < (int64_t{1} << 22);
    e = mnb::LaunchPrefill(plan->view, M, dA, Ys, work, s, fused ? H : nullptr, gamma, eps, dBias,
                           &bias_done);
    break;
  default: e = mnb::LaunchGeneric(plan->view, M, dA, Ys, s); break;
  }
  if (e == hipSuccess && H != nullptr && !fused) e = mnb::LaunchSiluMul(Ys, H, M, plan->view.N, s);
  if (e == hipSuccess && dBias != nullptr && !bias_done)
    e = LaunchAddBias(dY, dBias, M, plan->view.N, s);
  if (e != hipSuccess) {
    SetLastError("kernel launch", e);
    return MNB_ERR_HIP;
  }
  return MNB_OK;
}

int mnb_run_ex(const mnb_plan *plan, int64_t M, const float *dA, const float *dBias, float *dY,
               void *dWorkspace, size_t workspace_bytes, void *stream, int path) {
  return RunImpl(plan, M, dA, dBias, dY, dWorkspace, workspace_bytes, stream, path, nullptr, 0.0f);
}

// Workspace of mnb_run_rmsnorm: the normalized input (paths without the
// fused RMSNorm), then mnb_run's workspace.
static size_t RmsFrontBytes(const mnb_plan *plan, int64_t M) {
  return Round256(static_cast<size_t>(M) * plan->view.K * 4);
}

int mnb_rmsnorm_workspace_bytes(const mnb_plan *plan, int64_t M, size_t *bytes) {
  if (plan == nullptr || bytes == nullptr) return MNB_ERR_NULL_POINTER;
  size_t rest = 0;
  const int st = mnb_workspace_bytes(plan, M, &rest);
  if (st != MNB_OK) return st;
  *bytes = RmsFrontBytes(plan, M) + rest;
  return MNB_OK;
}

int mnb_run_rmsnorm(const mnb_plan *plan, int64_t M, const float *dX, const float *dGamma,
                    float epsilon, float *dY, void *dWorkspace, size_t workspace_bytes,
                    void *stream) {
  if (plan == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 0 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  if (M == 0) return MNB_OK;
  if (dX == nullptr || dGamma == nullptr || dY == nullptr) return MNB_ERR_NULL_POINTER;
  if (!(epsilon >= 0.0f) || !std::isfinite(epsilon)) return MNB_ERR_BAD_ATTRIBUTE;
  if ((plan->view.K % 4) != 0 || (reinterpret_cast<uintptr_t>(dX) % 16) != 0 ||
      (reinterpret_cast<uintptr_t>(dGamma) % 16) != 0)
    return MNB_ERR_UNSUPPORTED;
  const size_t front = RmsFrontBytes(plan, M);
  if (dWorkspace == nullptr || workspace_bytes < front ||
      (reinterpret_cast<uintptr_t>(dWorkspace) % 16) != 0)
    return MNB_ERR_WORKSPACE;
  float *Xn = static_cast<float *>(dWorkspace);
  void *rest = static_cast<char *>(dWorkspace) + front;
  const size_t rest_bytes = workspace_bytes - front;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != plan->device) return MNB_ERR_NO_DEVICE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int path = SelectPath(plan, M, dX);
  // Fused where the kernel multiplies the normalized input itself: the GEMM,
  // and the decode kernels that take gamma (the M = 1 GEMV, the M <= 4
  // fragment GEMV, the small-M MFMA decode with its workspace).
  if (path == 2 ||
      (path == 1 && DecodeTakesRms(plan, PickDecodeKernel(plan, M, rest, rest_bytes, true))))
    return RunImpl(plan, M, dX, nullptr, dY, rest, rest_bytes, stream, path, dGamma, epsilon);
  const hipError_t e = mnb::LaunchRmsNorm(dX, dGamma, Xn, M, plan->view.K, epsilon, s);
  if (e != hipSuccess) {
    SetLastError("kernel launch", e);
    return MNB_ERR_HIP;
  }
  return RunImpl(plan, M, Xn, nullptr, dY, rest, rest_bytes, stream, path, nullptr, 0.0f);
}

int mnb_run_path(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
                 size_t workspace_bytes, void *stream, int path) {
  return mnb_run_ex(plan, M, dA, nullptr, dY, dWorkspace, workspace_bytes, stream, path);
}

int mnb_run(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
            size_t workspace_bytes, void *stream) {
  return mnb_run_ex(plan, M, dA, nullptr, dY, dWorkspace, workspace_bytes, stream, 0);
}

const char *mnb_kernel_name(const mnb_plan *plan, int64_t M, size_t workspace_bytes) {
  if (plan == nullptr || M <= 0 || M > (int64_t{1} << 30)) return "";
  // The workspace's address only matters through its alignment here.
  const void *work = workspace_bytes > 0 ? reinterpret_cast<const void *>(uintptr_t{256}) : nullptr;
  size_t work_bytes = workspace_bytes;
  const size_t scratch = GateUpScratchBytes(plan, M);
  if (scratch > 0) {
    if (workspace_bytes < scratch) return "";
    work_bytes -= scratch;
  }
  switch (SelectPath(plan, M, reinterpret_cast<const float *>(uintptr_t{256}))) {
  case 1:
    switch (PickDecodeKernel(plan, M, work, work_bytes)) {
    case kDecM1: return "GemvM1Kernel";
    case kDecGemvFrag: return "GemvFragKernel";
    case kDecFrag: return "DecodeFragKernel";
    case kDecMfma: return "GemvMfmaKernel";
    case kDecSmallM: return "GemvSmallMKernel";
    case kDecFragGroups: return "GemvFragKernel";
    case kDecGemvFragSeg: return "GemvFragKernel (K segments)";
    default: return "GemvKernel";
    }
  case 2:
    return mnb::GemmUsesStream(plan->view, M)    ? "StreamKernel"
           : mnb::GemmUsesPrefill(plan->view, M) ? "PrefillKernel"
                                                 : "GemmKernel";
  case 4: return "exact groups of 16 rows";
  default: return "GenericKernel";
  }
}

// Whether `kernel` can serve M rows of the plan's weights (A's alignment is
// checked by the caller that has it).
static bool KernelServes(const mnb::WeightView &w, int64_t M, int kernel) {
  switch (kernel) {
  case MNB_KERNEL_GEMV_M1: return M == 1 && mnb::GemvM1Supports(w);
  case MNB_KERNEL_GEMV_FRAG: return mnb::GemvFragSupports(w, M);
  case MNB_KERNEL_GEMV_SMALL_M: return M >= 2 && mnb::GemvSmallMSupports(w, M);
  case MNB_KERNEL_GEMV_MFMA: return mnb::GemvMfmaSupports(w, M);
  case MNB_KERNEL_DECODE_FRAG: return mnb::DecodeFragSupports(w, M);
  case MNB_KERNEL_GEMM: return mnb::GemmKernelSupports(w, M);
  case MNB_KERNEL_PREFILL: return mnb::PrefillSupports(w, M);
  case MNB_KERNEL_STREAM: return mnb::StreamSupports(w, M);
  case MNB_KERNEL_GEMV: return M <= 16 && mnb::GemvSupports(w, M);
  case MNB_KERNEL_GENERIC: return true;
  default: return false;
  }
}

int mnb_kernel_workspace_bytes(const mnb_plan *plan, int64_t M, int kernel, int p0, int p1,
                               size_t *bytes) {
  if (plan == nullptr || bytes == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 1 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  const mnb::WeightView &w = plan->view;
  if (plan->gate_up || !KernelServes(w, M, kernel)) return MNB_ERR_UNSUPPORTED;
  switch (kernel) {
  case MNB_KERNEL_GEMV_MFMA:
    *bytes = mnb::GemvMfmaWorkspaceBytes(w, M);
    return MNB_OK;
  case MNB_KERNEL_DECODE_FRAG:
    *bytes = mnb::DecodeFragWorkspaceBytes(w, M, p0, p1);
    return MNB_OK;
  case MNB_KERNEL_GEMM:
    *bytes = p0 > 0 ? mnb::GemmShapeWorkspaceBytes(w, M, std::max(1, p1))
                    : mnb::GemmWorkspaceBytes(w, M);
    return MNB_OK;
  case MNB_KERNEL_PREFILL:
    *bytes = mnb::GemmShapeWorkspaceBytes(w, M, std::max(1, p0));
    if (p0 <= 0) *bytes = std::max(*bytes, mnb::GemmWorkspaceBytes(w, M));
    return MNB_OK;
  case MNB_KERNEL_STREAM:
    if (!mnb::StreamShapeOk(w, M, p0, p1)) return MNB_ERR_UNSUPPORTED;
    *bytes = mnb::StreamWorkspaceBytes(w, M, p0, p1);
    return MNB_OK;
  case MNB_KERNEL_GEMV_M1:
  case MNB_KERNEL_GEMV_FRAG:
  case MNB_KERNEL_GEMV_SMALL_M:
  case MNB_KERNEL_GEMV:
  case MNB_KERNEL_GENERIC:
    *bytes = 0;
    return MNB_OK;
  default: return MNB_ERR_UNSUPPORTED;
  }
}

int mnb_run_kernel(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *dWorkspace,
                   size_t workspace_bytes, void *stream, int kernel, int p0, int p1) {
  if (plan == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 1 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  if (dA == nullptr || dY == nullptr) return MNB_ERR_NULL_POINTER;
  if (plan->gate_up || p0 < 0 || p1 < 0) return MNB_ERR_UNSUPPORTED;
  auto one_of = [](int v, std::initializer_list<int> ok) {
    return std::find(ok.begin(), ok.end(), v) != ok.end();
  };
  bool shape_ok = true;
  switch (kernel) {
  case MNB_KERNEL_GEMV_M1: shape_ok = p0 <= 1024 && one_of(p1, {0, 1, 2, 4, 8}); break;
  case MNB_KERNEL_GEMV_SMALL_M: shape_ok = p0 <= 8 && one_of(p1, {0, 4, 8}); break;
  case MNB_KERNEL_GEMV_MFMA: shape_ok = p0 <= 2 && p1 <= 8; break;
  case MNB_KERNEL_DECODE_FRAG: shape_ok = p0 <= 8 && p1 <= 2; break;
  case MNB_KERNEL_GEMM: shape_ok = one_of(p0, {0, 32, 64, 128}) && p1 <= 16; break;
  case MNB_KERNEL_PREFILL: shape_ok = p0 <= 16 && p1 == 0; break;
  case MNB_KERNEL_STREAM: shape_ok = p0 <= 16 && one_of(p1, {0, 4, 8, 16}) && (p0 == 0) == (p1 == 0); break;
  case MNB_KERNEL_GEMV_FRAG: shape_ok = mnb::GemvFragShapeOk(plan->view, M, p0, p1); break;
  default: shape_ok = p0 == 0 && p1 == 0; break;
  }
  if (!shape_ok) return MNB_ERR_UNSUPPORTED;
  size_t need = 0;
  int st = mnb_kernel_workspace_bytes(plan, M, kernel, p0, p1, &need);
  if (st != MNB_OK) return st;
  if (!HasWorkspace(dWorkspace, workspace_bytes, need)) return MNB_ERR_WORKSPACE;
  const mnb::WeightView &w = plan->view;
  const bool a_aligned = (reinterpret_cast<uintptr_t>(dA) % 16) == 0;
  if (!a_aligned && kernel != MNB_KERNEL_GENERIC) return MNB_ERR_UNSUPPORTED;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != plan->device) return MNB_ERR_NO_DEVICE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  switch (kernel) {
  case MNB_KERNEL_GEMV_M1: e = mnb::LaunchGemvM1(w, dA, dY, s, p0, p1); break;
  case MNB_KERNEL_GEMV_FRAG: e = mnb::LaunchGemvFrag(w, M, dA, dY, s, p0, p1, nullptr, nullptr); break;
  case MNB_KERNEL_GEMV_SMALL_M: e = mnb::LaunchGemvSmallMShape(w, M, dA, dY, s, p0, p1, 0); break;
  case MNB_KERNEL_GEMV_MFMA: e = mnb::LaunchGemvMfmaShape(w, M, dA, dY, dWorkspace, s, p0, p1); break;
  case MNB_KERNEL_DECODE_FRAG: e = mnb::LaunchDecodeFrag(w, M, dA, dY, dWorkspace, s, nullptr, p0, p1); break;
  case MNB_KERNEL_GEMM: e = mnb::LaunchGemmShape(w, M, dA, dY, dWorkspace, s, p0, std::max(1, p1)); break;
  case MNB_KERNEL_PREFILL:
    e = p0 > 0 ? mnb::LaunchGemmShape(w, M, dA, dY, dWorkspace, s, mnb::kPrefillTileCode, p0)
               : mnb::LaunchPrefill(w, M, dA, dY, dWorkspace, s);
    break;
  case MNB_KERNEL_STREAM:
    e = mnb::LaunchStream(w, M, dA, dY, dWorkspace, s, nullptr, nullptr, 0.0f, nullptr, p0, p1);
    break;
  case MNB_KERNEL_GEMV: e = mnb::LaunchGemv(w, M, dA, dY, s); break;
  default: e = mnb::LaunchGeneric(w, M, dA, dY, s); break;
  }
  if (e != hipSuccess) {
    SetLastError("kernel launch", e);
    return e == hipErrorInvalidValue ? MNB_ERR_UNSUPPORTED : MNB_ERR_HIP;
  }
  return MNB_OK;
}

int mnb_run_no_alloc(const mnb_plan *plan, int64_t M, const float *dA, float *dY, void *stream) {
  if (plan == nullptr) return MNB_ERR_NULL_POINTER;
  if (M < 0 || M > (int64_t{1} << 30)) return MNB_ERR_BAD_SHAPE;
  if (M == 0) return MNB_OK;
  if (dA == nullptr || dY == nullptr) return MNB_ERR_NULL_POINTER;
  const size_t need = AutoWorkspaceBytes(plan, M, dA);
  int st = MNB_OK;
  if (need > kScratchBytes) {
    std::snprintf(g_last_error, sizeof(g_last_error),
                  "mnb_run_no_alloc: %zu workspace bytes needed for M = %lld, the scratch holds %zu",
                  need, static_cast<long long>(M), kScratchBytes);
    return MNB_ERR_WORKSPACE;
  }
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != plan->device) {
    std::snprintf(g_last_error, sizeof(g_last_error), "plan lives on device %d, current is %d",
                  plan->device, cur);
    return MNB_ERR_NO_DEVICE;
  }
  void *work = nullptr;
  st = ScratchAddress(cur, &work);
  if (st != MNB_OK) return st;
  return mnb_run_ex(plan, M, dA, nullptr, dY, need > 0 ? work : nullptr, need, stream, 0);
}

} // extern "C"
