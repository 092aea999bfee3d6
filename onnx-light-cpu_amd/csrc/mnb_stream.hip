// HBM read ceiling probe: one launch that only streams a buffer, the way the
// fastest streaming pattern of a sweep on MI355X does, folding the bytes into
// one word per wavefront so the loads are kept. The decode kernels' roofline
// fraction is reported next to what this probe reaches over the same number
// of bytes per launch. Sweep (31.5 MB per launch, 35 rotated buffers, graph
// replays): records of 4 / 8 / 16 / 32 KiB per wavefront with all their
// 16-byte loads in flight, 1024 to 8192 wavefronts, 256- to 1024-thread
// workgroups, non-temporal or default loads; the fastest were 8 KiB records
// over 2048 wavefronts in 256-thread workgroups with non-temporal loads
// (6.40-6.49 us), 16 KiB records 6.9 us, default-policy loads 0.4-1.0 us
// slower, 1024-thread workgroups slower still.
#include "../../include/mnb.h"
#include "mnb_kernels.h"

namespace mnb {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRecordBytes = 8192;
constexpr int kLoads = kRecordBytes / 1024;  // 16-byte loads per lane and record

__global__ __launch_bounds__(256) void StreamReadKernel(const uint8_t *__restrict__ src,
                                                        uint32_t *__restrict__ out, int bytes,
                                                        int records) {
  const int lane = threadIdx.x & 63;
  const int w = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  const int waves = static_cast<int>(gridDim.x) * 4;
  // bytes past the end read as zeros (no memory access)
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), 0, bytes, 0x00020000);
  uint32_t x = 0;
  for (int r = w; r < records; r += waves) {
    u32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rs, r * kRecordBytes + 1024 * i + 16 * lane, 0, 2));
#pragma unroll
    for (int i = 0; i < kLoads; ++i) x ^= (v[i][0] ^ v[i][1]) ^ (v[i][2] ^ v[i][3]);
  }
  for (int o = 32; o >= 1; o >>= 1) x ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), o, 64));
  if (lane == 0) out[w] = x;
}

// One contiguous share of `chunk` bytes per wavefront, eight 16-byte loads
// (8 KiB) in flight at a time.
__global__ __launch_bounds__(1024) void StreamChunkKernel(const uint8_t *__restrict__ src,
                                                          uint32_t *__restrict__ out, int bytes,
                                                          int chunk) {
  const int lane = threadIdx.x & 63;
  const int w = static_cast<int>(blockIdx.x) * static_cast<int>(blockDim.x >> 6) +
                static_cast<int>(threadIdx.x >> 6);
  // bytes past the end read as zeros (no memory access)
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), 0, bytes, 0x00020000);
  const int64_t base = static_cast<int64_t>(w) * chunk;
  uint32_t x = 0;
  for (int o = 0; o < chunk; o += kRecordBytes) {
    u32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      // loads past the share (the last group of a share that is not a
      // multiple of 8 KiB) or past the buffer go to offset `bytes`: zeros
      const int64_t off = base + o + 1024 * i + 16 * lane;
      const bool in = o + 1024 * i < chunk && off < bytes;
      v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rs, in ? static_cast<int>(off) : bytes, 0, 2));
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) x ^= (v[i][0] ^ v[i][1]) ^ (v[i][2] ^ v[i][3]);
  }
  for (int o = 32; o >= 1; o >>= 1) x ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), o, 64));
  if (lane == 0) out[w] = x;
}

} // namespace
} // namespace mnb

extern "C" int mnb_stream_read(const void *dSrc, size_t bytes, uint32_t *dOut, size_t out_words,
                               void *stream) {
  if (dSrc == nullptr || dOut == nullptr) return MNB_ERR_NULL_POINTER;
  if (bytes == 0 || bytes >= (size_t{1} << 31) - mnb::kRecordBytes) return MNB_ERR_BAD_SHAPE;
  if (out_words < MNB_STREAM_OUT_WORDS) return MNB_ERR_WORKSPACE;
  const int records = static_cast<int>((bytes + mnb::kRecordBytes - 1) / mnb::kRecordBytes);
  const int wgs = MNB_STREAM_OUT_WORDS / 4;  // 2048 wavefronts
  hipLaunchKernelGGL(mnb::StreamReadKernel, dim3(wgs), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint8_t *>(dSrc),
                     dOut, static_cast<int>(bytes), records);
  return hipGetLastError() == hipSuccess ? MNB_OK : MNB_ERR_HIP;
}

extern "C" int mnb_stream_read_grid(const void *dSrc, size_t bytes, uint32_t *dOut,
                                    size_t out_words, int workgroups, int threads, void *stream) {
  if (dSrc == nullptr || dOut == nullptr) return MNB_ERR_NULL_POINTER;
  if (bytes == 0 || bytes >= (size_t{1} << 31) - mnb::kRecordBytes) return MNB_ERR_BAD_SHAPE;
  if (threads < 64 || threads > 1024 || threads % 64 != 0 || workgroups < 1) return MNB_ERR_BAD_SHAPE;
  const int64_t waves = static_cast<int64_t>(workgroups) * (threads / 64);
  if (waves > 65536) return MNB_ERR_BAD_SHAPE;
  if (out_words < static_cast<size_t>(waves)) return MNB_ERR_WORKSPACE;
  const int64_t share = (static_cast<int64_t>(bytes) + waves - 1) / waves;
  const int chunk = static_cast<int>((share + 1023) / 1024 * 1024);
  hipLaunchKernelGGL(mnb::StreamChunkKernel, dim3(static_cast<unsigned>(workgroups)),
                     dim3(static_cast<unsigned>(threads)), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint8_t *>(dSrc), dOut, static_cast<int>(bytes), chunk);
  return hipGetLastError() == hipSuccess ? MNB_OK : MNB_ERR_HIP;
}
