// C entry points over functions of the onnx-light-cpu reference, compiled
// together with the reference's own source files (see oracle/Makefile) into
// oracle/_ref/libolc_ref.so -- TEST INFRASTRUCTURE ONLY. It exists to pin the
// oracle against the real reference code; the GPU product never loads it.
//
// Wrapped reference functions:
//   IntegerMatMul4Bit2D   onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.h:52-55
//   MatMulPlan<float>     onnx_light_cpu/impl/math/gemm/gemm_plan.h:161-195
//   FloatToFloat16Bits    onnx_light_cpu/impl/math/half_conversion.h:42-78
//   ExecutionExecutorView onnx_light_cpu/impl/execution.h:15-20 (thread injection)
#include "onnx_light_cpu/impl/execution.h"
#include "onnx_light_cpu/impl/math/gemm/gemm_plan.h"
#include "onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.h"
#include "onnx_light_cpu/impl/math/half_conversion.h"

#include <cstdint>
#include <thread>
#include <vector>

namespace {

// A CpuExecutor stand-in: one std::thread per block, the caller runs block 0.
void RunBlocksOnThreads(void * /*context*/, int64_t num_blocks, void *task_context,
                        onnx_light_cpu::ExecutionBlockFn task) {
  std::vector<std::thread> workers;
  workers.reserve(static_cast<size_t>(num_blocks > 0 ? num_blocks - 1 : 0));
  for (int64_t b = 1; b < num_blocks; ++b) workers.emplace_back(task, task_context, b);
  if (num_blocks > 0) task(task_context, 0);
  for (auto &w : workers) w.join();
}

} // namespace

extern "C" {

void olcref_int4_matmul(const uint8_t *a, int a_signed, const uint8_t *b, int b_signed,
                        int32_t *c, int64_t rows, int64_t cols, int64_t depth,
                        const int32_t *a_zp, int64_t a_zp_count, const int32_t *b_zp,
                        int64_t b_zp_count) {
  onnx_light_cpu::IntegerMatMul4Bit2D(a, a_signed != 0, b, b_signed != 0, c, rows, cols, depth,
                                      a_zp, a_zp_count, b_zp, b_zp_count);
}

// Y[M,N] = A[M,K] * B where B is [K,N] (trans_b = 0) or [N,K] (trans_b = 1).
// threads > 1 injects an executor view, as the onnx-light session would.
// Returns the GemmAlgorithm the plan selected.
// The plan is built inside the executor scope, as in a session: GemmPlan fixes
// its useful thread count when it is constructed (gemm_plan.cc:200-215).
static int PlanAndRun(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                      int trans_b, float *Y) {
  onnx_light_cpu::MatMulPlan<float> plan(static_cast<size_t>(M), static_cast<size_t>(N),
                                         static_cast<size_t>(K), false, trans_b != 0);
  plan.Execute(A, B, Y);
  return static_cast<int>(plan.gemm_plan().algorithm());
}

int olcref_matmul_f32(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                      int trans_b, float *Y, int threads) {
  if (threads <= 1) return PlanAndRun(M, N, K, A, B, trans_b, Y);
  onnx_light_cpu::ExecutionExecutorView view;
  view.context = nullptr;
  view.effective_threads = threads;
  view.run_blocks = &RunBlocksOnThreads;
  onnx_light_cpu::ExecutionExecutorScope scope(&view);
  return PlanAndRun(M, N, K, A, B, trans_b, Y);
}

uint16_t olcref_f32_to_f16_bits(float value) {
  return onnx_light_cpu::detail::FloatToFloat16Bits(value);
}

} // extern "C"
