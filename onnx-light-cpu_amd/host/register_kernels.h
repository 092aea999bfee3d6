// Registration entry points (onnx_light_cpu/kernels/register_kernels.h:22).
#pragma once

namespace onnx_light_cpu_amd {

// Registers every kernel of this library: com.microsoft::MatMulNBits on kGPU.
void RegisterAllKernels();

// Registers MatMulNBits alone (as RegisterMatMulKernel does for MatMul,
// onnx_light_cpu/kernels/math/matmul_kernel.cc:145-159).
void RegisterMatMulNBitsKernel();

} // namespace onnx_light_cpu_amd
