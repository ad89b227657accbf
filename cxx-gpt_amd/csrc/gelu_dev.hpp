// gelu_dev.hpp -- the exact GELU and its derivative as device functions,
// shared by the elementwise kernels and the FFN GEMM epilogues (so both give
// the same bits for the same input).
//   gelu(x)  = 0.5 x (1 + erf(x / sqrt(2)))
//   gelu'(x) = 0.5 (1 + erf(x / sqrt(2))) + x exp(-x^2 / 2) / sqrt(2 pi)
// (two_stage_cuda_kernels.cu:1888-1924; erf from the device math library,
// the Gaussian term through the fast exp as the reference's derivative has it).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace cxg {

__device__ __forceinline__ float gelu_f(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }

__device__ __forceinline__ float gelu_d(float x)
{
    return 0.5f * (1.0f + erff(x * 0.7071067811865476f)) +
           x * __expf(-0.5f * x * x) * 0.3989422804014327f;
}

} // namespace cxg
