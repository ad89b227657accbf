// gelu.hip -- exact (erf) GELU and its derivative, elementwise.
//
// Replaces two_stage_cuda::gelu_exact / gelu_exact_deriv
// (src/TwoStage/two_stage_cuda_kernels.cuh:84-85, .cu:1888-1924), applied to
// the q/k/v expander FFN activations of two_stage_gpt.hpp:86-99 (forward) and
// their backward:
//   gelu(x)  = 0.5 x (1 + erf(x / sqrt(2)))
//   gelu'(x) = 0.5 (1 + erf(x / sqrt(2))) + x exp(-x^2 / 2) / sqrt(2 pi)
// (erf from the device math library; the reference's derivative uses the
// fast exp, and so does this one).  HBM-bound: 8 bytes per element.
#include "common.hpp"
#include "gelu_dev.hpp"
#include "launch.hpp"

#include <algorithm>

namespace cxg {

// Aligned path: a workgroup takes tiles of GELU_TILE 4-element groups; each
// thread issues its GELU_U 16-byte loads before any arithmetic, so a compute
// unit keeps ~4x more bytes in flight than a one-load-per-trip loop.  The
// tile's loads and stores go through a buffer descriptor whose range ends at
// the tile's last whole group: lanes past it read 0 and their stores are
// dropped, so the ragged last tile needs no branch.  A and C may be the same
// tensor (in place): each element is read and then written by one thread.
constexpr int GELU_U = 4;
constexpr long GELU_TILE = 256L * GELU_U;

template <bool DERIV>
__global__ __launch_bounds__(256) void gelu_vec_kernel(const float* A, float* C, long n,
                                                       long ntiles)
{
    const long n4 = n / 4;
    for (long tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const long first = tile * GELU_TILE;
        const long cnt = n4 - first < GELU_TILE ? n4 - first : GELU_TILE;
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(A + first * 4), 0, (int)(cnt * 16), 0x00020000);
        const __amdgpu_buffer_rsrc_t rc =
            __builtin_amdgcn_make_buffer_rsrc(C + first * 4, 0, (int)(cnt * 16), 0x00020000);
        f4 v[GELU_U];
#pragma unroll
        for (int k = 0; k < GELU_U; k++)
            v[k] = buffer_load_f4(ra, (unsigned)(k * 256 + threadIdx.x) * 16u);
#pragma unroll
        for (int k = 0; k < GELU_U; k++) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[k][e] = DERIV ? gelu_d(v[k][e]) : gelu_f(v[k][e]);
            buffer_store_f4(rc, (unsigned)(k * 256 + threadIdx.x) * 16u, v[k]);
        }
    }
    // tail of n % 4 elements
    const long t = n4 * 4 + threadIdx.x;
    if (blockIdx.x == 0 && t < n)
        C[t] = DERIV ? gelu_d(A[t]) : gelu_f(A[t]);
}

// Unaligned path (either tensor not 16-byte aligned): one element per thread
// and trip of a grid-stride loop.
template <bool DERIV>
__global__ __launch_bounds__(256) void gelu_kernel(const float* A, float* C, long n)
{
    const long stride = (long)gridDim.x * 256;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        C[i] = DERIV ? gelu_d(A[i]) : gelu_f(A[i]);
}

hipError_t gelu_launch(const float* A, float* C, long n, bool deriv, hipStream_t st)
{
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const bool vec = (((uintptr_t)A | (uintptr_t)C) & 15u) == 0;
    ProfScope ps(st, deriv ? "gelu_deriv" : "gelu");
    if (vec) {
        const long ntiles = (n / 4 + GELU_TILE - 1) / GELU_TILE;
        const unsigned blocks = (unsigned)std::max(1L, std::min(ntiles, 1L << 20));
        if (deriv)
            CXG_LAUNCH((gelu_vec_kernel<true>), dim3(blocks), dim3(256), 0, st, A, C, n,
                               ntiles);
        else
            CXG_LAUNCH((gelu_vec_kernel<false>), dim3(blocks), dim3(256), 0, st, A, C, n,
                               ntiles);
    } else {
        const long want = (n + 255) / 256;
        const unsigned blocks = (unsigned)std::max(1L, std::min(want, 8L * cus));
        if (deriv)
            CXG_LAUNCH((gelu_kernel<true>), dim3(blocks), dim3(256), 0, st, A, C, n);
        else
            CXG_LAUNCH((gelu_kernel<false>), dim3(blocks), dim3(256), 0, st, A, C, n);
    }
    return hipGetLastError();
}

} // namespace cxg
