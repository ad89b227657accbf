// dropin_errors.cpp -- the C++ drop-in wrappers' error behaviour, checked
// without a GPU (no call here reaches a kernel launch).
//
//   dropin_errors abort_fwd   two_stage_cuda::fused_mha_fwd at head_dim 300:
//                             message on stderr, then std::abort()
//                             (two_stage_cuda_kernels.cu:316-321)
//   dropin_errors abort_bwd   fused_mha_bwd at head_dim 257 (:867-872)
//   dropin_errors throw_null  fused_mha_fwd at head_dim 64 with null device
//                             pointers: std::runtime_error, exit 0 when caught
//   dropin_errors macros      TENSORN_CUDA_AVAILABLE is defined and
//                             CHECK_CUDA_ERROR passes hipSuccess and throws on
//                             an error status; exit 0
#include "tensorn_shim.hpp"
#include "cxxgpt_dropin.hpp"

#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

namespace {

// Stands in for CudaTensor<float> without allocating device memory; the
// pointer is never dereferenced because every call below fails its argument
// checks first.
struct FakeTensor {
    void* p;
    std::vector<size_t> shp;
    void* device_ptr() const { return p; }
    const std::vector<size_t>& shape() const { return shp; }
    size_t size() const { return shp.empty() ? 0 : shp[0] * shp[1]; }
};

int run_abort(bool bwd)
{
    static float dummy[4];
    const size_t B = 1, S = 4, H = 1, Dh = bwd ? 257 : 300;
    FakeTensor t{dummy, {B * S, H * Dh}};
    if (bwd)
        two_stage_cuda::fused_mha_bwd(t, t, t, t, t, t, t, t, B, S, H, Dh);
    else
        two_stage_cuda::fused_mha_fwd(t, t, t, t, B, S, H, Dh);
    std::printf("returned without aborting\n");
    return 3;
}

int run_throw_null()
{
    FakeTensor t{nullptr, {4, 64}};
    try {
        two_stage_cuda::fused_mha_fwd(t, t, t, t, 1, 4, 1, 64);
    } catch (const std::runtime_error& e) {
        std::printf("caught: %s\n", e.what());
        return 0;
    }
    std::printf("no exception\n");
    return 3;
}

int run_macros()
{
#ifndef TENSORN_CUDA_AVAILABLE
    std::printf("TENSORN_CUDA_AVAILABLE not defined\n");
    return 3;
#endif
    CHECK_CUDA_ERROR(hipSuccess);
    try {
        CHECK_CUDA_ERROR(hipErrorInvalidValue);
    } catch (const std::runtime_error& e) {
        std::printf("caught: %s\n", e.what());
        return 0;
    }
    std::printf("no exception\n");
    return 3;
}

} // namespace

int main(int argc, char** argv)
{
    const char* mode = argc > 1 ? argv[1] : "";
    if (!std::strcmp(mode, "abort_fwd"))
        return run_abort(false);
    if (!std::strcmp(mode, "abort_bwd"))
        return run_abort(true);
    if (!std::strcmp(mode, "throw_null"))
        return run_throw_null();
    if (!std::strcmp(mode, "macros"))
        return run_macros();
    std::fprintf(stderr, "usage: dropin_errors abort_fwd|abort_bwd|throw_null|macros\n");
    return 2;
}
