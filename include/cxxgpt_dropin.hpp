// cxxgpt_dropin.hpp -- C++17 wrappers with the reference's kernel-library
// signatures, implemented on the C ABI of libcxxgpt_attn.so (cxxgpt_attn.h).
//
// A CXX-GPT caller that includes this header instead of
//   src/TwoStage/two_stage_cuda_kernels.cuh      (namespace two_stage_cuda)
//   src/LinearAttention/linear_cuda_kernels.cuh  (namespace linear_cuda)
// keeps every call site unchanged: same names, argument order, argument
// meaning and void return.  The tensor arguments are templates over any type
// with `device_ptr()` (TensorN's CudaTensor<float>, or the HIP-backed
// stand-in in tensorn_shim.hpp); `shape()` is used where the reference reads
// it (phi_elu_* take N from shape()[0]).
//
// Behaviour kept from the reference:
//   * launches are asynchronous on the legacy default stream (stream 0);
//   * outputs are fully overwritten; S_buf / z_buf are scratch;
//   * head_dim > 256 prints a message to stderr and calls std::abort()
//     (two_stage_cuda_kernels.cu:316-321, :867-872);
//   * any other failure throws std::runtime_error, as the reference's
//     CHECK_CUDA_ERROR after each launch does (caught by its mains,
//     two_stage_train.cpp:370-374).
#pragma once

#include "cxxgpt_attn.h"

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

namespace cxg_dropin {

inline void check(int status, const char* fn, size_t head_dim = 0)
{
    if (status == CXG_OK)
        return;
    if (status == CXG_ERR_HEAD_DIM) {
        std::fprintf(stderr, "two_stage_cuda::%s: head_dim %zu > 256 not supported\n", fn,
                     head_dim);
        std::abort();
    }
    throw std::runtime_error(std::string(fn) + ": " + cxg_status_str(status) +
                             " (hip error " + std::to_string(cxg_last_hip_error()) + ")");
}

template <class T>
inline const float* cptr(const T& t)
{
    return static_cast<const float*>(t.device_ptr());
}
template <class T>
inline float* mptr(T& t)
{
    return static_cast<float*>(t.device_ptr());
}

} // namespace cxg_dropin

namespace two_stage_cuda {

// two_stage_cuda_kernels.cuh:18-20
template <class CT>
void fused_mha_fwd(const CT& Q, const CT& K, const CT& V, CT& O, size_t B, size_t S, size_t H,
                   size_t Dh)
{
    using namespace cxg_dropin;
    check(cxg_mha_fwd(cptr(Q), cptr(K), cptr(V), mptr(O), nullptr, B, S, H, Dh, nullptr),
          "fused_mha_fwd", Dh);
}

// two_stage_cuda_kernels.cuh:22-27
template <class CT>
void fused_mha_bwd(const CT& Q, const CT& K, const CT& V, const CT& O, const CT& dO, CT& dQ,
                   CT& dK, CT& dV, size_t B, size_t S, size_t H, size_t Dh)
{
    using namespace cxg_dropin;
    check(cxg_mha_bwd(cptr(Q), cptr(K), cptr(V), cptr(O), cptr(dO), nullptr, mptr(dQ), mptr(dK),
                      mptr(dV), B, S, H, Dh, nullptr, 0, nullptr),
          "fused_mha_bwd", Dh);
}

// two_stage_cuda_kernels.cuh:39-44
template <class CT>
void kernel_attn_fwd(const CT& Q, const CT& K, const CT& V, CT& O, CT& den_cache, CT& z_cache,
                     CT& S_buf, CT& z_buf, size_t B, size_t S, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_kattn_fwd(cptr(Q), cptr(K), cptr(V), mptr(O), mptr(den_cache), mptr(z_cache),
                        mptr(S_buf), mptr(z_buf), B, S, D, E, nullptr),
          "kernel_attn_fwd");
}

// two_stage_cuda_kernels.cuh:46-49
template <class CT>
void kernel_attn_bwd_step1(const CT& O, const CT& dO, const CT& den_cache, CT& dnum, CT& dden,
                           size_t N, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_kattn_bwd_step1(cptr(O), cptr(dO), cptr(den_cache), mptr(dnum), mptr(dden), N, E,
                              nullptr),
          "kernel_attn_bwd_step1");
}

// two_stage_cuda_kernels.cuh:51-55
template <class CT>
void kernel_attn_bwd_dQ(const CT& K, const CT& V, const CT& dnum, const CT& dden,
                        const CT& z_cache, const CT& Q, CT& dQ, CT& S_buf, size_t B, size_t S,
                        size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_kattn_bwd_dQ(cptr(K), cptr(V), cptr(dnum), cptr(dden), cptr(z_cache), cptr(Q),
                           mptr(dQ), mptr(S_buf), B, S, D, E, nullptr),
          "kernel_attn_bwd_dQ");
}

// two_stage_cuda_kernels.cuh:57-61
template <class CT>
void kernel_attn_bwd_dKdV(const CT& Q, const CT& K, const CT& V, const CT& dnum, const CT& dden,
                          CT& dK, CT& dV, size_t B, size_t S, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_kattn_bwd_dKdV(cptr(Q), cptr(K), cptr(V), cptr(dnum), cptr(dden), mptr(dK),
                             mptr(dV), B, S, D, E, nullptr),
          "kernel_attn_bwd_dKdV");
}

// two_stage_cuda_kernels.cuh:72-76 (in place; Q and K may be one tensor)
template <class CT>
void rope_fwd(CT& Q, CT& K, size_t B, size_t S, size_t D, size_t head_dim)
{
    using namespace cxg_dropin;
    check(cxg_rope_fwd(mptr(Q), mptr(K), B, S, D, head_dim, nullptr), "rope_fwd");
}

template <class CT>
void rope_bwd(CT& dQ, CT& dK, size_t B, size_t S, size_t D, size_t head_dim)
{
    using namespace cxg_dropin;
    check(cxg_rope_bwd(mptr(dQ), mptr(dK), B, S, D, head_dim, nullptr), "rope_bwd");
}

// two_stage_cuda_kernels.cuh:84-85 (n = A.size(), as the reference's wrappers)
template <class CT>
void gelu_exact(const CT& A, CT& C)
{
    using namespace cxg_dropin;
    check(cxg_gelu_exact(cptr(A), mptr(C), A.size(), nullptr), "gelu_exact");
}

template <class CT>
void gelu_exact_deriv(const CT& A, CT& C)
{
    using namespace cxg_dropin;
    check(cxg_gelu_exact_deriv(cptr(A), mptr(C), A.size(), nullptr), "gelu_exact_deriv");
}

} // namespace two_stage_cuda

// The two-stage block's expander FFN as one call each way: StageBlock's
// q_ffn_fc.forward -> gelu_exact -> q_ffn_proj.forward (two_stage_gpt.hpp:86-89;
// likewise k, v and the final FFN) and its backward (:177-183).  Not a
// reference function: it replaces that call sequence.  X [M][E], W1 [F][E]
// (the fc weight), W2 [E][F] (the proj weight); pre may be null; dW1/dW2
// accumulate (Linear's W.grad +=); G is the tensor gelu' is evaluated at.
namespace cxg_blocks {

template <class CT>
void expander_ffn_fwd(const CT& X, const CT& W1, const CT& W2, CT* pre, CT& act, CT& Y, size_t M,
                      size_t E, size_t F)
{
    using namespace cxg_dropin;
    check(cxg_ffn_fwd(cptr(X), cptr(W1), cptr(W2), pre ? mptr(*pre) : nullptr, mptr(act),
                      mptr(Y), M, E, F, nullptr, 0, nullptr),
          "expander_ffn_fwd");
}

template <class CT>
void expander_ffn_bwd(const CT& X, const CT& W1, const CT& W2, const CT& act, const CT& G,
                      const CT& dY, CT& dX, CT& dW1, CT& dW2, size_t M, size_t E, size_t F)
{
    using namespace cxg_dropin;
    check(cxg_ffn_bwd(cptr(X), cptr(W1), cptr(W2), cptr(act), cptr(G), cptr(dY), mptr(dX),
                      mptr(dW1), mptr(dW2), M, E, F, nullptr, 0, nullptr),
          "expander_ffn_bwd");
}

} // namespace cxg_blocks

namespace linear_cuda {

// linear_cuda_kernels.cuh:11-16
template <class CT>
void causal_linear_attention_fwd(const CT& Q_phi, const CT& K_phi, const CT& V, CT& O,
                                 CT& den_cache, CT& z_cache, CT& S_buf, CT& z_buf, size_t B,
                                 size_t S, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_lin_fwd(cptr(Q_phi), cptr(K_phi), cptr(V), mptr(O), mptr(den_cache),
                      mptr(z_cache), mptr(S_buf), mptr(z_buf), B, S, D, E, nullptr),
          "causal_linear_attention_fwd");
}

// linear_cuda_kernels.cuh:18-22
template <class CT>
void causal_linear_attention_bwd_step1(const CT& O, const CT& dO, const CT& den_cache, CT& dnum,
                                       CT& dden, size_t N, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_lin_bwd_step1(cptr(O), cptr(dO), cptr(den_cache), mptr(dnum), mptr(dden), N, E,
                            nullptr),
          "causal_linear_attention_bwd_step1");
}

// linear_cuda_kernels.cuh:24-29
template <class CT>
void causal_linear_attention_bwd_dQ(const CT& K_phi, const CT& V, const CT& dnum,
                                    const CT& dden, const CT& z_cache, CT& dQ_phi, CT& S_buf,
                                    size_t B, size_t S, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_lin_bwd_dQ(cptr(K_phi), cptr(V), cptr(dnum), cptr(dden), cptr(z_cache),
                         mptr(dQ_phi), mptr(S_buf), B, S, D, E, nullptr),
          "causal_linear_attention_bwd_dQ");
}

// linear_cuda_kernels.cuh:31-37
template <class CT>
void causal_linear_attention_bwd_dKdV(const CT& Q_phi, const CT& K_phi, const CT& V,
                                      const CT& dnum, const CT& dden, CT& dK_phi, CT& dV,
                                      size_t B, size_t S, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_lin_bwd_dKdV(cptr(Q_phi), cptr(K_phi), cptr(V), cptr(dnum), cptr(dden),
                           mptr(dK_phi), mptr(dV), B, S, D, E, nullptr),
          "causal_linear_attention_bwd_dKdV");
}

// linear_cuda_kernels.cuh:39-41; N = x.shape()[0] (linear_cuda_kernels.cu:332)
template <class CT>
void phi_elu_forward(const CT& x, CT& phi, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_phi_elu_fwd(cptr(x), mptr(phi), x.shape()[0], D, E, nullptr), "phi_elu_forward");
}

// linear_cuda_kernels.cuh:43-46; N = dphi.shape()[0] (linear_cuda_kernels.cu:370)
template <class CT>
void phi_elu_backward(const CT& dphi, const CT& x, CT& dx, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_phi_elu_bwd(cptr(dphi), cptr(x), mptr(dx), dphi.shape()[0], D, E, nullptr),
          "phi_elu_backward");
}

// Hadamard+Exp feature map: no counterpart in the reference; same convention
// as phi_elu_* (x (N, E) -> phi (N, D), E % 64 == 0).
template <class CT>
void phi_hexp_forward(const CT& x, CT& phi, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_phi_hexp_fwd(cptr(x), mptr(phi), x.shape()[0], D, E, nullptr), "phi_hexp_forward");
}

template <class CT>
void phi_hexp_backward(const CT& dphi, const CT& x, CT& dx, size_t D, size_t E)
{
    using namespace cxg_dropin;
    check(cxg_phi_hexp_bwd(cptr(dphi), cptr(x), mptr(dx), dphi.shape()[0], D, E, nullptr),
          "phi_hexp_backward");
}

} // namespace linear_cuda
