// gptmat.hip -- GPT's attention for embeddings wider than 512 (gfx950).
//
// GPT's block computes attention as one head over the whole embedding E with
// TensorN matmuls, gpt_cuda::attention_mask (-1e10 on cross-batch and future
// entries, gpt_cuda_kernels.cu:458-480), a row softmax and, backward,
// gpt_cuda::softmax_backward (:131-173) (gpt_gpt.hpp:365-380, :420-438).  The
// reference sets no limit on E.  The fused wide-head kernels (mhawide.hip)
// hold a 16-row block of Q, K, V at full width in LDS and stop at E = 512;
// wider embeddings take this path, which keeps each sequence's S x S scores
// in memory (S^2 floats per sequence, one sequence at a time) and runs the
// products on the FP32 MFMA GEMM of ffn.hip:
//   forward   Sc = Q K^T;  P = softmax(Sc / sqrt(E)) causal (lse kept);  O = P V
//   backward  Sc again, P from lse;  dP = dO V^T;
//             dS = P (dP - rowsum(P dP)) / sqrt(E);
//             dV = P^T dO;  dQ = dS K;  dK = dS^T Q
// The masked entries' probabilities are exactly 0, as exp(-1e10 - max) is in
// the reference, so the full-width products give the causal result.  The
// GEMM needs S and E multiples of 4 and 16-byte aligned rows.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>

namespace cxg {

// Row softmax of one sequence's scores in place (one wave per row of the
// S x S matrix, row stride S): P[i][j] = 2^(Sc[i][j] c - L_i) for j <= i, else
// 0, with L_i the base-2 log-sum-exp of the row's unmasked scaled scores
// (c = log2(e) / sqrt(E)).  lse_in (natural log, nullable): use it instead of
// forming L_i; lse_out (nullable): store L_i ln 2.
__global__ __launch_bounds__(256) void gpt_softmax_kernel(float* __restrict__ P,
                                                         const float* __restrict__ lse_in,
                                                         float* __restrict__ lse_out, int S,
                                                         float c)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= S)
        return;
    float* r = P + (long)i * S;
    float L;
    if (lse_in != nullptr) {
        L = lse_in[i] * kLog2e;
    } else {
        float m = -INFINITY;
        for (int j = lane; j <= i; j += 64)
            m = fmaxf(m, r[j] * c);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1)
            m = fmaxf(m, __shfl_xor(m, o, 64));
        float l = 0.0f;
        for (int j = lane; j <= i; j += 64)
            l += fast_exp2(r[j] * c - m);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1)
            l += __shfl_xor(l, o, 64);
        L = m + fast_log2(l);
        if (lse_out != nullptr && lane == 0)
            lse_out[i] = L * kLn2;
    }
    for (int j = lane; j < S; j += 64)
        r[j] = j <= i ? fast_exp2(r[j] * c - L) : 0.0f;
}

// dS[i][j] = P[i][j] (dP[i][j] - sum_j P[i][j] dP[i][j]) * scale, in place
// over dP (one wave per row).
__global__ __launch_bounds__(256) void gpt_softmax_bwd_kernel(const float* __restrict__ P,
                                                             float* __restrict__ dP, int S,
                                                             float scale)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= S)
        return;
    const float* p = P + (long)i * S;
    float* d = dP + (long)i * S;
    float di = 0.0f;
    for (int j = lane; j <= i; j += 64)
        di += p[j] * d[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        di += __shfl_xor(di, o, 64);
    for (int j = lane; j < S; j += 64)
        d[j] = p[j] * (d[j] - di) * scale;
}

bool gpt_mat_ok(int S, int E) { return S % 4 == 0 && E % 4 == 0; }

// Scratch: two S x S matrices and the GEMM's partial tiles (the largest of
// the products' needs).
size_t gpt_mat_ws_floats(int S, int E)
{
    const size_t g = std::max({ffn_gemm_ws_floats(S, S, E), ffn_gemm_ws_floats(S, E, S)});
    return 2 * (size_t)S * S + g;
}

static hipError_t gemm(const float* A, long lda, bool ak, const float* B, long ldb, bool bk,
                       float* C, long ldc, int M, int N, int K, float* ws, hipStream_t st)
{
    FfnGemm op{};
    op.A = A;
    op.lda = lda;
    op.ak = ak;
    op.B = B;
    op.ldb = ldb;
    op.bk = bk;
    op.M = M;
    op.N = N;
    op.K = K;
    op.epi = FFN_EPI_STORE;
    op.C = C;
    op.ldc = ldc;
    return ffn_gemm_launch(op, ws, st);
}

static hipError_t softmax(float* P, const float* lse_in, float* lse_out, int S, int E,
                          hipStream_t st)
{
    ProfScope ps(st, "gpt_softmax");
    const float c = kLog2e / sqrtf((float)E);
    CXG_LAUNCH(gpt_softmax_kernel, dim3((unsigned)((S + 3) / 4)), dim3(256), 0, st, P,
                       lse_in, lse_out, S, c);
    return hipGetLastError();
}

hipError_t gpt_mat_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                              float* lse, int B, int S, int E, float* ws, hipStream_t st)
{
    float* Sc = ws;
    float* gws = ws + 2 * (size_t)S * S;
    for (int b = 0; b < B; b++) {
        const long r0 = (long)b * S * E;
        hipError_t e = gemm(Q + r0, E, true, K + r0, E, true, Sc, S, S, S, E, gws, st);
        if (e == hipSuccess)
            e = softmax(Sc, nullptr, lse != nullptr ? lse + (long)b * S : nullptr, S, E, st);
        if (e == hipSuccess && O != nullptr)
            e = gemm(Sc, S, true, V + r0, E, false, O + r0, E, S, E, S, gws, st);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

hipError_t gpt_mat_bwd_launch(const float* Q, const float* K, const float* V, const float* dO,
                              const float* lse, float* dQ, float* dK, float* dV, int B, int S,
                              int E, float* ws, hipStream_t st)
{
    float* P = ws;
    float* dS = ws + (size_t)S * S;
    float* gws = ws + 2 * (size_t)S * S;
    const float scale = 1.0f / sqrtf((float)E);
    for (int b = 0; b < B; b++) {
        const long r0 = (long)b * S * E;
        hipError_t e = gemm(Q + r0, E, true, K + r0, E, true, P, S, S, S, E, gws, st);
        if (e == hipSuccess)
            e = softmax(P, lse != nullptr ? lse + (long)b * S : nullptr, nullptr, S, E, st);
        if (e == hipSuccess)   // dP = dO V^T
            e = gemm(dO + r0, E, true, V + r0, E, true, dS, S, S, S, E, gws, st);
        if (e == hipSuccess) {
            ProfScope ps(st, "gpt_softmax_bwd");
            CXG_LAUNCH(gpt_softmax_bwd_kernel, dim3((unsigned)((S + 3) / 4)), dim3(256),
                               0, st, P, dS, S, scale);
            e = hipGetLastError();
        }
        if (e == hipSuccess)   // dV = P^T dO
            e = gemm(P, S, false, dO + r0, E, false, dV + r0, E, S, E, S, gws, st);
        if (e == hipSuccess)   // dQ = dS K
            e = gemm(dS, S, true, K + r0, E, false, dQ + r0, E, S, E, S, gws, st);
        if (e == hipSuccess)   // dK = dS^T Q
            e = gemm(dS, S, false, Q + r0, E, false, dK + r0, E, S, E, S, gws, st);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

} // namespace cxg
