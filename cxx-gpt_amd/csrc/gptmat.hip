// gptmat.hip -- GPT's attention for embeddings wider than 512 (gfx950).
//
// GPT's block computes attention as one head over the whole embedding E with
// TensorN matmuls, gpt_cuda::attention_mask (-1e10 on cross-batch and future
// entries, gpt_cuda_kernels.cu:458-480), a row softmax and, backward,
// gpt_cuda::softmax_backward (:131-173) (gpt_gpt.hpp:365-380, :420-438).  The
// reference sets no limit on E.  The fused wide-head kernels (mhawide.hip)
// hold a 16-row block of Q, K, V at full width in LDS and stop at E = 512;
// wider embeddings take this path, which keeps the S x S scores of a group of
// sequences in memory and runs the products on the FP32 MFMA GEMM of ffn.hip,
// one batched launch per product for the whole group:
//   forward   Sc = Q K^T;  P = softmax(Sc / sqrt(E)) causal (lse kept);  O = P V
//   backward  Sc again, P from lse;  dP = dO V^T;
//             dS = P (dP - rowsum(P dP)) / sqrt(E);
//             dV = P^T dO;  dQ = dS K;  dK = dS^T Q
// The masked entries' probabilities are exactly 0, as exp(-1e10 - max) is in
// the reference, so the full-width products give the causal result.  A
// sequence's score matrix has S rows of Sp = S rounded up to 4 floats; the
// padding columns hold probability 0, so every product can run its
// contraction over Sp (or S) with 16-byte aligned rows whatever S is.  The
// GEMM needs E a multiple of 4 and 16-byte aligned Q, K, V, O rows.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>
#include <cstdlib>

namespace cxg {

// Row softmax of a group's scores in place (one wave per row of a sequence's
// S x Sp matrix, row stride Sp, sequence blockIdx.y of the group): P[i][j] =
// 2^(Sc[i][j] c - L_i) for j <= i, else 0 (the padding columns j >= S
// included), with L_i the base-2 log-sum-exp of the row's unmasked scaled
// scores (c = log2(e) / sqrt(E)).  lse_in (natural log, nullable): use it
// instead of forming L_i; lse_out (nullable): store L_i ln 2.
__global__ __launch_bounds__(256) void gpt_softmax_kernel(float* __restrict__ P,
                                                         const float* __restrict__ lse_in,
                                                         float* __restrict__ lse_out, int S,
                                                         int Sp, float c)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= S)
        return;
    const long sq = blockIdx.y;
    float* r = P + (sq * S + i) * Sp;
    float L;
    if (lse_in != nullptr) {
        L = lse_in[sq * S + i] * kLog2e;
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
            lse_out[sq * S + i] = L * kLn2;
    }
    for (int j = lane; j < Sp; j += 64)
        r[j] = j <= i ? fast_exp2(r[j] * c - L) : 0.0f;
}

// dS[i][j] = P[i][j] (dP[i][j] - sum_j P[i][j] dP[i][j]) * scale, in place
// over dP (one wave per row, row stride Sp, padding columns included;
// sequence blockIdx.y of the group).
__global__ __launch_bounds__(256) void gpt_softmax_bwd_kernel(const float* __restrict__ P,
                                                             float* __restrict__ dP, int S,
                                                             int Sp, float scale)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= S)
        return;
    const long row = (long)blockIdx.y * S + i;
    const float* p = P + row * Sp;
    float* d = dP + row * Sp;
    float di = 0.0f;
    for (int j = lane; j <= i; j += 64)
        di += p[j] * d[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        di += __shfl_xor(di, o, 64);
    for (int j = lane; j < Sp; j += 64)
        d[j] = p[j] * (d[j] - di) * scale;
}

bool gpt_mat_ok(int S, int E)
{
    (void)S;
    return E % 4 == 0;
}

static int pad4(int S) { return (S + 3) & ~3; }

// Score-matrix floats a group may hold: 2^25 (128 MiB), or the value of the
// environment variable CXXGPT_GPT_SCORE_FLOATS when it is set to a positive
// number (read at each call; callers short of memory lower it, and tests use
// it to force several groups on small problems).
static long score_budget()
{
    const char* v = std::getenv("CXXGPT_GPT_SCORE_FLOATS");
    if (v != nullptr) {
        const long n = std::atol(v);
        if (n > 0)
            return n;
    }
    return 1L << 25;
}

// Sequences per group: as many as keep the group's score matrices (`mats` of
// S x Sp floats per sequence: one forward, two backward) within the budget,
// at least one.
static int gpt_group(int B, int S, int mats)
{
    const long per = (long)mats * S * pad4(S);
    return (int)std::max<long>(1, std::min<long>(B, score_budget() / per));
}

// Scratch: the group's score matrices and the GEMM's partial tiles (the
// largest of the products' needs).
static size_t ws_floats(int B, int S, int E, int mats)
{
    const int nb = gpt_group(B, S, mats), Sp = pad4(S);
    const size_t g = std::max({ffn_gemm_ws_floats(S, Sp, E, nb), ffn_gemm_ws_floats(S, E, Sp, nb),
                               ffn_gemm_ws_floats(S, E, S, nb)});
    return (size_t)mats * nb * S * Sp + g;
}

size_t gpt_mat_fwd_ws_floats(int B, int S, int E) { return ws_floats(B, S, E, 1); }
size_t gpt_mat_ws_floats(int B, int S, int E) { return ws_floats(B, S, E, 2); }

// C_b = A_b B_b for the nb sequences of a group (A, B, C at sequence strides
// sA, sB, sC), C stored over M x N; operand reads bounded by Mc, Nc, Kc.
static hipError_t gemm(const float* A, long lda, bool ak, long sA, const float* B, long ldb,
                       bool bk, long sB, float* C, long ldc, long sC, int M, int N, int K,
                       int Mc, int Nc, int Kc, int nb, float* ws, hipStream_t st)
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
    op.Mc = Mc;
    op.Nc = Nc;
    op.Kc = Kc;
    op.epi = FFN_EPI_STORE;
    op.C = C;
    op.ldc = ldc;
    op.batch = nb;
    op.sA = sA;
    op.sB = sB;
    op.sC = sC;
    return ffn_gemm_launch(op, ws, st);
}

static hipError_t softmax(float* P, const float* lse_in, float* lse_out, int S, int E, int nb,
                          hipStream_t st)
{
    ProfScope ps(st, "gpt_softmax");
    const float c = kLog2e / sqrtf((float)E);
    CXG_LAUNCH(gpt_softmax_kernel, dim3((unsigned)((S + 3) / 4), (unsigned)nb), dim3(256), 0, st,
               P, lse_in, lse_out, S, pad4(S), c);
    return hipGetLastError();
}

// The products, per group, with Sp = S rounded up to 4 (score rows padded):
//   scores  Q K^T    stored S x Sp; K's rows read below S
//   O       P V      summed over Sp (P's padding is 0); V's rows read below S
//   dV      P^T dO   summed over the S query rows; P's columns read below Sp
//   dQ      dS K     as O
//   dK      dS^T Q   as dV
hipError_t gpt_mat_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                              float* lse, int B, int S, int E, float* ws, hipStream_t st)
{
    const int G = gpt_group(B, S, 1), Sp = pad4(S);
    const long SE = (long)S * E, SS = (long)S * Sp;
    float* Sc = ws;
    float* gws = ws + (size_t)G * SS;
    for (int b0 = 0; b0 < B; b0 += G) {
        const int nb = std::min(G, B - b0);
        const long r0 = (long)b0 * SE;
        hipError_t e = gemm(Q + r0, E, true, SE, K + r0, E, true, SE, Sc, Sp, SS, S, Sp, E, S, S,
                            E, nb, gws, st);
        if (e == hipSuccess)
            e = softmax(Sc, nullptr, lse != nullptr ? lse + (long)b0 * S : nullptr, S, E, nb, st);
        if (e == hipSuccess && O != nullptr)
            e = gemm(Sc, Sp, true, SS, V + r0, E, false, SE, O + r0, E, SE, S, E, Sp, S, E, S, nb,
                     gws, st);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

hipError_t gpt_mat_bwd_launch(const float* Q, const float* K, const float* V, const float* dO,
                              const float* lse, float* dQ, float* dK, float* dV, int B, int S,
                              int E, float* ws, hipStream_t st)
{
    const int G = gpt_group(B, S, 2), Sp = pad4(S);
    const long SE = (long)S * E, SS = (long)S * Sp;
    float* P = ws;
    float* dS = ws + (size_t)G * SS;
    float* gws = ws + 2 * (size_t)G * SS;
    const float scale = 1.0f / sqrtf((float)E);
    for (int b0 = 0; b0 < B; b0 += G) {
        const int nb = std::min(G, B - b0);
        const long r0 = (long)b0 * SE;
        hipError_t e = gemm(Q + r0, E, true, SE, K + r0, E, true, SE, P, Sp, SS, S, Sp, E, S, S,
                            E, nb, gws, st);
        if (e == hipSuccess)
            e = softmax(P, lse != nullptr ? lse + (long)b0 * S : nullptr, nullptr, S, E, nb, st);
        if (e == hipSuccess)   // dP = dO V^T
            e = gemm(dO + r0, E, true, SE, V + r0, E, true, SE, dS, Sp, SS, S, Sp, E, S, S, E, nb,
                     gws, st);
        if (e == hipSuccess) {
            ProfScope ps(st, "gpt_softmax_bwd");
            CXG_LAUNCH(gpt_softmax_bwd_kernel, dim3((unsigned)((S + 3) / 4), (unsigned)nb),
                       dim3(256), 0, st, P, dS, S, Sp, scale);
            e = hipGetLastError();
        }
        if (e == hipSuccess)   // dV = P^T dO
            e = gemm(P, Sp, false, SS, dO + r0, E, false, SE, dV + r0, E, SE, S, E, S, Sp, E, S,
                     nb, gws, st);
        if (e == hipSuccess)   // dQ = dS K
            e = gemm(dS, Sp, true, SS, K + r0, E, false, SE, dQ + r0, E, SE, S, E, Sp, S, E, S,
                     nb, gws, st);
        if (e == hipSuccess)   // dK = dS^T Q
            e = gemm(dS, Sp, false, SS, Q + r0, E, false, SE, dK + r0, E, SE, S, E, S, Sp, E, S,
                     nb, gws, st);
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

} // namespace cxg
