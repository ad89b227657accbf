/*
 * attn_oracle.h -- CPU restatement of CXX-GPT's attention CPU reference.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * attention path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (libcxxgpt_attn.so) never
 * links or calls it.
 *
 * Every routine computes in float (fp32) with the loop order of the
 * reference routine it cites, so its rounding behaves like the
 * reference's own CPU oracle.  Paths are relative to the reference tree.
 *
 * Layouts:
 *   softmax MHA:  Q/K/V/O are (B*S, H*Dh) row-major; head h of row r at
 *                 [(r*H + h)*Dh, +Dh)  (src/TwoStage/kernel_test.cpp:19-22)
 *   linear attn:  Q/K (B*S, D), V/O (B*S, E), one sequence per "batch"
 *                 index b (multi-head callers pass B' = B*H head-major rows).
 */
#ifndef CXXGPT_ATTN_ORACLE_H
#define CXXGPT_ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- generators ---------------- */

/* MT19937 (Matsumoto & Nishimura 1998), the engine behind std::mt19937.
 * The reference's kernel_test draws its inputs from std::mt19937(1234)
 * (src/TwoStage/kernel_test.cpp:12-14). */
typedef struct { uint32_t mt[624]; int idx; } orc_mt19937;
void     orc_mt_seed(orc_mt19937 *g, uint32_t seed);
uint32_t orc_mt_next(orc_mt19937 *g);
/* frand(): (float)rgen() / (float)rgen.max() * 2 - 1 (kernel_test.cpp:14) */
float    orc_mt_frand(orc_mt19937 *g);
void     orc_mt_fill_frand(orc_mt19937 *g, float *out, size_t n);

/* splitmix64 -> Box-Muller normal stream used for the synthetic
 * benchmark inputs: out[i] = mean + std * N(0,1). */
void orc_fill_normal(uint64_t seed, float mean, float stdev, float *out, size_t n);

/* ---------------- softmax MHA ---------------- */

/* Literal ref_mha_fwd called once per output element
 * (kernel_test.cpp:24-46 and the call loop :233-238).  O(B*H*S^2*Dh^2). */
void orc_mha_fwd_literal(const float *Q, const float *K, const float *V, float *O,
                         size_t B, size_t S, size_t H, size_t Dh);

/* Row form of the same arithmetic: scores, max and sum computed once per
 * query row instead of once per output column.  Every output element is
 * produced by the identical float operation sequence as the literal form,
 * so the two agree bit for bit.  O(B*H*S^2*Dh).  nthreads<=1 -> serial.
 * lse (nullable, B*H*S floats, index (b*H+h)*S+s) receives m + log(l)
 * in the natural-log domain of the scaled scores. */
void orc_mha_fwd(const float *Q, const float *K, const float *V, float *O, float *lse,
                 size_t B, size_t S, size_t H, size_t Dh, int nthreads);

/* Literal ref_mha_bwd (kernel_test.cpp:48-94).  dQ/dK/dV are OVERWRITTEN
 * (zeroed first, then accumulated as the reference does).  Heads are
 * independent, so nthreads>1 splits (b,h) over threads without changing any
 * per-element operation order. */
void orc_mha_bwd(const float *Q, const float *K, const float *V, const float *O,
                 const float *dO, float *dQ, float *dK, float *dV,
                 size_t B, size_t S, size_t H, size_t Dh, int nthreads);

/* Same as orc_mha_bwd restricted to the (b,h) pairs listed in heads[]
 * (values b*H+h); other entries of dQ/dK/dV are left untouched. */
void orc_mha_bwd_heads(const float *Q, const float *K, const float *V, const float *O,
                       const float *dO, float *dQ, float *dK, float *dV,
                       size_t B, size_t S, size_t H, size_t Dh,
                       const size_t *heads, size_t nheads, int nthreads);
void orc_mha_fwd_heads(const float *Q, const float *K, const float *V, float *O,
                       size_t B, size_t S, size_t H, size_t Dh,
                       const size_t *heads, size_t nheads, int nthreads);

/* ---------------- ELU+1 linear "kernel" attention (two_stage API) ------- */

float orc_phi_elu(float x);      /* kernel_test.cpp:16 */
float orc_phi_elu_der(float x);  /* kernel_test.cpp:17 */

/* ref_kernel_attn_fwd (kernel_test.cpp:96-126) plus the z_cache output the
 * GPU entry point writes (inclusive cumsum of phi(K), two_stage_cuda_kernels.cu:
 * 1027-1032).  den excludes eps; O divides by den + 1e-8. z_cache nullable. */
void orc_kattn_fwd(const float *Q, const float *K, const float *V,
                   float *O, float *den, float *z_cache,
                   size_t B, size_t S, size_t D, size_t E, int nthreads);

/* Literal ref_kernel_attn_bwd (kernel_test.cpp:128-193): O(B*S^2*D*E). */
void orc_kattn_bwd_literal(const float *Q, const float *K, const float *V,
                           const float *O, const float *dO, const float *den,
                           float *dQ, float *dK, float *dV,
                           size_t B, size_t S, size_t D, size_t E);

/* kernel_attn_bwd_step1 closed form (kernel_test.cpp:277-286;
 * two_stage_cuda_kernels.cu:1190-1219): dnum = dO/den, dden = -sum_e dO*O/den. */
void orc_kattn_bwd_step1(const float *O, const float *dO, const float *den,
                         float *dnum, float *dden, size_t N, size_t E);

/* kernel_attn_bwd_dQ as an O(S*D*E) forward scan
 * (two_stage_cuda_kernels.cu:1253-1300):
 *   dQ_t[d] = (z_cache_t[d]*dden_t + sum_e S_t[e][d]*dnum_t[e]) * phi'(Q_t[d]) */
void orc_kattn_bwd_dQ(const float *K, const float *V, const float *dnum,
                      const float *dden, const float *z_cache, const float *Q,
                      float *dQ, size_t B, size_t S, size_t D, size_t E, int nthreads);

/* kernel_attn_bwd_dKdV as an O(S*D*E) reverse scan
 * (two_stage_cuda_kernels.cu:1596-1676). */
void orc_kattn_bwd_dKdV(const float *Q, const float *K, const float *V,
                        const float *dnum, const float *dden,
                        float *dK, float *dV, size_t B, size_t S, size_t D, size_t E,
                        int nthreads);

/* ---------------- linear_cuda API (phi applied outside) ---------------- */

/* causal_linear_attention_fwd (src/LinearAttention/linear_cuda_kernels.cu:10-79):
 * state [d][e]; den_cache = phiQ.z + 1e-8 (eps INCLUDED); O = num/den_cache.
 * S_buf (B*D, E) and z_buf (B, D) receive the final state (nullable). */
void orc_lcu_fwd(const float *Qp, const float *Kp, const float *V,
                 float *O, float *den_cache, float *z_cache, float *S_buf, float *z_buf,
                 size_t B, size_t S, size_t D, size_t E, int nthreads);
/* causal_linear_attention_bwd_step1 (linear_cuda_kernels.cu:101-134). */
void orc_lcu_bwd_step1(const float *O, const float *dO, const float *den_cache,
                       float *dnum, float *dden, size_t N, size_t E);
/* causal_linear_attention_bwd_dQ (linear_cuda_kernels.cu:152-197): no phi'. */
void orc_lcu_bwd_dQ(const float *Kp, const float *V, const float *dnum,
                    const float *dden, const float *z_cache, float *dQp,
                    size_t B, size_t S, size_t D, size_t E, int nthreads);
/* causal_linear_attention_bwd_dKdV (linear_cuda_kernels.cu:217-273). */
void orc_lcu_bwd_dKdV(const float *Qp, const float *Kp, const float *V,
                      const float *dnum, const float *dden, float *dKp, float *dV,
                      size_t B, size_t S, size_t D, size_t E, int nthreads);
/* phi_elu_forward / backward (linear_cuda_kernels.cu:305-364):
 * phi = (x>0 ? x : expf(x)-1) + 1 with columns d>=E zero; x is (N,E), phi (N,D). */
void orc_phi_elu_forward(const float *x, float *phi, size_t N, size_t D, size_t E);
void orc_phi_elu_backward(const float *dphi, const float *x, float *dx,
                          size_t N, size_t D, size_t E);

/* ---------------- Hadamard+Exp feature map ----------------
 * Not present in the reference code; defined by the benchmark configuration:
 * phi(x) = exp(H_64 x / 8) per 64-wide block of a row, H_64 the Sylvester
 * Hadamard matrix (H[i][j] = (-1)^popcount(i&j)).  Follows the phi_elu_*
 * convention: x (N,E) with E % 64 == 0, phi (N,D) with columns d>=E zero.
 * Backward: dx = H_64 (dphi * phi(x)) / 8 per block (H symmetric). */
float orc_hadamard_entry(int i, int j);
void orc_phi_hexp_forward(const float *x, float *phi, size_t N, size_t D, size_t E);
void orc_phi_hexp_backward(const float *dphi, const float *x, float *dx,
                           size_t N, size_t D, size_t E);

/* ---------------- rotary position embedding ----------------
 * src/TwoStage/kernel_test.cpp:451-471 (ref_rope / rope_one): X (B*S, D),
 * heads of width head_dim; row r has position p = r % S; pair i of a head
 * rotates by sign * p * w_i, w_i = powf(10000, -2i/head_dim), all in float:
 *   x'_2i = x_2i cos - x_2i+1 sin,   x'_2i+1 = x_2i sin + x_2i+1 cos.
 * sign = +1: two_stage_cuda::rope_fwd; -1: rope_bwd (the inverse rotation).
 * In place. */
void orc_rope(float *X, size_t B, size_t S, size_t D, size_t head_dim, float sign);

/* ---------------- exact GELU ----------------
 * src/TwoStage/two_stage_cuda_kernels.cu:1888-1924 (gelu_exact_kernel,
 * gelu_exact_deriv_kernel), in float with the C library's erff / expf:
 *   gelu(x) = 0.5 x (1 + erf(x * 0.7071067811865476))
 *   gelu'(x) = 0.5 (1 + erf(x * 0.70710678...)) + x exp(-0.5 x^2) * 0.3989422804014327 */
void orc_gelu_exact(const float *A, float *C, size_t n);
void orc_gelu_exact_deriv(const float *A, float *C, size_t n);

/* The two-stage block's expander FFN (two_stage_gpt.hpp:86-99, :177-195):
 * Linear (no bias, gpt_gpt.hpp:86-112) -> exact GELU -> Linear.
 * X [M][E], W1 [F][E], W2 [E][F] row-major.
 *   fwd: pre = X W1^T (if pre != NULL), act = gelu(X W1^T), Y = act W2^T
 *   bwd: dact = (dY W2) * gelu'(G); dW2 += dY^T act; dX = dact W1;
 *        dW1 += dact^T X
 * Products accumulate in double and round once to float (the reference's
 * GEMMs are TensorN's cuBLAS calls, whose summation order is not available;
 * this is the correctly rounded fp32 result any order is measured against).
 * Rows are spread over nthreads threads. */
void orc_ffn_fwd(const float *X, const float *W1, const float *W2, float *pre, float *act,
                 float *Y, size_t M, size_t E, size_t F, int nthreads);
void orc_ffn_bwd(const float *X, const float *W1, const float *W2, const float *act,
                 const float *G, const float *dY, float *dX, float *dW1, float *dW2, size_t M,
                 size_t E, size_t F, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
