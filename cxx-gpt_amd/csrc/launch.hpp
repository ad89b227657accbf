// launch.hpp -- host-side launch helpers shared by the kernel files and the
// C-ABI: argument checks, the optional per-kernel timing hook and the
// internal launcher declarations.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cxg {

// ---- per-kernel timing hook (off by default) --------------------------------
// When enabled, a ProfScope names the kernel launches made inside it and
// times them with two hipEvents that the launches themselves record: every
// kernel goes out through CXG_LAUNCH, which passes the innermost open scope's
// events to hipExtLaunchKernelGGL (the first launch of the scope sets the
// start event, each launch the stop event), so the events carry the
// dispatches' own start and end times, as a profiler's kernel trace does,
// rather than those of markers placed around the launches.  prof_query()
// synchronises them and reports the summed device time per name.  Used by the
// benchmark to attribute time to the dominant kernel; with the hook off a
// launch is a plain hipLaunchKernelGGL.
bool prof_enabled();
int prof_begin(hipEvent_t* a, hipEvent_t* b);
void prof_end(int token, const char* name);

struct ProfScope {
    int tok;
    const char* name;
    hipEvent_t a, b;
    bool started;
    ProfScope* outer;
    ProfScope(hipStream_t, const char* n);
    ~ProfScope();
};
// The innermost open scope of this thread whose events the next launch
// records (null with the hook off or no scope open).
ProfScope* prof_scope();

#define CXG_LAUNCH(kernel, grid, block, shmem, stream, ...)                                    \
    do {                                                                                      \
        ::cxg::ProfScope* cxg_ps_ = ::cxg::prof_scope();                                     \
        if (cxg_ps_ != nullptr) {                                                             \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream,                         \
                                  cxg_ps_->started ? nullptr : cxg_ps_->a, cxg_ps_->b, 0,     \
                                  __VA_ARGS__);                                               \
            cxg_ps_->started = true;                                                          \
        } else {                                                                              \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);              \
        }                                                                                     \
    } while (0)

// ---- launchers (defined next to their kernels) -----------------------------
// Softmax MHA.  Layout (B*S, H*Dh) row-major.  lse is [B*H][S] (natural log of
// the softmax denominator of the scaled scores, max included).
// Rotary embedding fused into the MHA kernels (rope != nullptr): Q and K are
// read unrotated and rotated per head (head_dim = Dh) as they are loaded, and
// the backward's dQ, dK are the gradients with respect to the unrotated
// inputs.  w[i] = 10000^(-2i/Dh), i < Dh/2.
struct MhaRope {
    float w[128];
};
void mha_rope_freqs(int Dh, MhaRope* r);

// The backward's pre-pass inside the backward kernel (mha_bwd_main_launch
// with ip != nullptr, see mha_bwd_iprep_ok): each job forms Di = rowsum(O dO)
// of the query tiles it visits from their O rows (ip.O), and the persistent
// workgroups zero dQ for the query tiles they own before their first job,
// post their arrival on sync[0] and, before their first atomic into another
// workgroup's tile, wait for all arrivals.  sync: three device words, zero
// before the launch and left zero after it (sync[1] counts departures and the
// last one resets both); sync[2] counts waits that gave up (a workgroup that
// never arrived), so the host can report them.
struct MhaIPrep {
    const float* O;
    unsigned* sync;
};
bool mha_bwd_iprep_ok(int B, int S, int H, int Dh, const float* Q, const float* K,
                      const float* V, const float* dO, const float* O, const float* dQ,
                      const float* dK, const float* dV);
hipError_t mha_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                          float* lse, int B, int S, int H, int Dh, hipStream_t st,
                          const MhaRope* rope = nullptr);
// Narrow heads on short sequences (mhanarrow.hip): Dh <= 16 with the head's
// rows staged in LDS (S rounded up to 16, times 8 or 16 columns, at most 4096
// floats); one workgroup per head, no scratch.  The backward takes lse or,
// when it is null, recomputes the statistics itself; O (forward) may be null
// (lse only).  rope (Dh even): Q and K rotated inside, dQ and dK rotated
// back.  mha_fwd_launch routes forwards of these shapes here; the C ABI's
// backward does the same.
bool mha_nar_ok(int B, int S, int H, int Dh);
hipError_t mha_nar_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                              float* lse, int B, int S, int H, int Dh, hipStream_t st,
                              const MhaRope* rope = nullptr);
hipError_t mha_nar_bwd_launch(const float* Q, const float* K, const float* V, const float* O,
                              const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                              int B, int S, int H, int Dh, hipStream_t st,
                              const MhaRope* rope = nullptr);
hipError_t mha_bwd_prep_launch(const float* O, const float* dO, float* Di, float* dQ,
                               int B, int S, int H, int Dh, hipStream_t st);
// lse (the statistics pass) and the pre-pass's Di and dQ = 0 in one launch, for
// the shapes mha_stats_prep_ok accepts (Dh <= 64, one round of jobs;
// hipErrorInvalidValue otherwise: the two launches above then).
bool mha_stats_prep_ok(int B, int S, int H, int Dh);
hipError_t mha_stats_prep_launch(const float* Q, const float* K, const float* V, const float* O,
                                 const float* dO, float* lse, float* Di, float* dQ, int B, int S,
                                 int H, int Dh, hipStream_t st, const MhaRope* rope = nullptr);
hipError_t mha_bwd_main_launch(const float* Q, const float* K, const float* V,
                               const float* dO, const float* lse, const float* Di,
                               float* dQ, float* dK, float* dV, int B, int S, int H, int Dh,
                               hipStream_t st, const MhaRope* rope = nullptr,
                               const MhaIPrep* ip = nullptr);

// Causal softmax attention for 256 < Dh <= 512 (same layout, lse and backward
// contract as the launchers above; O may be null: statistics only).
constexpr int MHA_WIDE_MAX_DH = 512;
// Split-KV partial records for few-job shapes: mha_wide_fwd_ws_floats(B*H, S)
// floats at `part` (0: no split, part may be null).
size_t mha_wide_fwd_ws_floats(int BH, int S);
hipError_t mha_wide_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                               float* lse, int B, int S, int H, int Dh, float* part,
                               hipStream_t st);
// Chunked backward jobs' partial records: mha_wide_bwd_ws_floats(B*H, S)
// floats at `part` (0: not chunked, part may be null).
size_t mha_wide_bwd_ws_floats(int BH, int S);
hipError_t mha_wide_bwd_launch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, float* part,
                               hipStream_t st);

// GPT's attention for E > 512 (gptmat.hip): a group of sequences' S x S
// scores in memory (rows padded to a multiple of 4), products on the FP32
// GEMM below, batched over the group.  Any S; E a multiple of 4 and 16-byte
// aligned rows; scratch gpt_mat_fwd_ws_floats(B, S, E) floats for the
// forward, gpt_mat_ws_floats(B, S, E) for the backward.  O may be null
// (statistics only); lse [B][S] natural log, nullable in both.
bool gpt_mat_ok(int S, int E);
size_t gpt_mat_fwd_ws_floats(int B, int S, int E);
size_t gpt_mat_ws_floats(int B, int S, int E);
hipError_t gpt_mat_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                              float* lse, int B, int S, int E, float* ws, hipStream_t st);
hipError_t gpt_mat_bwd_launch(const float* Q, const float* K, const float* V, const float* dO,
                              const float* lse, float* dQ, float* dK, float* dV, int B, int S,
                              int E, float* ws, hipStream_t st);

// GPT's attention through block score matrices in scratch (linquad.hip):
// E a multiple of 16 and the scratch within the block-score budget
// (CXXGPT_GPT_PATH=mat in the environment keeps the GEMM path above).  The
// forward forms the scaled causal 16x16 score blocks, their row softmax (P
// over the scores, lse) and O = P V; the backward P and dS = P (dP - Di) /
// sqrt(E) from S and dP = dO V^T, then dQ = dS K, dK = dS^T Q, dV = P^T dO.
// O may be null (statistics only); lse nullable in both (recomputed).
bool gpt_qs_ok(int B, int S, int E);
size_t gpt_qs_ws_bytes(int B, int S, int E, bool bwd);
hipError_t gpt_qs_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                             float* lse, int B, int S, int E, void* ws, hipStream_t st);
hipError_t gpt_qs_bwd_launch(const float* Q, const float* K, const float* V, const float* O,
                             const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                             int B, int S, int E, void* ws, hipStream_t st);

// Exact (erf) GELU or its derivative over n elements (C may alias A).
hipError_t gelu_launch(const float* A, float* C, long n, bool deriv, hipStream_t st);

// FP32 GEMM for the expander FFNs: C[M][N] = epi(sum_k A(i,k) B(k,j)).
//   ak: A(i,k) = A[i*lda + k], else A[k*lda + i]  (ak = false needs bk = false)
//   bk: B(k,j) = B[j*ldb + k], else B[k*ldb + j]
// Epilogues: STORE C = acc; GELU pre = acc (if pre != null), C = gelu(acc);
// DGELU C = acc * gelu'(G) (G indexed like C); ACCUM C += acc.
// N % 4 == 0; a k-contiguous operand needs K % 4 == 0, a row-contiguous one
// its row count % 4 == 0; all tensors 16-byte aligned, strides % 4 == 0.
// ws: ffn_gemm_ws_floats(M, N, K) floats (partial tiles).
enum { FFN_EPI_STORE = 0, FFN_EPI_GELU = 1, FFN_EPI_DGELU = 2, FFN_EPI_ACCUM = 3 };
struct FfnGemm {
    const float* A;
    long lda;
    bool ak;
    const float* B;
    long ldb;
    bool bk;
    int M, N, K;
    int epi;
    float* C;
    long ldc;
    const float* G;
    float* pre;
    // a batch of independent products: product b uses A + b sA, B + b sB and
    // C (G, pre) + b sC (element strides)
    int batch = 1;
    long sA = 0, sB = 0, sC = 0;
    // extents that bound the operand reads, when they differ from the stored
    // extents M, N and the summed K (0: the same).  Rows i >= Mc of A and
    // j >= Nc of B read row Mc-1 / Nc-1 instead (k-contiguous operands) or the
    // last aligned 4-row group below Mc / Nc (row-contiguous ones); a
    // row-contiguous operand's k >= Kc reads k-row Kc-1 (k >= K reads 0).
    int Mc = 0, Nc = 0, Kc = 0;
};
size_t ffn_gemm_ws_floats(int M, int N, int K, int batch = 1);
hipError_t ffn_gemm_launch(const FfnGemm& op, float* ws, hipStream_t st);

// Rotary position embedding, in place on (B*S, D) rows (Q and/or K; either
// may be null, and they may be one buffer).  Frequencies of pairs 0 ..
// head_dim/2-1 travel in the kernel arguments.
constexpr int ROPE_MAX_HEAD_DIM = 1024;
struct RopeFreqs {
    float w[ROPE_MAX_HEAD_DIM / 2];
};
void rope_freqs(int head_dim, RopeFreqs* fr);
hipError_t rope_launch(float* Q, float* K, long B, int S, int D, int head_dim, float sign,
                       hipStream_t st);

} // namespace cxg
