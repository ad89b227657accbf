// linattn.hpp -- internal interface of the linear-attention kernels (linattn.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>

namespace cxg {

// Feature map applied inside the kernels: ELU+1 as two_stage computes it, none
// (inputs are features already: linear_cuda), ELU+1 in linear_cuda's
// phi_elu form (LinearGPT's feature map fused into the scans),
// Hadamard+Exp (exp(H x / 8) per 64-column row, phi_hexp fused into the
// fused pair's kernels; D = E = 64 only), or two_stage's ELU+1 of q and k
// rotated by RoPE over their whole width first (head_dim = D: TwoStageGPT's
// stage 2, two_stage_gpt.hpp:113; D even, D <= 512, the fused pair's kernels
// and the quadratic form only).
enum { PHI_ELU1 = 0, PHI_NONE = 1, PHI_ELU1_LG = 2, PHI_HEXP = 3, PHI_ELU1_ROPE = 4 };

__host__ __device__ constexpr bool phi_rope(int phi) { return phi == PHI_ELU1_ROPE; }

// Rotary frequencies for the PHI_ELU1_ROPE kernels, passed by value:
// w[i] = 10000^(-2i/D), i < D/2 (one float for the other maps).
constexpr int LIN_ROPE_MAX_D = 512;
template <int PHI>
struct LinRopeArg {
    float w[phi_rope(PHI) ? LIN_ROPE_MAX_D / 2 : 1];
};
template <int PHI>
inline LinRopeArg<PHI> lin_rope_arg(int D)
{
    LinRopeArg<PHI> a{};
    if constexpr (phi_rope(PHI)) {
        // kernel_test.cpp:453 (the reference's CPU RoPE): powf of the same float exponent
        for (int i = 0; i < D / 2 && i < LIN_ROPE_MAX_D / 2; i++)
            a.w[i] = powf(10000.0f, -2.0f * (float)i / (float)D);
    }
    return a;
}

// floats per segment record in the scan workspace: 64x64 state [d][e] + z[64]
constexpr int LIN_WS = 64 * 64 + 64;

// State anchors of the fused backward.  The fused backward walks each segment
// from its last chunk to its first and obtains the prefix state S before a
// chunk by subtracting chunk products from a later exact prefix.  The
// rounding error of that subtraction is relative to the later prefix, so the
// prefix before chunk 2^k (k = 0, 1, ...) of every sequence, as a forward sum
// forms it, is kept as an anchor (a 64x64 [d][e] record, LIN_ANCH floats) and
// chunk 0 starts from zero: the state of a chunk c >= 1 is then recovered
// from a forward-summed prefix at most c chunks later (of at most about twice
// its size), and chunks of later segments (which start at least one segment
// length into the sequence) from their own segment's end prefix.  lin_nanch(n): anchors below chunk n, i.e. #{k : 2^k < n}.
constexpr int LIN_ANCH = 64 * 64;
__host__ __device__ inline int lin_nanch(long nchunks)
{
    int k = 0;
    while ((1L << k) < nchunks)
        k++;
    return k;
}

struct LinPlan {
    bool quad;   // the quadratic-form kernels (lin_quad_ok)
    bool fast;   // D <= 64 and E <= 64 and not quad: chunked MFMA scan
    int nseg;    // segments per sequence (fast path)
    int L;       // rows per segment (multiple of 16)
    int pass;    // LinPass the plan was made for
};

// The scan pass a plan is for: each sizes its segments to its own main
// kernel's resident workgroups.
enum LinPass { LIN_PASS_FWD = 0, LIN_PASS_DQ = 1, LIN_PASS_DKDV = 2, LIN_PASS_BWD = 3 };

LinPlan lin_plan(int Bq, int S, int D, int E, int pass);
// device scratch (bytes) the fwd / dQ / dKdV launchers need for this plan
size_t lin_ws_bytes(const LinPlan& p, int Bq, int D, int E);

// den_eps: 1 stores den + 1e-8 (linear_cuda), 0 stores den (two_stage).  O is
// num / (den + 1e-8) either way.  Sfin/zfin (nullable) receive the final state,
// sfin_de selecting [d][e] (1) or [e][d] (0) layout.
// ctot / ztab / anch (nullable, fast path only): the context for the fused
// backward: each sequence's final state as a segment record, z before every
// 16-row chunk ([S / 16][64] per sequence) and the state anchors
// ([lin_nanch(S / 16)][LIN_ANCH] per sequence).  ws then holds the segment
// prefix records.
hipError_t lin_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                          float* den, float* zc, float* Sfin, float* zfin, int sfin_de,
                          int den_eps, int Bq, int S, int D, int E, void* ws, hipStream_t st,
                          float* ctot = nullptr, float* ztab = nullptr, float* anch = nullptr);
hipError_t lin_step1_launch(const float* O, const float* dO, const float* den, float* dnum,
                            float* dden, long N, int E, hipStream_t st);
hipError_t lin_dq_launch(int phi, const float* K, const float* V, const float* dnum,
                         const float* dden, const float* zc, const float* Q, float* dQ, int Bq,
                         int S, int D, int E, void* ws, hipStream_t st);
hipError_t lin_dkdv_launch(int phi, const float* Q, const float* K, const float* V,
                           const float* dnum, const float* dden, float* dK, float* dV, int Bq,
                           int S, int D, int E, void* ws, hipStream_t st);
// Fused backward (step 1 + dQ + dK/dV, linbwd.hip) for D, E <= 64 and sequences
// the quadratic form does not take (lin_bwd_fused_ok).  den is the
// forward's den_cache; dnum = dO / den and dden = -(dO . O) / den as in step 1.
bool lin_bwd_fused_ok(int D, int E, long S);
int lin_bwd_slots();   // resident fused-backward workgroups per compute unit
size_t lin_bwd_ws_bytes(const LinPlan& p, int Bq, int S);
size_t lin_bwd_fused_ws_bytes(int Bq, int S, int D, int E, bool with_ctx);
// Forward-to-backward context of the fused pair: the forward's segment prefix
// records, each sequence's final-state record and the z table.
struct LinCtx {
    float* rec;    // Bq * nseg_fwd records (the forward's scan workspace)
    float* tot;    // Bq records
    float* zt;     // Bq * ceil(S / 16) * 64
    float* anch;   // Bq * lin_nanch(ceil(S / 16)) anchors of LIN_ANCH floats
};
// 0: shapes neither the fused kernels nor the block-score path take; for the
// block-score path the context is lin_qs_ctx_bytes (features and score blocks
// A), and lin_ctx_split does not apply.
size_t lin_ctx_bytes(int Bq, int S, int D, int E);
LinCtx lin_ctx_split(void* ctx, int Bq, int S, int D, int E);
// ctx (nullable): as written by the forward with the same dimensions; the
// backward then takes the prefix state and z from it instead of recomputing them.
hipError_t lin_bwd_fused_launch(int phi, const float* Q, const float* K, const float* V,
                                const float* O, const float* dO, const float* den, float* dQ,
                                float* dK, float* dV, int Bq, int S, int D, int E, void* ws,
                                hipStream_t st, const void* ctx);
// The same for other widths, through the split kernels (workspace: zc, dnum,
// dden and the scan scratch).
size_t lin_bwd_split_ws_bytes(int Bq, int S, int D, int E);
// ctx (nullable): the block-score path's context from the forward (then the
// quadratic form's backward takes its features and score blocks).
hipError_t lin_bwd_split_launch(int phi, const float* Q, const float* K, const float* V,
                                const float* O, const float* dO, const float* den, float* dQ,
                                float* dK, float* dV, int Bq, int S, int D, int E, void* ws,
                                hipStream_t st, const void* ctx = nullptr);
// Whether the block-score path serves these dimensions (and so writes and
// takes a context).
bool lin_qs_path(int Bq, int S, int D, int E);
// Segment records of short sequences in one launch (linseq.hip): one pass
// with two workgroups per sequence forms the records the aggregate + scan
// pair writes (reverse = 0: exclusive prefix over segments of
// sum phi(X)^T Y and sum w phi(X); 1: exclusive suffix), for plans where
// lin_seq_cpw(chunks, chunks per segment) > 0.
int lin_seq_cpw(int nch, int cps);
template <int PHI>
hipError_t lin_seqrec_launch(const float* X, const float* Y, const float* w, float* ws, int Bq,
                             int S, int D, int E, int L, int nseg, int reverse, hipStream_t st);
// The whole forward of short sequences (S <= 256) at D = E = 64 in one launch
// (linseq.hip): O, den, z_cache (nullable) and the outputs lin_fwd_launch
// documents (Sfin/zfin, ctot/ztab/anch, nullable); rec (nullable) receives the
// prefix records of the plan's segments (nseg segments of L rows), as the
// records pass would have written them.  No RoPE or Hadamard+Exp map.
bool lin_seqfwd_ok(int S);
template <int PHI>
hipError_t lin_seqfwd_launch(const float* Q, const float* K, const float* V, float* O, float* den,
                             float* zc, float* rec, int nseg, int L, float* Sfin, float* zfin,
                             int sfin_de, float* ctot, float* ztab, float* anch, int den_eps,
                             int Bq, int S, hipStream_t st);
// Wide heads (64 < max(D, E) <= LIN_WIDE_MAX, linwide.hip): the quadratic
// form on FP32 MFMA.  Forward: O, den (den_eps as lin_fwd_launch) and
// z_cache (nullable).
// Backward from step 1's dnum, dden: kinds 1 = dK, dV; 2 = dQ; 3 = all three
// (Q may be null for kinds 2 with PHI_NONE).  State: the final S (layout as
// lin_fwd_launch's sfin_de) and z (nullable) of every sequence.
constexpr int LIN_WIDE_MAX = 512;
bool lin_wide_ok(int D, int E);
// The quadratic form serves every width in (64, 512] and, for D, E <= 64,
// sequences of at most LIN_QUAD_MAX_S rows, where the chunked scan is bound by
// its launches and its serial chunk chain rather than by work.  Measured at
// B' = 96, D = E = 64 (fwd + one-call bwd): S = 128, 42.0 against 48.7 us;
// S = 256, 84.6 against 66.5 us.
constexpr int LIN_QUAD_MAX_S = 128;
bool lin_quad_ok(int D, int E, long S);
// ws: lin_wide_ws_bytes of scratch (query blocks may then be split over
// their keys when B' x S / 16 leaves workgroup slots free), or null.
size_t lin_wide_ws_bytes(int Bq, int S, int D, int E);
hipError_t lin_wide_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                               float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                               void* ws, hipStream_t st);
// ws: lin_wide_bwd_ws_bytes(.., kinds) of scratch, or null (then only widths
// up to LIN_WIDE_MAX, through the one-workgroup-per-block kernels).
size_t lin_wide_bwd_ws_bytes(int Bq, int S, int D, int E, int kinds);
hipError_t lin_wide_bwd_launch(int phi, const float* Q, const float* K, const float* V,
                               const float* dnum, const float* dden, float* dQ, float* dK,
                               float* dV, int Bq, int S, int D, int E, int kinds, hipStream_t st,
                               const float* Qx = nullptr, const float* Kx = nullptr,
                               void* ws = nullptr);
// The quadratic form through block score matrices in scratch (linquad.hip):
// widths multiples of 16, any size, while the scratch (lin_qs_bytes; kinds
// 0 = forward, else as lin_wide_bwd_launch) stays within the path's budget.
// The wide launchers take it whenever they are given the scratch.
bool lin_qs_ok(int Bq, int S, int D, int E);
size_t lin_qs_bytes(int Bq, int S, int D, int E, int kinds);
// ctx (nullable, lin_qs_ctx_bytes): the forward leaves phi(Q), phi(K) (ELU+1
// maps) and the score blocks A there, and the backward (kinds 3) takes them
// instead of forming them again.  The RoPE map's callers write its features
// into the context's feature buffers (lin_qs_ctx_features: 0 = Q, 1 = K) and
// pass them as Q, K.
size_t lin_qs_ctx_bytes(int Bq, int S, int D, int E);
float* lin_qs_ctx_features(void* ctx, int Bq, int S, int D, int which);
hipError_t lin_qs_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                             float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                             void* ws, hipStream_t st, void* ctx = nullptr);
hipError_t lin_qs_bwd_launch(int phi, const float* Q, const float* K, const float* V,
                             const float* dnum, const float* dden, float* dQ, float* dK,
                             float* dV, int Bq, int S, int D, int E, int kinds, void* ws,
                             hipStream_t st, const float* Qx, const float* Kx,
                             const void* ctx = nullptr);
// The quadratic form for any width: lin_quad_ok, or widths above LIN_WIDE_MAX
// when lin_qs_ok.
bool lin_quad_any(int Bq, int S, int D, int E);
// The RoPE map's features for the quadratic form: Fq = phi(rot(Q)), Fk =
// phi(rot(K)) (B' x S rows of width D, D even, D <= LIN_ROPE_MAX_D).  The
// forward then runs with PHI_NONE on them; the backward (lin_wide_bwd_launch
// with phi = PHI_ELU1_ROPE) streams them and takes the raw Q, K as Qx, Kx.
hipError_t lin_rope_feat_launch(const float* Q, const float* K, float* Fq, float* Fk, int Bq,
                                int S, int D, hipStream_t st);
hipError_t lin_wide_state_launch(int phi, const float* K, const float* V, float* Sfin,
                                 float* zfin, int sfin_de, int Bq, int S, int D, int E,
                                 hipStream_t st);
hipError_t phi_elu_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st);
hipError_t phi_elu_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D, int E,
                              hipStream_t st);
hipError_t phi_hexp_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st);
hipError_t phi_hexp_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D,
                               int E, hipStream_t st);

} // namespace cxg
