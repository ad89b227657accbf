/*
 * cxxgpt_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in replacement for CXX-GPT's attention kernels: one entry point per
 * C++ function the reference's callers bind (two_stage_cuda:: and
 * linear_cuda::), taking raw device pointers, the reference's size_t
 * dimensions and a HIP stream.  The header needs no HIP or C++ headers.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (hipMalloc'd or equivalent), fp32,
 *     row-major, dense.  Outputs are fully overwritten.
 *   - stream: a hipStream_t passed as void*; NULL is the legacy default
 *     stream, which is what the reference launches on.
 *   - Launches are asynchronous; no entry point synchronises the device.
 *   - Return value: CXG_OK or one of the CXG_ERR_* codes below.  A call with
 *     an error code launched nothing (except CXG_ERR_HIP, reported by the
 *     HIP runtime at launch).
 *   - Empty problems (B, S, H or N equal to 0) return CXG_OK and launch
 *     nothing.
 *   - Scratch.  Where an entry point needs device scratch and the caller
 *     passes no workspace, the library uses a buffer it keeps per (device,
 *     stream), grown to the largest request seen on that stream (growth
 *     calls hipFree/hipMalloc, which wait for the device) and held until the
 *     process ends; under stream capture it takes stream-ordered memory for
 *     the call instead (hipMallocAsync, recorded as graph memory nodes).  A
 *     stream handle that is destroyed and reused inherits its buffer: destroy
 *     a stream only once its work is done.
 *
 * Citations are relative to the reference tree (yauntyour/CXX-GPT).
 */
#ifndef CXXGPT_ATTN_H
#define CXXGPT_ATTN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *cxg_stream_t; /* hipStream_t */

enum {
    CXG_OK = 0,
    CXG_ERR_NULL = 1,      /* a required pointer is NULL */
    CXG_ERR_DIMS = 2,      /* a dimension is zero where it may not be, or too large */
    CXG_ERR_HEAD_DIM = 3,  /* softmax head_dim > 256 (the reference aborts) */
    CXG_ERR_HIP = 4,       /* the HIP runtime reported an error */
    CXG_ERR_WORKSPACE = 5, /* workspace too small, or its allocation failed */
    CXG_ERR_ALIGN = 6      /* a tensor is not 16-byte aligned, or a width is not a multiple of 4 */
};

/* Human-readable name of a status code (static string). */
const char *cxg_status_str(int status);
/* hipError_t of the last CXG_ERR_HIP on this thread (0 if none). */
int cxg_last_hip_error(void);
/* Library version string. */
const char *cxg_version(void);
/* Frees the scratch buffer the library keeps for (current device, stream),
 * e.g. after a one-off call with large sizes; the next call that needs
 * scratch on that stream allocates it again.  Waits for the stream's work
 * first.  Not for use while another thread calls into the library on the
 * same stream, nor under stream capture.  No counterpart in the reference
 * (it allocates its temporaries per call). */
int cxg_release_scratch(cxg_stream_t stream);

/* ===================== fused causal softmax MHA =====================
 * Q/K/V/O/dO/dQ/dK/dV: (B*S, H*Dh); head h of row r at [(r*H+h)*Dh, +Dh).
 * scale = 1/sqrt(Dh), causal mask key <= query.  1 <= Dh <= 256.
 */

/* two_stage_cuda::fused_mha_fwd (src/TwoStage/two_stage_cuda_kernels.cuh:18-20,
 * two_stage_cuda_kernels.cu:285-326).  lse (nullable): [B*H][S] natural-log
 * softmax normaliser of the scaled scores (row max included); passing it to
 * cxg_mha_bwd skips the backward's statistics pass. */
int cxg_mha_fwd(const float *Q, const float *K, const float *V, float *O, float *lse,
                size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream);

/* two_stage_cuda::fused_mha_bwd (two_stage_cuda_kernels.cuh:22-27,
 * two_stage_cuda_kernels.cu:830-882).  lse: as written by cxg_mha_fwd, or NULL
 * to recompute it (the reference's signature has no lse).  workspace: at least
 * cxg_mha_bwd_workspace_size() bytes of device memory, or NULL for the
 * library's scratch (see the conventions above).  Narrow heads on short
 * sequences (Dh <= 16, and S rounded up to 16 times 8 columns for Dh <= 8, or
 * 16 columns otherwise, at most 4096) run as one kernel per call that uses no
 * scratch: a workspace passed is still checked for size and left unused, and
 * NULL allocates nothing. */
int cxg_mha_bwd(const float *Q, const float *K, const float *V, const float *O,
                const float *dO, const float *lse, float *dQ, float *dK, float *dV,
                size_t B, size_t S, size_t H, size_t Dh, void *workspace,
                size_t workspace_bytes, cxg_stream_t stream);

/* Waits inside cxg_mha_bwd that gave up (0 normally).  With lse, head_dim 64
 * and 16-byte aligned tensors, the backward kernel forms Di = rowsum(O dO)
 * and zeroes dQ itself: each of its workgroups (one per compute unit or
 * fewer, all resident at once) does so for the query tiles it owns, then,
 * before it reads another's, waits until all have done theirs.  That wait is
 * bounded (about half a second); a wait that gives up is counted per
 * (device, stream), and the backward results of that call are then not
 * reliable.  *count receives the stream's count (it waits for the stream's
 * work first).  Without such calls on the stream the count is 0.  No
 * counterpart in the reference. */
int cxg_wait_timeouts(cxg_stream_t stream, unsigned *count);
size_t cxg_mha_bwd_workspace_size(size_t B, size_t S, size_t H, size_t Dh);

/* Allocation-free cxg_mha_bwd.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, results
 * and errors as cxg_mha_bwd without a workspace; the scratch (the row sums
 * Di and, with lse == NULL, the statistics pass's lse) is a static device
 * array of 2 * CXG_MHA_BWD_NOALLOC_MAX_ROWS floats (4 MiB) per GPU, held
 * until the process ends.  B*H*S above CXG_MHA_BWD_NOALLOC_MAX_ROWS returns
 * CXG_ERR_WORKSPACE and launches nothing.  The call allocates nothing
 * (no hipMalloc, hipFree or allocating library routine).  Every call on one
 * GPU uses that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race. */
#define CXG_MHA_BWD_NOALLOC_MAX_ROWS (1u << 19)
int cxg_mha_bwd_noalloc(const float *Q, const float *K, const float *V, const float *O,
                        const float *dO, const float *lse, float *dQ, float *dK, float *dV,
                        size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream);

/* RoPE fused into the MHA kernels.  No single counterpart in the reference:
 * cxg_mha_rope_fwd(Q, K, ...) computes what two_stage_gpt.hpp:102-106 does
 * with rope_fwd(Q, K, B, S, H*Dh, Dh) followed by fused_mha_fwd, reading Q
 * and K unrotated and leaving them unchanged (they are rotated as they are
 * loaded).  cxg_mha_rope_bwd takes the same unrotated Q, K and returns dQ,
 * dK with respect to them: fused_mha_bwd on the rotated tensors followed by
 * rope_bwd(dQ, dK) (two_stage_gpt.hpp:171-174).  Dh even; otherwise as
 * cxg_mha_fwd / cxg_mha_bwd (lse from cxg_mha_rope_fwd, same workspace). */
int cxg_mha_rope_fwd(const float *Q, const float *K, const float *V, float *O, float *lse,
                     size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream);
int cxg_mha_rope_bwd(const float *Q, const float *K, const float *V, const float *O,
                     const float *dO, const float *lse, float *dQ, float *dK, float *dV,
                     size_t B, size_t S, size_t H, size_t Dh, void *workspace,
                     size_t workspace_bytes, cxg_stream_t stream);

/* GPT's attention (src/GPT/gpt_gpt.hpp:365-380 forward, :420-438 backward):
 * one head over the embedding, scores (B*S) x (B*S) with the block-diagonal
 * causal mask of gpt_cuda::attention_mask (gpt_cuda_kernels.cu:458-480),
 * softmax, times V, and the backward through gpt_cuda::softmax_backward.  No
 * single counterpart in the reference (it is matmuls, a mask, a softmax and
 * transposes).  Q, K, V, O (B*S, E) row-major; lse [B][S] natural log; the
 * same as cxg_mha_fwd / cxg_mha_bwd with H = 1, Dh = E, which serve E <= 256.
 * Above 256, widths that are multiples of 16 keep the causal 16x16 score
 * blocks in scratch (B * nb(nb+1)/2 KB per matrix, nb = ceil(S/16): the
 * forward one matrix, the backward two plus Di and lse rows) whenever that
 * fits the library's 512 MB budget for them, and run every product per
 * 64-column slice; the environment variable CXXGPT_GPT_PATH=mat (read at
 * each call) turns this off.  Otherwise 256 < E <= 512 (the reference GPT's
 * training configuration has E = 512) takes wider-head kernels.  There, shapes with few 16-row query blocks
 * split the forward's key range over more workgroups and merge the partial
 * softmax states: the forward then takes the library's scratch for them, and
 * cxg_gpt_attn_bwd_workspace_size counts them for the backward's statistics
 * pass (lse == NULL), as well as the partial sums of the backward's own
 * chunked jobs.  Above E = 512 (the reference has no limit) each sequence's
 * S x S scores (rows padded to a multiple of 4 floats) are kept in scratch
 * and the products run as FP32 MFMA GEMMs; any S up to 16384 (CXG_ERR_DIMS
 * beyond), E a multiple of 4 and the tensors 16-byte aligned (CXG_ERR_ALIGN
 * otherwise).  The forward takes the library's scratch for one score matrix
 * per sequence of a group, the backward's workspace holds two per sequence of
 * a group and the GEMMs' partial tiles; a group is as many sequences as keep
 * its score matrices within 2^25 floats (128 MiB), or within the value of the
 * environment variable CXXGPT_GPT_SCORE_FLOATS when it is set (read at each
 * call, so workspace size and call must see the same value). */
int cxg_gpt_attn_fwd(const float *Q, const float *K, const float *V, float *O, float *lse,
                     size_t B, size_t S, size_t E, cxg_stream_t stream);
int cxg_gpt_attn_bwd(const float *Q, const float *K, const float *V, const float *O,
                     const float *dO, const float *lse, float *dQ, float *dK, float *dV,
                     size_t B, size_t S, size_t E, void *workspace, size_t workspace_bytes,
                     cxg_stream_t stream);
size_t cxg_gpt_attn_bwd_workspace_size(size_t B, size_t S, size_t E);

/* ============ ELU+1 linear "kernel" attention, two_stage_cuda API ============
 * phi(x) = x > 0 ? x + 1 : exp(x), fused.  Q/K (B*S, D), V/O (B*S, E); one
 * sequence per b (multi-head callers pass B = batch*heads, head-major rows).
 * den_cache (B*S) excludes eps; O = num / (den + 1e-8).
 */

/* two_stage_cuda::kernel_attn_fwd (two_stage_cuda_kernels.cuh:39-44,
 * two_stage_cuda_kernels.cu:1133-1185).  z_cache (B*S, D): inclusive cumsum of
 * phi(K); may be NULL (not written) when the backward is cxg_kattn_bwd, which
 * does not read it.  S_buf (B*E, D) and z_buf (B, D): scratch, contents
 * unspecified after the call (may be NULL). */
int cxg_kattn_fwd(const float *Q, const float *K, const float *V, float *O,
                  float *den_cache, float *z_cache, float *S_buf, float *z_buf,
                  size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream);

/* two_stage_cuda::kernel_attn_bwd_step1 (two_stage_cuda_kernels.cuh:46-49,
 * two_stage_cuda_kernels.cu:1190-1248): dnum = dO/den, dden = -sum_e dO*O/den. */
int cxg_kattn_bwd_step1(const float *O, const float *dO, const float *den_cache,
                        float *dnum, float *dden, size_t N, size_t E,
                        cxg_stream_t stream);

/* two_stage_cuda::kernel_attn_bwd_dQ (two_stage_cuda_kernels.cuh:51-55,
 * two_stage_cuda_kernels.cu:1253-1453).  S_buf: scratch (may be NULL). */
int cxg_kattn_bwd_dQ(const float *K, const float *V, const float *dnum,
                     const float *dden, const float *z_cache, const float *Q, float *dQ,
                     float *S_buf, size_t B, size_t S, size_t D, size_t E,
                     cxg_stream_t stream);

/* two_stage_cuda::kernel_attn_bwd_dKdV (two_stage_cuda_kernels.cuh:57-61,
 * two_stage_cuda_kernels.cu:1467-1809). */
int cxg_kattn_bwd_dKdV(const float *Q, const float *K, const float *V,
                       const float *dnum, const float *dden, float *dK, float *dV,
                       size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream);

/* Fused backward: kernel_attn_bwd_step1 + kernel_attn_bwd_dQ +
 * kernel_attn_bwd_dKdV in one call, as two_stage_gpt.hpp:149-157 issues them
 * (two_stage_cuda_kernels.cuh:46-61).  No single counterpart in the reference.
 * Reads Q, K, V, O, dO and den_cache once and writes dQ, dK, dV; the step-1
 * intermediates (dnum = dO/den, dden = -sum_e dO*O/den) stay on chip and no
 * z_cache is needed.  ctx: NULL, or the context cxg_kattn_fwd_ctx wrote for the
 * same Q, K, V and dimensions (the backward then skips re-reading K and V for
 * the prefix state).  The library remembers, per context pointer, the device,
 * dimensions and feature map of the forward that last wrote it: a context
 * with no such record, or written for other dimensions, another device or
 * another API's forward (cxg_lin_fwd_ctx, cxg_lin_elu_fwd), is refused with
 * CXG_ERR_WORKSPACE before any launch.  The check compares dimensions, device
 * and feature map only: it cannot see that a context's memory was freed and
 * reused for another context of the same shape.  A forward that writes a
 * context forgets every earlier record whose bytes it overlaps, and at most
 * 4096 records are kept.  D <= 64 and E <= 64 take the fused
 * kernels (sequences of up to 128 rows the quadratic form); wider heads run
 * step 1 and the quadratic-form backward (dnum, dden in the library's
 * scratch): with both widths multiples of 16 through block score matrices,
 * and then the context holds the forward's phi(Q), phi(K) and score blocks,
 * which the backward takes instead of forming them again; other widths up to
 * 512 through the one-workgroup-per-block kernels and wider ones through the
 * split kernels, where the forward writes no context (cxg_lin_ctx_size is 0)
 * and ctx is not read. */
int cxg_kattn_bwd(const float *Q, const float *K, const float *V, const float *O,
                  const float *dO, const float *den_cache, const void *ctx, float *dQ,
                  float *dK, float *dV, size_t B, size_t S, size_t D, size_t E,
                  cxg_stream_t stream);

/* Forward that leaves a context for the fused backward instead of z_cache:
 * O and den_cache as cxg_kattn_fwd writes them, plus in ctx (device memory of
 * cxg_lin_ctx_size() bytes) the per-segment prefix states, each sequence's
 * final state and z before every 16-row chunk.  No counterpart in the
 * reference (its forward hands the backward z_cache, B*S*D floats; the context
 * is about a fifth of that at B' = 96, S = 4096, D = E = 64).  Wider heads
 * whose widths are multiples of 16 (the block-score quadratic form) keep
 * phi(Q), phi(K) and the causal 16x16 score blocks there instead:
 * 2*B*S*D + B*nb(nb+1)/2*256 floats, nb = ceil(S/16) (9.4 MB at B = 8,
 * S = 256, D = E = 512).  For shapes neither takes, cxg_lin_ctx_size() is 0,
 * ctx may be NULL and nothing is written to it. */
size_t cxg_lin_ctx_size(size_t B, size_t S, size_t D, size_t E);
int cxg_kattn_fwd_ctx(const float *Q, const float *K, const float *V, float *O,
                      float *den_cache, void *ctx, size_t ctx_bytes, size_t B, size_t S,
                      size_t D, size_t E, cxg_stream_t stream);

/* TwoStageGPT's stage 2 with its RoPE fused into the linear-attention
 * kernels: cxg_kattn_rope_fwd replaces two_stage_cuda::rope_fwd(lqc, lkc, B,
 * S, E, E) followed by kernel_attn_fwd (two_stage_gpt.hpp:113-122), and
 * cxg_kattn_rope_bwd replaces kernel_attn_bwd_step1 + _bwd_dQ + _bwd_dKdV
 * followed by rope_bwd(dlq, dlk, B, S, E, E) (:149-160; the rotation is
 * two_stage_cuda_kernels.cu:1810-1878).  No single counterpart in the
 * reference.  Q and K are read unrotated and left unchanged: each row t of a
 * sequence is rotated over its whole width (head_dim = D, pair i by
 * t * 10000^(-2i/D)) as it is loaded, phi = ELU+1 is applied to the rotated
 * row, and dQ, dK are the gradients with respect to the unrotated Q, K.  The
 * forward writes O and den_cache as cxg_kattn_fwd (no z_cache: the backward
 * here does not need it) and, like cxg_kattn_fwd_ctx, the context ctx for the
 * backward when cxg_lin_ctx_size(B, S, D, E) is not 0 (ctx may be NULL with
 * ctx_bytes 0 otherwise, and for the backward).  A context written by
 * another forward is refused (CXG_ERR_WORKSPACE).  D even and at most 1024
 * (CXG_ERR_DIMS).  The chunked scan (D, E <= 64, more than 128 rows) rotates
 * rows inside its kernels as it stages them and rotates dQ, dK back before
 * storing them; the quadratic form (widths up to 512, and shorter sequences)
 * forms phi(rot(Q)), phi(rot(K)) once in a pre-pass into the library's
 * scratch, or into the context when it has one (the block-score path: the
 * backward then takes them and the score blocks from there), and its backward
 * applies phi' and the inverse rotation as it stores dQ, dK; heads wider than
 * 512 rotate copies of Q and K in the library's scratch and rotate dQ, dK
 * back in place, and use no context. */
int cxg_kattn_rope_fwd(const float *Q, const float *K, const float *V, float *O,
                       float *den_cache, void *ctx, size_t ctx_bytes, size_t B, size_t S,
                       size_t D, size_t E, cxg_stream_t stream);
int cxg_kattn_rope_bwd(const float *Q, const float *K, const float *V, const float *O,
                       const float *dO, const float *den_cache, const void *ctx, float *dQ,
                       float *dK, float *dV, size_t B, size_t S, size_t D, size_t E,
                       cxg_stream_t stream);

/* ============ causal linear attention, linear_cuda API (phi outside) ==========
 * Inputs are feature-mapped already: Q_phi/K_phi (B*S, D), V/O (B*S, E).
 * State layout [d][e]; den_cache includes eps (den = phiQ.z + 1e-8).
 */

/* linear_cuda::causal_linear_attention_fwd (src/LinearAttention/
 * linear_cuda_kernels.cuh:11-16, linear_cuda_kernels.cu:10-99).  S_buf (B*D, E)
 * and z_buf (B, D) receive the final state (may be NULL). */
int cxg_lin_fwd(const float *Q_phi, const float *K_phi, const float *V, float *O,
                float *den_cache, float *z_cache, float *S_buf, float *z_buf,
                size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream);

/* Fused backward of the linear_cuda API: causal_linear_attention_bwd_step1 +
 * _bwd_dQ + _bwd_dKdV in one call, as linear_gpt.hpp:154-167 issues them.  No
 * single counterpart in the reference.  den_cache as written by cxg_lin_fwd
 * (eps included); widths and ctx as cxg_kattn_bwd (ctx from cxg_lin_fwd_ctx).
 * z_cache of cxg_lin_fwd may be NULL when this backward is used. */
int cxg_lin_bwd(const float *Q_phi, const float *K_phi, const float *V, const float *O,
                const float *dO, const float *den_cache, const void *ctx, float *dQ_phi,
                float *dK_phi, float *dV, size_t B, size_t S, size_t D, size_t E,
                cxg_stream_t stream);
/* The context-writing forward of the linear_cuda API (as cxg_kattn_fwd_ctx;
 * den_cache includes eps). */
int cxg_lin_fwd_ctx(const float *Q_phi, const float *K_phi, const float *V, float *O,
                    float *den_cache, void *ctx, size_t ctx_bytes, size_t B, size_t S,
                    size_t D, size_t E, cxg_stream_t stream);

/* linear_cuda::causal_linear_attention_bwd_step1 (linear_cuda_kernels.cuh:18-22,
 * linear_cuda_kernels.cu:101-150). */
int cxg_lin_bwd_step1(const float *O, const float *dO, const float *den_cache,
                      float *dnum, float *dden, size_t N, size_t E, cxg_stream_t stream);

/* linear_cuda::causal_linear_attention_bwd_dQ (linear_cuda_kernels.cuh:24-29,
 * linear_cuda_kernels.cu:152-215).  S_buf: scratch (may be NULL). */
int cxg_lin_bwd_dQ(const float *K_phi, const float *V, const float *dnum,
                   const float *dden, const float *z_cache, float *dQ_phi, float *S_buf,
                   size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream);

/* linear_cuda::causal_linear_attention_bwd_dKdV (linear_cuda_kernels.cuh:31-37,
 * linear_cuda_kernels.cu:217-298). */
int cxg_lin_bwd_dKdV(const float *Q_phi, const float *K_phi, const float *V,
                     const float *dnum, const float *dden, float *dK_phi, float *dV,
                     size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream);

/* LinearGPT's attention block with the feature map fused into the scans
 * (linear_gpt.hpp:100-112 forward, :154-172 backward).  No single counterpart
 * in the reference.  cxg_lin_elu_fwd = phi_elu_forward(Xq), phi_elu_forward(Xk)
 * then causal_linear_attention_fwd, on the raw projections Xq, Xk (B*S, E)
 * (phi in the (expf(x)-1)+1 form of phi_elu_fwd_kernel; the reference's
 * zero-padded phi columns E..D-1 contribute nothing and are not formed): O and
 * den_cache (eps included) as the reference's, plus the context for the
 * backward (cxg_lin_ctx_size(B, S, E, E) bytes; may be NULL with ctx_bytes 0).
 * cxg_lin_elu_bwd = step1, dQ, dKdV and the two phi_elu_backward calls: dXq,
 * dXk (B*S, E) with respect to the raw projections, and dV. */
int cxg_lin_elu_fwd(const float *Xq, const float *Xk, const float *V, float *O,
                    float *den_cache, void *ctx, size_t ctx_bytes, size_t B, size_t S,
                    size_t E, cxg_stream_t stream);
int cxg_lin_elu_bwd(const float *Xq, const float *Xk, const float *V, const float *O,
                    const float *dO, const float *den_cache, const void *ctx, float *dXq,
                    float *dXk, float *dV, size_t B, size_t S, size_t E, cxg_stream_t stream);

/* Hadamard+Exp attention block with the feature map fused into the scans: no
 * single counterpart in the reference; its benchmark configuration (96
 * sequences, S = 1024, D = E = 64) applies phi(x) = exp(H x / 8)
 * (cxg_phi_hexp_fwd below) to the raw projections before
 * causal_linear_attention_fwd and maps the feature gradients back with phi's
 * backward after the three backward calls (linear_cuda_kernels.cu:
 * 10-298).  cxg_lin_hexp_fwd: O and den_cache (eps included) from the raw
 * Xq, Xk (B*S, E) and V, plus the context for the backward
 * (cxg_lin_ctx_size(B, S, E, E) bytes; may be NULL with ctx_bytes 0).
 * cxg_lin_hexp_bwd: dXq, dXk (B*S, E) with respect to the raw projections,
 * and dV.  E must be 64 (one Hadamard block; other widths: cxg_phi_hexp_*
 * around cxg_lin_fwd / cxg_lin_bwd) and S < 2^22; every row pointer 16-byte
 * aligned (CXG_ERR_ALIGN otherwise).  Sequences of at most 128 rows, which
 * the quadratic-form kernels take, run the feature-map kernels through the
 * library's scratch instead and use no context. */
int cxg_lin_hexp_fwd(const float *Xq, const float *Xk, const float *V, float *O,
                     float *den_cache, void *ctx, size_t ctx_bytes, size_t B, size_t S,
                     size_t E, cxg_stream_t stream);
int cxg_lin_hexp_bwd(const float *Xq, const float *Xk, const float *V, const float *O,
                     const float *dO, const float *den_cache, const void *ctx, float *dXq,
                     float *dXk, float *dV, size_t B, size_t S, size_t E, cxg_stream_t stream);

/* linear_cuda::phi_elu_forward / phi_elu_backward (linear_cuda_kernels.cuh:39-46,
 * linear_cuda_kernels.cu:305-378).  x (N, E) -> phi (N, D), columns >= E zero;
 * dx (N, E) = dphi[:, :E] * phi'(x). */
int cxg_phi_elu_fwd(const float *x, float *phi, size_t N, size_t D, size_t E,
                    cxg_stream_t stream);
int cxg_phi_elu_bwd(const float *dphi, const float *x, float *dx, size_t N, size_t D,
                    size_t E, cxg_stream_t stream);

/* Hadamard+Exp feature map.  No counterpart in the reference's code; it
 * plugs into the linear_cuda API the way phi_elu_* does (same argument
 * meaning).  phi[n, 64j+i] = exp((H_64 x[n, 64j:64j+64])_i / 8) with H_64 the
 * Sylvester Hadamard matrix; E % 64 == 0, D >= E, columns >= E zero.
 * Backward: dx = H_64 (dphi * phi(x)) / 8 per 64-block. */
int cxg_phi_hexp_fwd(const float *x, float *phi, size_t N, size_t D, size_t E,
                     cxg_stream_t stream);
int cxg_phi_hexp_bwd(const float *dphi, const float *x, float *dx, size_t N, size_t D,
                     size_t E, cxg_stream_t stream);

/* ===================== rotary position embedding =====================
 * two_stage_cuda::rope_fwd / rope_bwd (two_stage_cuda_kernels.cuh:72-76,
 * two_stage_cuda_kernels.cu:1810-1878), in place on (B*S, D) rows: pair i of
 * each head of width head_dim in a row at position p = row % S rotates by
 * +-p * 10000^(-2i/head_dim) (fwd +, bwd - = the inverse).  Either pointer
 * may be NULL (that tensor is skipped); Q == K rotates the buffer twice, as
 * the reference does.  head_dim even, 2..1024, D % head_dim == 0. */
int cxg_rope_fwd(float *Q, float *K, size_t B, size_t S, size_t D, size_t head_dim,
                 cxg_stream_t stream);
int cxg_rope_bwd(float *dQ, float *dK, size_t B, size_t S, size_t D, size_t head_dim,
                 cxg_stream_t stream);

/* ===================== per-kernel timing hook =====================
 * Off by default.  When on, each kernel launch is bracketed by HIP events on
 * its stream; cxg_prof_query synchronises them and returns the summed device
 * time (ms) and launch count for a kernel name ("mha_fwd", "mha_bwd", ...).
 * Returns 0 if the name was seen, -1 otherwise. */
void cxg_prof_enable(int on);
void cxg_prof_reset(void);
int cxg_prof_query(const char *kernel_name, double *total_ms, int *count);

/* two_stage_cuda::gelu_exact / gelu_exact_deriv (two_stage_cuda_kernels.cuh:84-85,
 * two_stage_cuda_kernels.cu:1888-1924): C = gelu(A) or gelu'(A) over n floats,
 * exact (erf) form; C may be A. */
int cxg_gelu_exact(const float *A, float *C, size_t n, cxg_stream_t stream);
int cxg_gelu_exact_deriv(const float *A, float *C, size_t n, cxg_stream_t stream);

/* The two-stage block's expander FFN: two bias-free Linear layers with the
 * exact GELU between them (two_stage_gpt.hpp:37-40; the call sequence
 * q_ffn_fc.forward -> gelu_exact -> q_ffn_proj.forward at :86-89, and the
 * same for k, v and the final FFN at :91-99, :126-129; Linear::forward /
 * backward at gpt_gpt.hpp:86-112).  Row-major X [M][E], W1 [F][E] (the fc
 * weight), W2 [E][F] (the proj weight); the reference's F is 4*N*n_embd.
 *   cxg_ffn_fwd:  pre = X W1^T (stored if pre != NULL, else not kept),
 *                 act = gelu(pre), Y = act W2^T.
 *   cxg_ffn_bwd:  dact = (dY W2) * gelu'(G); dW2 += dY^T act; dX = dact W1;
 *                 dW1 += dact^T X  (weight gradients accumulate, as Linear
 *                 does).  G is the tensor gelu' is evaluated at: the
 *                 reference's q/k/v expanders pass act (:179,187,195), its
 *                 final FFN the pre-activation (:141).
 * FP32 MFMA GEMMs with GELU / gelu' in their epilogues.  E and F multiples of
 * 4 and every tensor 16-byte aligned (else CXG_ERR_ALIGN); any M.  workspace
 * of cxg_ffn_workspace_size(M, E, F) bytes (fwd and bwd), or NULL for the
 * library's scratch. */
size_t cxg_ffn_workspace_size(size_t M, size_t E, size_t F);
int cxg_ffn_fwd(const float *X, const float *W1, const float *W2, float *pre, float *act,
                float *Y, size_t M, size_t E, size_t F, void *workspace, size_t ws_bytes,
                cxg_stream_t stream);
int cxg_ffn_bwd(const float *X, const float *W1, const float *W2, const float *act,
                const float *G, const float *dY, float *dX, float *dW1, float *dW2, size_t M,
                size_t E, size_t F, void *workspace, size_t ws_bytes, cxg_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* CXXGPT_ATTN_H */
