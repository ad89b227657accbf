// linquad.hip -- causal linear attention in the quadratic form with the block
// score matrices in scratch memory (gfx950, FP32 MFMA).
//
// Same algebra as linwide.hip (per sequence, 16-row blocks i, j):
//   A[t][s] = phi(Q_t) . phi(K_s)            (s <= t)
//   den_t = sum_s A[t][s],   O_t = (sum_s A[t][s] V_s) / (den_t + 1e-8)
//   G[t][s] = dnum_t . V_s + dden_t          (s <= t)
//   dQ_t = (sum_s G[t][s] phi(K_s)) * phi'(Q_t)
//   dK_s = (sum_t G[t][s] phi(Q_t)) * phi'(K_s)
//   dV_s = sum_t A[t][s] dnum_t
// the forms two_stage_cuda::kernel_attn_fwd / _bwd_dQ / _bwd_dKdV
// (src/TwoStage/two_stage_cuda_kernels.cu:988-1809) and
// linear_cuda::causal_linear_attention_fwd / _bwd_dQ / _bwd_dKdV
// (src/LinearAttention/linear_cuda_kernels.cu:10-298) compute with a running
// state.  linwide.hip gives each 16-row block to one workgroup that streams
// every other block of its sequence through LDS: at LinearGPT's shape (8
// sequences of 256 rows, D = E = 512) 256 jobs for 256 compute units whose 16
// block steps run one after another.  Here the work is cut into small
// independent jobs instead:
//   0. features Fq = phi(Q), Fk = phi(K) into scratch (ELU+1 maps; PHI_NONE
//      reads Q and K as they are; the RoPE map's callers pass its features);
//   1. scores: one workgroup per (sequence, pair of 32-row tiles) forms the
//      16x16 blocks A_ij and/or G_ij (j <= i), masked to s <= t, into scratch,
//      the rows staged through LDS a 32-column chunk at a time;
//   2. products: one wave per (sequence, block, 64-column slice of one
//      output) -- O and z_cache over the query blocks' keys, dQ likewise, dK
//      and dV over the key blocks' queries -- then the epilogue (1/(den +
//      1e-8), or phi' and the RoPE map's inverse rotation).
// Every job owns its outputs: no atomics, no ordering between workgroups.
// Scratch: B' * nb(nb+1)/2 blocks of 256 floats per score matrix (nb =
// ceil(S/16)) and the features; the path is taken when that fits
// kQsBudget.
#include "common.hpp"
#include "launch.hpp"
#include "linattn.hpp"
#include "linattn_dev.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace cxg {

constexpr size_t kQsBudget = (size_t)512 << 20;   // bytes of scratch the path may take

enum { QS_O = 0, QS_Z = 1, QS_DQ = 2, QS_DK = 3, QS_DV = 4 };

constexpr int kQsStages = 2;   // register stages of the product kernels' operand loads

struct QsArgs {
    const float* Fq;     // phi(Q) (or Q / the RoPE features)
    const float* Fk;     // phi(K)
    const float* V;
    const float* dnum;
    const float* dden;
    float* Ab;           // score blocks: [seq][pair][16 * 16], pair = i(i+1)/2 + j
    float* Gb;
    float* O;
    float* den;
    float* zc;
    float* dQ;
    float* dK;
    float* dV;
    const float* Qx;     // raw inputs for phi'
    const float* Kx;
    int S, D, E, Bq, nb, npairs;
    int ntp;             // pairs of 32-row tiles per sequence
    int den_eps;
    int units;           // product units (output slices) per (sequence, block)
    int nslD, nslE;      // 64-column slices of the widths
    int kinds;           // backward: 1 = dK, dV; 2 = dQ; 3 = both
    int norm;            // O divided by den + 1e-8 (linear attention; 0: P is normalised)
    // softmax attention (GPT's, one head of width E): scores are formed as
    // q . k * qk_scale (scale * log2 e, the exp2 domain); the backward takes
    // lse (natural log) and Di = rowsum(dO * O) per row and stores
    // dS = P (dP - Di) * sm_scale
    float qk_scale, sm_scale;
    const float* lse_in;
    const float* Di;
    float* lse_out;
};

__host__ __device__ inline int qs_slices(int W) { return (W + 63) / 64; }

// Raw buffer over a sequence's rows of width W: reads past the last row return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qs_rows(const float* X, long rb, int S, int W)
{
    return buf_rsrc_n(X + rb * W, (unsigned)((long)S * W * 4));
}

// Workgroup b's job among B' sequences of n jobs each (jobs numbered in the
// order they should start).  The dispatcher places workgroup b on XCD b % 8,
// and each XCD has its own L2: spread over all eight, every XCD would fetch
// nearly every row of every sequence.  So each XCD gets whole sequences
// (B' >= 8: sequences [x B'/8, (x+1) B'/8), their jobs interleaved in job
// order) or, with fewer sequences than XCDs, a share of one sequence (sequence
// floor(x B'/8), every m-th of its jobs, m = its XCD count).  False for the
// grid's spare slots (qs_grid rounds up).
__device__ __forceinline__ bool qs_xcd_job(int b, int Bq, int n, int& seq, int& job)
{
    const int x = b & 7, k = b >> 3;
    if (Bq >= 8) {
        const int s0 = x * Bq / 8, ns = (x + 1) * Bq / 8 - s0;
        job = k / ns;
        seq = s0 + k % ns;
        return job < n;
    }
    seq = x * Bq / 8;
    const int x0 = (8 * seq + Bq - 1) / Bq, x1 = (8 * (seq + 1) + Bq - 1) / Bq;
    job = (x - x0) + k * (x1 - x0);
    return job < n;
}

// ---------------------------------------------------------------------------
// phase 0: features (ELU+1 maps)
// ---------------------------------------------------------------------------
template <int PHI>
__global__ __launch_bounds__(256) void lin_qs_feat_kernel(const f4* __restrict__ Q,
                                                          const f4* __restrict__ K,
                                                          f4* __restrict__ Fq, f4* __restrict__ Fk,
                                                          long n4)
{
    // Q null: phi(K) only
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
        f4 k = K[i];
#pragma unroll
        for (int r = 0; r < 4; r++)
            k[r] = Phi<PHI>::f(k[r]);
        Fk[i] = k;
        if (Q != nullptr) {
            f4 q = Q[i];
#pragma unroll
            for (int r = 0; r < 4; r++)
                q[r] = Phi<PHI>::f(q[r]);
            Fq[i] = q;
        }
    }
}

// z_cache = inclusive column sums of phi(K) over each sequence's rows (the
// forwards that return it): workgroup = (sequence, 64-column slice), wave w
// of 16 walking a sixteenth of the rows twice (its column sums, then the
// running sums from the earlier waves' totals), lane = column, so every load
// and store is a row's 256 contiguous bytes.
constexpr int QS_ZC_WAVES = 16;

__global__ __launch_bounds__(64 * QS_ZC_WAVES) void lin_qs_zc_kernel(
    const float* __restrict__ Fk, float* __restrict__ zc, int S, int D, int nsl)
{
    __shared__ float tot[QS_ZC_WAVES][64];
    const int seq = (int)(blockIdx.x / (unsigned)nsl), sl = (int)(blockIdx.x % (unsigned)nsl);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = 64 * sl + lane;
    const bool cok = c < D;
    const long base = (long)seq * S * D + (cok ? c : 0);
    const int q = (S + QS_ZC_WAVES - 1) / QS_ZC_WAVES, r0 = min(S, w * q), r1 = min(S, r0 + q);
    float sum = 0.0f;
#pragma unroll 16
    for (int t = r0; t < r1; t++)
        sum += Fk[base + (long)t * D];
    tot[w][lane] = sum;
    __syncthreads();
    float z = 0.0f;
    for (int u = 0; u < w; u++)
        z += tot[u][lane];
#pragma unroll 16
    for (int t = r0; t < r1; t++) {
        z += Fk[base + (long)t * D];
        if (cok)
            zc[base + (long)t * D] = z;
    }
}

// ---------------------------------------------------------------------------
// phase 1: score blocks.  Workgroup = (sequence, pair of 32-row tiles J <= I);
// wave w forms block (2I + w/2, 2J + w%2) of it (blocks above the diagonal are
// formed and dropped).  The contraction runs in 32-column chunks staged in
// LDS by whole 128-byte rows (thread t: row t/8, columns 4(t%8)..+3 of the
// chunk), double-buffered, one barrier a chunk; a wave reads its operands
// from LDS as 16-byte pieces, lane (l16, g) taking row l16 of its block at
// columns 16h + 4g .. +3, the same k order for both operands, in two
// accumulation chains (h = 0, 1).  MODE: 1 = A, 2 = G, 3 = both.  Lane
// (l16, g), element r of a block <-> [t = 4g + r][s = l16].
// ---------------------------------------------------------------------------
constexpr int QS_TR = 32;            // score tile rows
constexpr int QS_KC = 32;            // contraction chunk (columns)
constexpr int QS_LD = QS_KC + 4;     // LDS row stride

__device__ __forceinline__ f4 qs_tile_dot(float (*xs)[2][QS_TR * QS_LD], const float* X1,
                                          const float* X2, long rb, int S, int W, int I, int J,
                                          int tid, int bi, int bj, int l16, int g)
{
    constexpr int NU = QS_KC / 32;   // 16-byte pieces a thread stages per operand and chunk
    const __amdgpu_buffer_rsrc_t b1 = qs_rows(X1, rb, S, W), b2 = qs_rows(X2, rb, S, W);
    const int sr = tid >> 3, sc = 4 * (tid & 7);
    const unsigned o1 = (unsigned)(((QS_TR * I + sr) * W + sc) * 4);
    const unsigned o2 = (unsigned)(((QS_TR * J + sr) * W + sc) * 4);
    const int nch = (W + QS_KC - 1) / QS_KC;
    auto fetch = [&](int c, f4 (&r1)[NU], f4 (&r2)[NU]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NU; u++) {
            const int col = QS_KC * c + 32 * u;
            const bool ok = col + sc < W;   // W % 16 == 0: whole 16-column groups
            const f4 v1 = buffer_load_f4(b1, o1 + (unsigned)(4 * col));
            const f4 v2 = buffer_load_f4(b2, o2 + (unsigned)(4 * col));
            r1[u] = ok ? v1 : f4zero();
            r2[u] = ok ? v2 : f4zero();
        }
    };
    f4 r1[NU], r2[NU];
    fetch(0, r1, r2);
    f4 c0 = f4zero(), c1 = f4zero();
    for (int c = 0; c < nch; c++) {
        float* s1 = xs[c & 1][0];
        float* s2 = xs[c & 1][1];
#pragma unroll
        for (int u = 0; u < NU; u++) {
            *reinterpret_cast<f4*>(&s1[sr * QS_LD + sc + 32 * u]) = r1[u];
            *reinterpret_cast<f4*>(&s2[sr * QS_LD + sc + 32 * u]) = r2[u];
        }
        if (c + 1 < nch)
            fetch(c + 1, r1, r2);
        __syncthreads();
        const float* pa = &s1[(16 * bi + l16) * QS_LD + 4 * g];
        const float* pb = &s2[(16 * bj + l16) * QS_LD + 4 * g];
#pragma unroll
        for (int h = 0; h < QS_KC / 16; h += 2) {
            const f4 a0 = *reinterpret_cast<const f4*>(pa + 16 * h);
            const f4 a1 = *reinterpret_cast<const f4*>(pa + 16 * h + 16);
            const f4 e0 = *reinterpret_cast<const f4*>(pb + 16 * h);
            const f4 e1 = *reinterpret_cast<const f4*>(pb + 16 * h + 16);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                c0 = mfma16(a0[r], e0[r], c0);
                c1 = mfma16(a1[r], e1[r], c1);
            }
        }
    }
    return c0 + c1;
}

// SM: 0 linear attention (A, G as above); 1 softmax forward (A = the scaled
// scores, exp2 domain, for lin_qs_softmax_kernel); 2 softmax backward (MODE 3:
// A = P = exp2(S - lse log2 e), G = dS).
template <int MODE, int SM = 0>
__global__ __launch_bounds__(256) void lin_qs_score_kernel(const QsArgs a)
{
    __shared__ __attribute__((aligned(16))) float xs[2][2][QS_TR * QS_LD];
    int seq, tp;
    if (!qs_xcd_job((int)blockIdx.x, a.Bq, a.ntp, seq, tp))
        return;   // the whole workgroup
    // tp = I(I+1)/2 + J
    int I = (int)((sqrtf(8.0f * (float)tp + 1.0f) - 1.0f) * 0.5f);
    while ((I + 1) * (I + 2) / 2 <= tp)
        I++;
    while (I * (I + 1) / 2 > tp)
        I--;
    const int J = tp - I * (I + 1) / 2;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int bi = w >> 1, bj = w & 1;
    const int i = 2 * I + bi, j = 2 * J + bj;
    const long rb = (long)seq * a.S;
    f4 sa = f4zero(), sg = f4zero();
    if (MODE & 1)
        sa = qs_tile_dot(xs, a.Fq, a.Fk, rb, a.S, a.D, I, J, tid, bi, bj, l16, g);
    if (MODE == 3)
        __syncthreads();   // the last chunk's buffers are read before they are refilled
    if (MODE & 2)
        sg = qs_tile_dot(xs, a.dnum, a.V, rb, a.S, a.E, I, J, tid, bi, bj, l16, g);
    if (j > i || i >= a.nb)
        return;
    const long blk = ((long)seq * a.npairs + i * (i + 1) / 2 + j) * 256;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int t = 16 * i + 4 * g + r, s = 16 * j + l16;
        const bool ok = s <= t && t < a.S;
        const int e = (4 * g + r) * 16 + l16;
        if constexpr (SM == 0) {
            if (MODE & 1)
                a.Ab[blk + e] = ok ? sa[r] : 0.0f;
            if (MODE & 2)
                a.Gb[blk + e] = ok ? sg[r] + a.dden[rb + min(t, a.S - 1)] : 0.0f;
        } else if constexpr (SM == 1) {
            a.Ab[blk + e] = ok ? sa[r] * a.qk_scale : 0.0f;
        } else {
            const long rt = rb + min(t, a.S - 1);
            const float p = ok ? fast_exp2(sa[r] * a.qk_scale - a.lse_in[rt] * kLog2e) : 0.0f;
            a.Ab[blk + e] = p;
            a.Gb[blk + e] = p * (sg[r] - a.Di[rt]) * a.sm_scale;
        }
    }
}

// Row softmax of the scaled score blocks of one (sequence, query block i) per
// workgroup: the blocks (i, 0..i) are consecutive in the packed layout; wave w
// takes blocks j = w, w+4, ..., lane (l16, g) reading row l16 at columns
// 4g..4g+3 of each.  Three passes, the first two combined across the waves
// through LDS: the row maximum, the sum of exp2(S - max), then P = exp2(S -
// max) / sum written over the scores (0 above the diagonal and in rows past
// S), and lse = (max + log2 sum) ln 2 when lse_out is given.
__global__ __launch_bounds__(256) void lin_qs_softmax_kernel(const QsArgs a)
{
    __shared__ float red[2][4][16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int seq = (int)(blockIdx.x / (unsigned)a.nb), i = (int)(blockIdx.x % (unsigned)a.nb);
    float* base = a.Ab + ((long)seq * a.npairs + (long)i * (i + 1) / 2) * 256 + l16 * 16 + 4 * g;
    const int t = 16 * i + l16;
    float m = -INFINITY;
    for (int j = w; j <= i; j += 4) {
        const f4 v = *reinterpret_cast<const f4*>(base + j * 256);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (16 * j + 4 * g + r <= t)
                m = fmaxf(m, v[r]);
    }
    m = xrow_max(m);
    if (g == 0)
        red[0][w][l16] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0][0][l16], red[0][1][l16]), fmaxf(red[0][2][l16], red[0][3][l16]));
    float l = 0.0f;   // every row has its diagonal entry, so m is finite
    for (int j = w; j <= i; j += 4) {
        const f4 v = *reinterpret_cast<const f4*>(base + j * 256);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (16 * j + 4 * g + r <= t)
                l += fast_exp2(v[r] - m);
    }
    l = xrow_sum(l);
    if (g == 0)
        red[1][w][l16] = l;
    __syncthreads();
    l = (red[1][0][l16] + red[1][1][l16]) + (red[1][2][l16] + red[1][3][l16]);
    const float inv = 1.0f / l;
    const bool rok = t < a.S;
    for (int j = w; j <= i; j += 4) {
        f4 v = *reinterpret_cast<const f4*>(base + j * 256);
#pragma unroll
        for (int r = 0; r < 4; r++)
            v[r] = (rok && 16 * j + 4 * g + r <= t) ? fast_exp2(v[r] - m) * inv : 0.0f;
        *reinterpret_cast<f4*>(base + j * 256) = v;
    }
    if (a.lse_out != nullptr && rok && w == 0 && g == 0)
        a.lse_out[(long)seq * a.S + t] = (m + fast_log2(l)) * kLn2;
}

// ---------------------------------------------------------------------------
// phase 2: products.  Unit = (kind, 64-column slice) of one (sequence, block),
// worked by `split` waves (1, 2 or 4, so that short launches still fill the
// SIMDs), wave part p taking block steps p, p + split, ..., with the loads of
// its next two steps in flight; the parts are summed through LDS.  A
// workgroup takes 4 / split consecutive units of one (sequence, step count
// L).  Query-side kinds (O, z_cache, dQ) run over key blocks j = 0..i,
// key-side kinds (dK, dV) over query blocks i = j..nb-1.  Results are
// transposed: MFMA q (q = 0..3) covers the output columns c0 + 4m + q,
// m = 0..15, so acc[q] element r is column c0 + 16g + 4r + q of row
// 16 blk + l16 and each lane ends with four 16-byte pieces of its own row.
// Per step: A operand X[16 b + 4g + r][c0 + 4 l16 + q] (X = V, phi(K), phi(Q)
// or dnum at block row b; one 16-byte load per r, so a load instruction reads
// 4 rows of 256 contiguous bytes), B operand the score block read by rows
// (query side: lane row l16, columns 4g + r) or by columns (key side: row
// 4g + r, column l16).
// ---------------------------------------------------------------------------
template <int PHI, bool BWD>
__global__ __launch_bounds__(256) void lin_qs_prod_kernel(const QsArgs a,
                                                          const LinRopeArg<PHI> rope, int split)
{
    __shared__ __attribute__((aligned(16))) float red[4][17 * 64];   // parts > 0: acc + dp
    __shared__ float rope_w[phi_rope(PHI) ? LIN_ROPE_MAX_D / 2 : 1];
    rope_tab_lds<PHI, LIN_ROPE_MAX_D / 2>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();   // the rope table
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    // heaviest units first: job = (nb - L) * groups + group for L block steps
    const int upw = 4 / split, groups = (a.units + upw - 1) / upw;
    int seq, job;
    if (!qs_xcd_job((int)blockIdx.x, a.Bq, a.nb * groups, seq, job))
        return;   // the whole workgroup
    const int L = a.nb - job / groups, unit = upw * (job % groups) + w / split;
    const int part = w % split;
    if (unit >= a.units) {
        if (split > 1)
            __syncthreads();   // the other units' reduction
        return;
    }
    int kind, sl;
    if (!BWD) {
        kind = unit < a.nslE ? QS_O : QS_Z;
        sl = unit < a.nslE ? unit : unit - a.nslE;
    } else {
        int u = unit;
        kind = -1;
        sl = 0;
        if (a.kinds & 2) {
            if (u < a.nslD) {
                kind = QS_DQ;
                sl = u;
            }
            u -= a.nslD;
        }
        if (kind < 0) {
            if (u < a.nslD) {
                kind = QS_DK;
                sl = u;
            } else {
                kind = QS_DV;
                sl = u - a.nslD;
            }
        }
    }
    const bool qside = kind == QS_O || kind == QS_Z || kind == QS_DQ;
    const int blk = qside ? L - 1 : a.nb - L;
    const int W = (kind == QS_O || kind == QS_DV) ? a.E : a.D;
    const float* X = kind == QS_O ? a.V : kind == QS_DK ? a.Fq : kind == QS_DV ? a.dnum : a.Fk;
    const float* Sb = (kind == QS_O || kind == QS_DV) ? a.Ab : a.Gb;
    const long rb = (long)seq * a.S;
    const int c0 = 64 * sl;
    const __amdgpu_buffer_rsrc_t bx = qs_rows(X, rb, a.S, W);
    const float* sbase = Sb != nullptr ? Sb + (long)seq * a.npairs * 256 : nullptr;

    f4 acc[4] = {f4zero(), f4zero(), f4zero(), f4zero()};
    float dp = 0.0f;   // O: this lane's partial row sum of A (row l16, columns 4g..4g+3)
    // step k: block row b of X and score block p
    auto load = [&](int k, f4 (&xa)[4], f4& sb) __attribute__((always_inline)) {
        const int b = qside ? k : blk + k;                 // key block (query side) / query block
        const int i = qside ? blk : b, j = qside ? b : blk;
        const unsigned xo = (unsigned)(((16 * b + 4 * g) * W + c0 + 4 * l16) * 4);
#pragma unroll
        for (int r = 0; r < 4; r++)
            xa[r] = buffer_load_f4(bx, xo + (unsigned)(r * W * 4));
        if (kind == QS_Z) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                sb[r] = (j < i || 4 * g + r <= l16) ? 1.0f : 0.0f;
        } else {
            const float* sp = sbase + (long)(i * (i + 1) / 2 + j) * 256;
            if (qside) {
                sb = *reinterpret_cast<const f4*>(sp + l16 * 16 + 4 * g);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    sb[r] = sp[(4 * g + r) * 16 + l16];
            }
        }
    };
    auto math = [&](const f4 (&xa)[4], const f4& sb) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                acc[q] = mfma16(xa[r][q], sb[r], acc[q]);
        dp += (sb[0] + sb[1]) + (sb[2] + sb[3]);
    };
    // The epilogue's phi' operands (dQ, dK units of the first part), requested
    // now so that they arrive during the block steps.
    const int row = 16 * blk + l16;
    const float* raw = kind == QS_DQ ? a.Qx : a.Kx;
    const float* fea = kind == QS_DQ ? a.Fq : a.Fk;
    const bool from_f = !phi_rope(PHI) && fea != raw;
    f4 xe[4] = {f4zero(), f4zero(), f4zero(), f4zero()};
    if (BWD && PHI != PHI_NONE && part == 0 && (kind == QS_DQ || kind == QS_DK)) {
        const __amdgpu_buffer_rsrc_t be = qs_rows(from_f ? fea : raw, rb, a.S, a.D);
#pragma unroll
        for (int r = 0; r < 4; r++)
            xe[r] = buffer_load_f4(be, (unsigned)((row * a.D + c0 + 16 * g + 4 * r) * 4));
    }
    // register stages: with three, step n + 2 is requested before step n's
    // products (steps part + split n, n < nk); with two, step n + 1
    const int nk = (L - part + split - 1) / split;
    auto ld = [&](int n, f4 (&xa)[4], f4& sb) __attribute__((always_inline)) {
        load(part + split * n, xa, sb);
    };
    if (nk > 0) {
        f4 x0[4], x1[4];
        f4 s0, s1;
        ld(0, x0, s0);
        if constexpr (kQsStages == 3) {
            f4 x2[4];
            f4 s2;
            if (nk > 1)
                ld(1, x1, s1);
            for (int n = 0;; n += 3) {
                if (n + 2 < nk)
                    ld(n + 2, x2, s2);
                math(x0, s0);
                if (n + 1 >= nk)
                    break;
                if (n + 3 < nk)
                    ld(n + 3, x0, s0);
                math(x1, s1);
                if (n + 2 >= nk)
                    break;
                if (n + 4 < nk)
                    ld(n + 4, x1, s1);
                math(x2, s2);
                if (n + 3 >= nk)
                    break;
            }
        } else {
            for (int n = 0;; n += 2) {
                if (n + 1 < nk)
                    ld(n + 1, x1, s1);
                math(x0, s0);
                if (n + 1 >= nk)
                    break;
                if (n + 2 < nk)
                    ld(n + 2, x0, s0);
                math(x1, s1);
                if (n + 2 >= nk)
                    break;
            }
        }
    }
    if (split > 1) {
        if (part > 0) {
#pragma unroll
            for (int q = 0; q < 4; q++)
                *reinterpret_cast<f4*>(&red[w][(4 * q) * 64 + lane * 4]) = acc[q];
            red[w][16 * 64 + lane] = dp;
        }
        __syncthreads();
        if (part > 0)
            return;
        for (int u = 1; u < split; u++) {
#pragma unroll
            for (int q = 0; q < 4; q++)
                acc[q] += *reinterpret_cast<const f4*>(&red[w + u][(4 * q) * 64 + lane * 4]);
            dp += red[w + u][16 * 64 + lane];
        }
    }
    // piece r: columns c0 + 16g + 4r .. +3 of this lane's row
    f4 out[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
        out[r] = f4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    if (kind == QS_O) {
        const float d = xrow_sum(dp);   // row l16's sum over every key
        if (row < a.S) {
            const float inv = a.norm ? 1.0f / (d + 1e-8f) : 1.0f;
            float* orow = a.O + (rb + row) * a.E;
#pragma unroll
            for (int r = 0; r < 4; r++)
                store4<true>(orow, c0 + 16 * g + 4 * r, a.E, out[r] * inv);
            if (a.norm && sl == 0 && g == 0)
                a.den[rb + row] = a.den_eps ? d + 1e-8f : d;
        }
        return;
    }
    if (row >= a.S)
        return;
    if (kind == QS_Z || kind == QS_DV) {
        float* orow = (kind == QS_Z ? a.zc + (rb + row) * a.D : a.dV + (rb + row) * a.E);
#pragma unroll
        for (int r = 0; r < 4; r++)
            store4<true>(orow, c0 + 16 * g + 4 * r, W, out[r]);
        return;
    }
    // dQ, dK: phi' (ELU+1 maps: min(phi, 1) from the features, which is
    // exp(x) for x <= 0 as phi is, or at the raw input where no features were
    // formed (the dQ-only backward's Q); the RoPE map: at the raw input, then
    // the inverse rotation); the operands were requested at the unit's start
    float* orow = (kind == QS_DQ ? a.dQ : a.dK) + (rb + row) * a.D;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int c = c0 + 16 * g + 4 * r;
        if (c < a.D) {
            f4 v = out[r];
            if constexpr (phi_rope(PHI)) {
                v = rope_phi_grad4<PHI>(v, xe[r], row, c, rope_w);
            } else if constexpr (PHI != PHI_NONE) {
                const f4 xv = xe[r];
                if (from_f) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        v[i] *= Phi<PHI>::d_from_f(xv[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        v[i] *= Phi<PHI>::d(xv[i]);
                }
            }
            *reinterpret_cast<f4*>(orow + c) = v;
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static size_t qs_al(size_t b) { return (b + 255) / 256 * 256; }

static bool qs_needs_feat(int phi) { return phi == PHI_ELU1 || phi == PHI_ELU1_LG; }

static long qs_npairs(int S)
{
    const long nb = (S + 15) / 16;
    return nb * (nb + 1) / 2;
}

// kinds: 0 forward (A); backward 1 = dK, dV (A, G), 2 = dQ (G), 3 = all (A, G)
static size_t qs_bytes(bool feat, int Bq, int S, int D, int kinds)
{
    const size_t N = (size_t)Bq * S;
    const size_t blocks = qs_al((size_t)Bq * qs_npairs(S) * 256 * sizeof(float));
    const int nmat = kinds == 0 ? 1 : kinds == 2 ? 1 : 2;
    return (feat ? 2 * qs_al(N * D * sizeof(float)) : 0) + nmat * blocks;
}

// Forward -> backward context of the path: phi(Q), phi(K) (ELU+1 maps; the
// RoPE map's callers put its features there) and the score blocks A.
struct QsCtx {
    float* fq;
    float* fk;
    float* ab;
};

static QsCtx qs_ctx_split(const void* ctx, int Bq, int S, int D)
{
    const size_t N = (size_t)Bq * S, t = qs_al(N * D * sizeof(float));
    char* c = (char*)const_cast<void*>(ctx);
    return QsCtx{(float*)c, (float*)(c + t), (float*)(c + 2 * t)};
}

size_t lin_qs_ctx_bytes(int Bq, int S, int D, int E)
{
    (void)E;
    const size_t N = (size_t)Bq * S;
    return 2 * qs_al(N * D * sizeof(float)) +
           qs_al((size_t)Bq * qs_npairs(S) * 256 * sizeof(float));
}

float* lin_qs_ctx_features(void* ctx, int Bq, int S, int D, int which)
{
    const QsCtx c = qs_ctx_split(ctx, Bq, S, D);
    return which == 0 ? c.fq : c.fk;
}

size_t lin_qs_bytes(int Bq, int S, int D, int E, int kinds)
{
    (void)E;
    return qs_bytes(true, Bq, S, D, kinds);
}

bool lin_qs_ok(int Bq, int S, int D, int E)
{
    if (Bq < 1 || S < 1 || D < 16 || E < 16 || D % 16 != 0 || E % 16 != 0)
        return false;
    const long nb = (S + 15) / 16;
    if ((long)S * std::max(D, E) * 4 >= (1L << 31) || (Bq + 8L) * qs_npairs(S) >= (1L << 31) ||
        nb * qs_slices(std::max(D, E)) * 3 * (Bq + 8L) >= (1L << 31))
        return false;
    return lin_qs_bytes(Bq, S, D, E, 3) <= kQsBudget;
}

static inline bool qs_al16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (cached per device).
static int qs_cus()
{
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 256;
    if (cus[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Grid of qs_xcd_job for B' sequences of n jobs each.
static unsigned qs_grid(int Bq, long n)
{
    if (Bq >= 8)
        return (unsigned)(8L * ((Bq + 7) / 8) * n);
    const long m = 8 / Bq;   // the fewest XCDs a sequence gets
    return (unsigned)(8L * ((n + m - 1) / m));
}

static QsArgs qs_base(int Bq, int S, int D, int E)
{
    QsArgs a{};
    a.norm = 1;
    a.S = S;
    a.D = D;
    a.E = E;
    a.Bq = Bq;
    a.nb = (S + 15) / 16;
    a.npairs = (int)qs_npairs(S);
    const int nt = (S + QS_TR - 1) / QS_TR;
    a.ntp = nt * (nt + 1) / 2;
    a.nslD = qs_slices(D);
    a.nslE = qs_slices(E);
    return a;
}

// Features into ws (ELU+1 maps) or the inputs as they are; returns the bytes
// of ws taken.
// need_q false: phi(K) only (the dQ-only backward); Fq then stays Q, unused.
// dst (nullable): a context's feature buffers instead of ws.
static size_t qs_features(int phi, const float* Q, const float* K, bool need_q, QsArgs& a,
                          char* ws, hipError_t& e, hipStream_t st, const QsCtx* dst = nullptr)
{
    a.Fq = Q;
    a.Fk = K;
    e = hipSuccess;
    if (!qs_needs_feat(phi))
        return 0;
    const size_t N = (size_t)a.Bq * a.S, t = qs_al(N * a.D * sizeof(float));
    float* fq = dst ? dst->fq : (float*)ws;
    float* fk = dst ? dst->fk : (float*)(ws + t);
    const long n4 = (long)(N * a.D / 4);
    const unsigned grid = (unsigned)std::min<long>((n4 + 255) / 256, 4096);
    ProfScope ps(st, "lin_qs_feat");
    const f4* q4 = need_q ? (const f4*)Q : nullptr;
    if (phi == PHI_ELU1)
        CXG_LAUNCH(lin_qs_feat_kernel<PHI_ELU1>, dim3(grid), dim3(256), 0, st, q4, (const f4*)K,
                   (f4*)fq, (f4*)fk, n4);
    else
        CXG_LAUNCH(lin_qs_feat_kernel<PHI_ELU1_LG>, dim3(grid), dim3(256), 0, st, q4,
                   (const f4*)K, (f4*)fq, (f4*)fk, n4);
    e = hipGetLastError();
    if (need_q)
        a.Fq = fq;
    a.Fk = fk;
    return dst ? 0 : 2 * t;
}

template <int MODE, int SM = 0>
static void qs_scores(const QsArgs& a, hipStream_t st)
{
    ProfScope ps(st, SM != 0 ? (SM == 1 ? "gpt_qs_score" : "gpt_qs_bscore")
                             : (MODE == 1 ? "lin_qs_score" : "lin_qs_bscore"));
    CXG_LAUNCH((lin_qs_score_kernel<MODE, SM>), dim3(qs_grid(a.Bq, a.ntp)), dim3(256), 0, st, a);
}

// Waves per product unit: the fewest that give every SIMD four waves (4 SIMDs
// per compute unit), at most 4.  The forward counts its O units only, so that
// O and den do not depend on whether z_cache is requested.
static int qs_split(const QsArgs& a, bool bwd)
{
    const long units = (long)a.Bq * a.nb * (bwd ? a.units : a.nslE), want = 4L * 4 * qs_cus();
    return units >= want ? 1 : 2 * units >= want ? 2 : 4;
}

template <int PHI, bool BWD>
static void qs_prod(const QsArgs& a, int D, hipStream_t st)
{
    ProfScope ps(st, a.norm ? (BWD ? "lin_qs_grad" : "lin_qs_out")
                            : (BWD ? "gpt_qs_grad" : "gpt_qs_out"));
    const LinRopeArg<PHI> rope = lin_rope_arg<PHI>(D);
    const int split = qs_split(a, BWD), upw = 4 / split;
    CXG_LAUNCH((lin_qs_prod_kernel<PHI, BWD>),
               dim3(qs_grid(a.Bq, (long)a.nb * ((a.units + upw - 1) / upw))), dim3(256), 0, st, a,
               rope, split);
}

hipError_t lin_qs_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                             float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                             void* ws, hipStream_t st, void* ctx)
{
    if ((ws == nullptr && ctx == nullptr) || !lin_qs_ok(Bq, S, D, E) || phi_rope(phi) ||
        phi == PHI_HEXP || !qs_al16(Q) || !qs_al16(K) || !qs_al16(V) || !qs_al16(O) ||
        !qs_al16(zc))
        return hipErrorInvalidValue;
    QsArgs a = qs_base(Bq, S, D, E);
    hipError_t e;
    if (ctx != nullptr) {   // features and score blocks into the context
        const QsCtx c = qs_ctx_split(ctx, Bq, S, D);
        qs_features(phi, Q, K, true, a, nullptr, e, st, &c);
        a.Ab = c.ab;
    } else {
        char* p = (char*)ws;
        p += qs_features(phi, Q, K, true, a, p, e, st);
        a.Ab = (float*)p;
    }
    if (e != hipSuccess)
        return e;
    a.V = V;
    a.O = O;
    a.den = den;
    a.zc = nullptr;   // z_cache: lin_qs_zc_kernel below
    a.den_eps = den_eps;
    a.units = a.nslE;
    qs_scores<1>(a, st);
    qs_prod<PHI_NONE, false>(a, D, st);
    if (zc != nullptr) {
        ProfScope ps(st, "lin_qs_zc");
        CXG_LAUNCH(lin_qs_zc_kernel, dim3((unsigned)((long)Bq * a.nslD)),
                   dim3(64 * QS_ZC_WAVES), 0, st, a.Fk, zc, S, D, a.nslD);
    }
    return hipGetLastError();
}

// with_a: A is already in a.Ab (the forward's context): G only.
template <int PHI>
static void qs_bwd_t(const QsArgs& a, int D, bool with_a, hipStream_t st)
{
    if (a.kinds == 2 || with_a)
        qs_scores<2>(a, st);
    else
        qs_scores<3>(a, st);
    qs_prod<PHI, true>(a, D, st);
}

hipError_t lin_qs_bwd_launch(int phi, const float* Q, const float* K, const float* V,
                             const float* dnum, const float* dden, float* dQ, float* dK,
                             float* dV, int Bq, int S, int D, int E, int kinds, void* ws,
                             hipStream_t st, const float* Qx, const float* Kx, const void* ctx)
{
    if (ws == nullptr || !lin_qs_ok(Bq, S, D, E) || phi == PHI_HEXP || kinds < 1 || kinds > 3 ||
        (phi_rope(phi) && D > LIN_ROPE_MAX_D) || (ctx != nullptr && kinds != 3))
        return hipErrorInvalidValue;
    if (!qs_al16(Q) || !qs_al16(K) || !qs_al16(V) || !qs_al16(dnum) || !qs_al16(dQ) ||
        !qs_al16(dK) || !qs_al16(dV) || !qs_al16(Qx) || !qs_al16(Kx))
        return hipErrorInvalidValue;
    QsArgs a = qs_base(Bq, S, D, E);
    hipError_t e = hipSuccess;
    char* p = (char*)ws;
    if (ctx != nullptr) {
        // the forward's features (ELU+1 maps) and score blocks A
        const QsCtx c = qs_ctx_split(ctx, Bq, S, D);
        a.Fq = qs_needs_feat(phi) ? c.fq : Q;
        a.Fk = qs_needs_feat(phi) ? c.fk : K;
        a.Ab = c.ab;
        a.Gb = (float*)p;
    } else {
        p += qs_features(phi, Q, K, kinds != 2, a, p, e, st);
        if (e != hipSuccess)
            return e;
        const size_t blocks = qs_al((size_t)Bq * a.npairs * 256 * sizeof(float));
        a.Gb = (float*)p;
        a.Ab = kinds == 2 ? nullptr : (float*)(p + blocks);
    }
    a.V = V;
    a.dnum = dnum;
    a.dden = dden;
    a.dQ = dQ;
    a.dK = dK;
    a.dV = dV;
    a.Qx = Qx != nullptr ? Qx : Q;
    a.Kx = Kx != nullptr ? Kx : K;
    a.kinds = kinds;
    a.units = ((kinds & 2) ? a.nslD : 0) + ((kinds & 1) ? a.nslD + a.nslE : 0);
    if (phi == PHI_ELU1)
        qs_bwd_t<PHI_ELU1>(a, D, ctx != nullptr, st);
    else if (phi == PHI_ELU1_LG)
        qs_bwd_t<PHI_ELU1_LG>(a, D, ctx != nullptr, st);
    else if (phi == PHI_ELU1_ROPE)
        qs_bwd_t<PHI_ELU1_ROPE>(a, D, ctx != nullptr, st);
    else
        qs_bwd_t<PHI_NONE>(a, D, ctx != nullptr, st);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GPT's attention (softmax, one head of width E) through the same blocks
// ---------------------------------------------------------------------------
static bool qs_gpt_forced_mat()
{
    const char* v = getenv("CXXGPT_GPT_PATH");
    return v != nullptr && strcmp(v, "mat") == 0;
}

bool gpt_qs_ok(int B, int S, int E)
{
    return !qs_gpt_forced_mat() && lin_qs_ok(B, S, E, E);
}

// forward: the score blocks; backward: P and dS blocks, Di and lse rows
size_t gpt_qs_ws_bytes(int B, int S, int E, bool bwd)
{
    (void)E;
    const size_t blocks = qs_al((size_t)B * qs_npairs(S) * 256 * sizeof(float));
    const size_t rows = qs_al((size_t)B * S * sizeof(float));
    return bwd ? 2 * blocks + 2 * rows : blocks;
}

static QsArgs gpt_args(const float* Q, const float* K, const float* V, int B, int S, int E)
{
    QsArgs a = qs_base(B, S, E, E);
    a.Fq = Q;
    a.Fk = K;
    a.V = V;
    a.norm = 0;
    const float scale = 1.0f / sqrtf((float)E);
    a.qk_scale = scale * kLog2e;
    a.sm_scale = scale;
    return a;
}

hipError_t gpt_qs_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                             float* lse, int B, int S, int E, void* ws, hipStream_t st)
{
    if (ws == nullptr || !lin_qs_ok(B, S, E, E) || !qs_al16(Q) || !qs_al16(K) || !qs_al16(V) ||
        !qs_al16(O))
        return hipErrorInvalidValue;
    QsArgs a = gpt_args(Q, K, V, B, S, E);
    a.Ab = (float*)ws;
    a.O = O;
    a.lse_out = lse;
    a.units = a.nslE;
    qs_scores<1, 1>(a, st);
    {
        ProfScope ps(st, "gpt_qs_softmax");
        CXG_LAUNCH(lin_qs_softmax_kernel, dim3((unsigned)((long)B * a.nb)), dim3(256), 0, st,
                   a);
    }
    if (O != nullptr)
        qs_prod<PHI_NONE, false>(a, E, st);
    return hipGetLastError();
}

hipError_t gpt_qs_bwd_launch(const float* Q, const float* K, const float* V, const float* O,
                             const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                             int B, int S, int E, void* ws, hipStream_t st)
{
    if (ws == nullptr || !lin_qs_ok(B, S, E, E) || !qs_al16(Q) || !qs_al16(K) || !qs_al16(V) ||
        !qs_al16(dO) || !qs_al16(dQ) || !qs_al16(dK) || !qs_al16(dV))
        return hipErrorInvalidValue;
    const size_t blocks = qs_al((size_t)B * qs_npairs(S) * 256 * sizeof(float));
    const size_t rows = qs_al((size_t)B * S * sizeof(float));
    char* p = (char*)ws;
    float* Ab = (float*)p;
    float* Gb = (float*)(p + blocks);
    float* Di = (float*)(p + 2 * blocks);
    float* lse_ws = (float*)(p + 2 * blocks + rows);
    hipError_t e;
    if (lse == nullptr) {   // the forward's statistics again
        e = gpt_qs_fwd_launch(Q, K, V, nullptr, lse_ws, B, S, E, Ab, st);
        if (e != hipSuccess)
            return e;
        lse = lse_ws;
    }
    e = mha_bwd_prep_launch(O, dO, Di, nullptr, B, S, 1, E, st);
    if (e != hipSuccess)
        return e;
    QsArgs a = gpt_args(Q, K, V, B, S, E);
    a.Ab = Ab;
    a.Gb = Gb;
    a.dnum = dO;
    a.lse_in = lse;
    a.Di = Di;
    a.dQ = dQ;
    a.dK = dK;
    a.dV = dV;
    a.Qx = Q;
    a.Kx = K;
    a.kinds = 3;
    a.units = 2 * a.nslD + a.nslE;
    qs_scores<3, 2>(a, st);
    qs_prod<PHI_NONE, true>(a, E, st);
    return hipGetLastError();
}

}  // namespace cxg
