// linwide.hip -- causal linear attention for wide heads (64 < D, E <= 512),
// gfx950, FP32 MFMA, in the quadratic ("parallel") form.
//
// Replaces, for feature widths above 64, the per-timestep scans of
//   two_stage_cuda::kernel_attn_fwd / _bwd_dQ / _bwd_dKdV
//     (src/TwoStage/two_stage_cuda_kernels.cu:988-1809), phi = ELU+1 fused, and
//   linear_cuda::causal_linear_attention_fwd / _bwd_dQ / _bwd_dKdV
//     (src/LinearAttention/linear_cuda_kernels.cu:10-298), phi applied outside.
// The reference's callers run these at D = E = n_embd = 512 (TwoStageGPT's
// stage 2, two_stage_train.cpp:168-170; LinearGPT, linear_train.cpp:168-172)
// with S = block_size = 256.
//
// Why the quadratic form.  The recurrence carries a D x E state: per token it
// costs 2 D E multiply-adds forward (state product and update) and about
// 5 D E backward.  Written as a masked product instead,
//   A[t][s] = phi(Q_t) . phi(K_s)  (s <= t),   den_t = sum_s A[t][s],
//   O_t = (sum_s A[t][s] V_s) / (den_t + 1e-8),
// it costs about (t + 1)(D + E) per token: at S = 256, D = E = 512 a quarter of
// the recurrence's work, and no state has to be scanned across segments.  It
// is cheaper whenever S < 2D; at the reference's shapes S <= D.
// The backward, with dnum = dO / den and dden = -(dO . O) / den (step 1):
//   G[t][s] = dnum_t . V_s + dden_t                      (s <= t)
//   dQ_t = (sum_s G[t][s] phi(K_s)) * phi'(Q_t)
//   dK_s = (sum_t G[t][s] phi(Q_t)) * phi'(K_s)
//   dV_s = sum_t A[t][s] dnum_t
// which is the recurrence's dQ = (z dden + S dnum) phi', dK = (z* + S* V) phi',
// dV = S*^T phi(K) with the sums over s and t taken in the other order.
// z_cache (inclusive cumsum of phi(K)) is not needed by this dQ; the APIs that
// write it get it from lin_zc_kernel.
//
// Layout.  A workgroup of NW waves (NW = 2, 4, 8 for widths up to 128, 256,
// 512) works on 16-row blocks; wave w owns feature columns 64w .. 64w+63 of
// Q/K (for the score partials and dQ/dK) and of V/O (for O, dV).  A 16x16
// score block is NW partial products summed through LDS.  Scores are formed
// transposed where a lane owns a query row (forward, dQ jobs) and plainly
// where it owns a key (dK/dV jobs).  Streamed blocks are staged in LDS with
// 16-byte row loads, fetched one block ahead into registers.
#include "common.hpp"
#include "launch.hpp"
#include "linattn.hpp"
#include "linattn_dev.hpp"

#include <algorithm>

namespace cxg {

constexpr int LWB = 16;   // rows per block

template <int NW>
struct LW {
    static constexpr int DP = 64 * NW;        // padded feature width
    static constexpr int LD = DP + 4;          // LDS row stride of a staged block
    static constexpr int T = 64 * NW;          // threads
    static constexpr int U = LWB * DP / 4 / T; // 16-byte units of a block per thread (4)
    static constexpr int TILE = LWB * LD;      // floats per staged block
};

template <int NW>
struct LwRegs {
    f4 v[LW<NW>::U];
};

// Rows [r0, r0+16) x [0, n) of a (rows, ld) matrix; rows past S repeat row S-1
// (clamped), columns past n read a clamped copy (zeroed when stored).
template <int NW, bool VEC>
__device__ __forceinline__ void lw_fetch(LwRegs<NW>& R, const float* __restrict__ base, int ld,
                                         int r0, int S, int n, int tid)
{
    constexpr int UPR = LW<NW>::DP / 4;   // units per row
#pragma unroll
    for (int k = 0; k < LW<NW>::U; k++) {
        const int u = tid + LW<NW>::T * k;
        const int row = u / UPR, c = 4 * (u % UPR);
        R.v[k] = load4c<VEC>(base + (long)min(r0 + row, S - 1) * ld, c, n);
    }
}

// Store a fetched block to LDS, applying phi (APPLY) and zeroing columns >= n.
template <int NW, int PHI, bool APPLY>
__device__ __forceinline__ void lw_store(float* __restrict__ dst, const LwRegs<NW>& R, int n,
                                         int tid)
{
    static_assert(!phi_rope(PHI), "RoPE maps stream features (lin_rope_feat_kernel)");
    constexpr int UPR = LW<NW>::DP / 4;
#pragma unroll
    for (int k = 0; k < LW<NW>::U; k++) {
        const int u = tid + LW<NW>::T * k;
        const int row = u / UPR, c = 4 * (u % UPR);
        f4 v = R.v[k];
        if (APPLY && PHI != PHI_NONE)
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[i] = Phi<PHI>::f(v[i]);
        *reinterpret_cast<f4*>(&dst[row * LW<NW>::LD + c]) = mask4(v, c, n, true);
    }
}

// ---------------------------------------------------------------------------
// forward: job = (sequence, 16-query block, part), latest blocks first (they
// see the most keys).  A part is a run of at most PL key blocks; with PL >= the
// block count every job is one whole query block (the sums over keys are
// plain, so a query block split into parts is finished by adding the parts'
// numerators and denominators: lin_wide_fin_kernel).  Per key block: A^T[j][i]
// (lane i = query, element r <-> key 4g + r) from the waves' column partials,
// den_i += sum_j A[i][j], and over the wave's V columns
// O^T[e][i] += sum_j V[j][e] A^T[j][i].
// ---------------------------------------------------------------------------
template <int PHI, int NW, bool VEC>
__global__ __launch_bounds__(64 * NW) void lin_wide_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ den, float* __restrict__ zc, int S, int D, int E,
    int Bq, int den_eps, int PL, int PMAX, float* __restrict__ wsO, float* __restrict__ wsD)
{
    using P = LW<NW>;
    __shared__ __attribute__((aligned(16))) float lds[4 * P::TILE + NW * 256];
    float* Sp = lds + 4 * P::TILE;   // score partials [wave][lane * 4 + r]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int nqb = (S + LWB - 1) / LWB;
    const int unit = (int)(blockIdx.x / Bq);
    const int qb = nqb - 1 - unit / PMAX, part = unit % PMAX;
    const int nparts = (qb + PL) / PL;   // parts of this query block
    if (part >= nparts)
        return;   // the whole workgroup: no barrier is skipped
    const int kb0 = part * PL, kb1 = min(kb0 + PL, qb + 1);
    const int seq = (int)(blockIdx.x % Bq);
    const long rb = (long)seq * S;
    const int q0 = qb * LWB, c0 = 64 * w;
    const int qi = q0 + l16;   // this lane's query row

    // this wave's column slice of phi(Q) rows q0 + l16 (B operand)
    f4 q[4], o[4];
    {
        const float* qrow = Q + (rb + min(qi, S - 1)) * D;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int c = c0 + 16 * t + 4 * g;
            f4 v = load4c<VEC>(qrow, c, D);
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[i] = Phi<PHI>::f(v[i]);
            q[t] = mask4(v, c, D, true);
            o[t] = f4zero();
        }
    }
    float dsum = 0.0f;
    // z_cache (zc != null, whole query blocks only): column sums of phi(K)
    // over the key blocks before this query block, columns c0 + 16t + l16
    // (each lane's own column)
    float zrun[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    // A^T partial of key block kb over this wave's columns (two accumulation
    // chains) to Sp, and z_cache from the block's phi(K) columns
    auto scores = [&](const float* __restrict__ Ks, int kb) __attribute__((always_inline)) {
        f4 sp = f4zero(), sp2 = f4zero();
#pragma unroll
        for (int t = 0; t < 4; t += 2) {
            const f4 kv = *reinterpret_cast<const f4*>(&Ks[l16 * P::LD + c0 + 16 * t + 4 * g]);
            const f4 kv2 = *reinterpret_cast<const f4*>(&Ks[l16 * P::LD + c0 + 16 * t + 16 + 4 * g]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sp = mfma16(kv[r], q[t][r], sp);
                sp2 = mfma16(kv2[r], q[t + 1][r], sp2);
            }
        }
        *reinterpret_cast<f4*>(&Sp[w * 256 + lane * 4]) = sp + sp2;
        if (zc != nullptr) {
            // z_t = zrun + inclusive prefix within the query block (the last key
            // block); rows 4g + r of this lane's columns
#pragma unroll
            for (int t = 0; t < 4; t++) {
                f4 col;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    col[r] = Ks[(4 * g + r) * P::LD + c0 + 16 * t + l16];
                float tot;
                const f4 zp = col_prefix16(col, tot, lane) + zrun[t];
                zrun[t] += tot;
                const int c = c0 + 16 * t + l16;
                if (kb == qb && c < D)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (q0 + 4 * g + r < S)
                            zc[(rb + q0 + 4 * g + r) * D + c] = zp[r];
            }
        }
    };
    // the waves' partials summed and masked, den, and O^T[e][i] += sum_j
    // V[j][e] A^T[j][i] over this wave's columns
    auto accumulate = [&](const float* __restrict__ Vs, int kb) __attribute__((always_inline)) {
        const int k0 = kb * LWB;
        f4 a = f4zero();
#pragma unroll
        for (int u = 0; u < NW; u++)
            a += *reinterpret_cast<const f4*>(&Sp[u * 256 + lane * 4]);
        float aloc = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int kj = k0 + 4 * g + r;
            a[r] = (kj <= qi && kj < S) ? a[r] : 0.0f;
            aloc += a[r];
        }
        dsum += xrow_sum(aloc);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            f4 acc = o[t];
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(Vs[(4 * g + r) * P::LD + c0 + 16 * t + l16], a[r], acc);
            o[t] = acc;
        }
    };
    LwRegs<NW> kr, vr;
    lw_fetch<NW, VEC>(kr, K + rb * D, D, kb0 * LWB, S, D, tid);
    lw_fetch<NW, VEC>(vr, V + rb * E, E, kb0 * LWB, S, E, tid);
    // two LDS copies: block kb goes to copy (kb - kb0) & 1 at the top of its
    // step, and the register stage is refilled with block kb+1 (the last step
    // refetches its own block)
    for (int kb = kb0; kb < kb1; kb++) {
        float* Ks = lds + ((kb - kb0) & 1) * 2 * P::TILE;
        float* Vs = Ks + P::TILE;
        lw_store<NW, PHI, true>(Ks, kr, D, tid);
        lw_store<NW, PHI, false>(Vs, vr, E, tid);
        __builtin_amdgcn_sched_barrier(0);
        const int kn = min(kb + 1, kb1 - 1) * LWB;
        lw_fetch<NW, VEC>(kr, K + rb * D, D, kn, S, D, tid);
        lw_fetch<NW, VEC>(vr, V + rb * E, E, kn, S, E, tid);
        __syncthreads();
        scores(Ks, kb);
        __syncthreads();
        accumulate(Vs, kb);
        // Sp and this copy are rewritten after a later step's first barrier;
        // the reads above come before it
    }
    if (qi < S) {
        if (nparts == 1) {
            const float inv = 1.0f / (dsum + 1e-8f);
            float* orow = O + (rb + qi) * E;
#pragma unroll
            for (int t = 0; t < 4; t++)
                store4<VEC>(orow, c0 + 16 * t + 4 * g, E, o[t] * inv);
            if (w == 0 && g == 0)
                den[rb + qi] = den_eps ? dsum + 1e-8f : dsum;
        } else {
            // this part's numerator and denominator
            const long N = (long)Bq * S;
            float* orow = wsO + ((long)part * N + rb + qi) * E;
#pragma unroll
            for (int t = 0; t < 4; t++)
                store4<VEC>(orow, c0 + 16 * t + 4 * g, E, o[t]);
            if (w == 0 && g == 0)
                wsD[(long)part * N + rb + qi] = dsum;
        }
    }
}

// Rows of the query blocks split into parts: O = (sum of the parts'
// numerators) / (sum of their denominators + 1e-8), den as the forward.  One
// thread per element; parts are added in order.
__global__ __launch_bounds__(256) void lin_wide_fin_kernel(
    const float* __restrict__ wsO, const float* __restrict__ wsD, float* __restrict__ O,
    float* __restrict__ den, int S, int E, int Bq, int PL, int den_eps)
{
    const long N = (long)Bq * S;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= N * E)
        return;
    const long row = i / E;
    const int c = (int)(i - row * E);
    const int qb = (int)(row % S) / LWB;
    const int nparts = (qb + PL) / PL;
    if (nparts == 1)
        return;
    float num = 0.0f, ds = 0.0f;
    for (int p = 0; p < nparts; p++) {
        num += wsO[((long)p * N + row) * E + c];
        ds += wsD[(long)p * N + row];
    }
    O[row * E + c] = num / (ds + 1e-8f);
    if (c == 0)
        den[row] = den_eps ? ds + 1e-8f : ds;
}

// ---------------------------------------------------------------------------
// backward: job kinds selected by `kinds` (1: key jobs, 2: query jobs, 3: both,
// interleaved longest first).
//  * key job (sequence, key block kb): for every query block from kb on,
//    A[i][j] and X[i][j] = dnum_i . V_j (lane j = key, element r <-> query
//    4g + r), G = X + dden_i; over the wave's columns dK^T += phi(Q)^T G and
//    dV^T += dnum^T A; dK * phi'(K) and dV stored at the end.
//  * query job (sequence, query block qb): for every key block up to qb, X^T
//    (lane i = query), G^T = X^T + dden_i, dQ^T += phi(K)^T G^T; dQ * phi'(Q)
//    stored at the end.
// LDS tiles: T0 phi(K), T1 V (a key job's own, a query job's streamed), T2
// phi(Q), T3 dnum (a key job's streamed; T3 a query job's own).
// ---------------------------------------------------------------------------
template <int PHI, int NW, bool VEC>
__global__ __launch_bounds__(64 * NW) void lin_wide_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dnum, const float* __restrict__ dden, float* __restrict__ dQ,
    float* __restrict__ dK, float* __restrict__ dV, int S, int D, int E, int Bq, int kinds,
    const float* __restrict__ Qx, const float* __restrict__ Kx, const LinRopeArg<PHI> rope)
{
    // RoPE maps: Q and K are the features phi(rot(x)) (lin_rope_feat_kernel),
    // streamed as they are; Qx, Kx the raw inputs, for phi' and the inverse
    // rotation of dQ, dK at the end.  Other maps: Qx = Q, Kx = K.
    constexpr int PS = phi_rope(PHI) ? PHI_NONE : PHI;   // the map applied to streamed rows
    using P = LW<NW>;
    __shared__ __attribute__((aligned(16))) float lds[4 * P::TILE + 2 * NW * 256 + LWB];
    __shared__ float rope_w[phi_rope(PHI) ? 32 * NW : 1];
    rope_tab_lds<PHI, 32 * NW>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();
    float* Ks = lds;
    float* Vs = Ks + P::TILE;
    float* Qs = Vs + P::TILE;
    float* Ns = Qs + P::TILE;
    float* Sp = Ns + P::TILE;         // [wave][A, X][lane * 4 + r]
    float* dd = Sp + 2 * NW * 256;    // dden of the current query block
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int nb = (S + LWB - 1) / LWB;
    const int ent = (int)(blockIdx.x / Bq);
    const int seq = (int)(blockIdx.x % Bq);
    int L, kjob;
    if (kinds == 3) {
        L = nb - ent / 2;
        kjob = (ent & 1) == 0;
    } else {
        L = nb - ent;
        kjob = kinds == 1;
    }
    const int blk = kjob ? nb - L : L - 1;   // key job: key block; query job: query block
    const long rb = (long)seq * S;
    const int x0 = blk * LWB, c0 = 64 * w;
    // the job's own tiles
    if (kjob) {
        LwRegs<NW> t;
        lw_fetch<NW, VEC>(t, K + rb * D, D, x0, S, D, tid);
        lw_store<NW, PS, true>(Ks, t, D, tid);
        lw_fetch<NW, VEC>(t, V + rb * E, E, x0, S, E, tid);
        lw_store<NW, PS, false>(Vs, t, E, tid);
    } else {
        LwRegs<NW> t;
        lw_fetch<NW, VEC>(t, dnum + rb * E, E, x0, S, E, tid);
        lw_store<NW, PS, false>(Ns, t, E, tid);
        if (tid < LWB)
            dd[tid] = dden[rb + min(x0 + tid, S - 1)];
    }
    f4 acc1[4], acc2[4];   // key job: dK^T, dV^T; query job: dQ^T (acc1)
#pragma unroll
    for (int t = 0; t < 4; t++) {
        acc1[t] = f4zero();
        acc2[t] = f4zero();
    }
    const int sbeg = kjob ? blk : 0, send = kjob ? nb : blk + 1;
    // streamed blocks: phi(Q), dnum, dden (key job) or phi(K), V (query job)
    const float* s1 = kjob ? Q + rb * D : K + rb * D;
    const float* s2 = kjob ? dnum + rb * E : V + rb * E;
    const int n1 = D, n2 = E;
    float* d1 = kjob ? Qs : Ks;
    float* d2 = kjob ? Ns : Vs;
    LwRegs<NW> r1, r2;
    lw_fetch<NW, VEC>(r1, s1, kjob ? D : D, sbeg * LWB, S, n1, tid);
    lw_fetch<NW, VEC>(r2, s2, E, sbeg * LWB, S, n2, tid);
    float ddn = (kjob && tid < LWB) ? dden[rb + min(sbeg * LWB + tid, S - 1)] : 0.0f;
    for (int sb = sbeg; sb < send; sb++) {
        const int y0 = sb * LWB;
        lw_store<NW, PS, true>(d1, r1, n1, tid);
        lw_store<NW, PS, false>(d2, r2, n2, tid);
        if (kjob && tid < LWB)
            dd[tid] = ddn;
        __builtin_amdgcn_sched_barrier(0);
        const int yn = min(sb + 1, send - 1) * LWB;   // the last step refetches its own block
        lw_fetch<NW, VEC>(r1, s1, D, yn, S, n1, tid);
        lw_fetch<NW, VEC>(r2, s2, E, yn, S, n2, tid);
        if (kjob && tid < LWB)
            ddn = dden[rb + min(yn + tid, S - 1)];
        __syncthreads();
        // key job: A, X (lane = key); query job: X^T (lane = query)
        f4 ap = f4zero(), xp = f4zero();
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int c = c0 + 16 * t + 4 * g;
            const f4 na = *reinterpret_cast<const f4*>(&Ns[l16 * P::LD + c]);
            const f4 va = *reinterpret_cast<const f4*>(&Vs[l16 * P::LD + c]);
            if (kjob) {
                const f4 qa = *reinterpret_cast<const f4*>(&Qs[l16 * P::LD + c]);
                const f4 ka = *reinterpret_cast<const f4*>(&Ks[l16 * P::LD + c]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    ap = mfma16(qa[r], ka[r], ap);
                    xp = mfma16(na[r], va[r], xp);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    xp = mfma16(va[r], na[r], xp);
            }
        }
        if (kjob)
            *reinterpret_cast<f4*>(&Sp[(2 * w) * 256 + lane * 4]) = ap;
        *reinterpret_cast<f4*>(&Sp[(2 * w + 1) * 256 + lane * 4]) = xp;
        __syncthreads();
        f4 a = f4zero(), x = f4zero();
#pragma unroll
        for (int u = 0; u < NW; u++) {
            if (kjob)
                a += *reinterpret_cast<const f4*>(&Sp[(2 * u) * 256 + lane * 4]);
            x += *reinterpret_cast<const f4*>(&Sp[(2 * u + 1) * 256 + lane * 4]);
        }
        const int q0 = kjob ? y0 : x0, k0 = kjob ? x0 : y0;
        f4 gg;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qo = kjob ? 4 * g + r : l16;   // query row within its block
            const int kj = k0 + (kjob ? l16 : 4 * g + r);
            const int qi = q0 + qo;
            const bool ok = kj <= qi && qi < S && kj < S;
            a[r] = ok ? a[r] : 0.0f;
            gg[r] = ok ? x[r] + dd[qo] : 0.0f;
        }
        if (kjob) {
            // dK^T[d][j] += sum_i phi(Q)[i][d] G[i][j];  dV^T[e][j] += sum_i dnum[i][e] A[i][j]
#pragma unroll
            for (int t = 0; t < 4; t++) {
                f4 ak = acc1[t], av = acc2[t];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int e = (4 * g + r) * P::LD + c0 + 16 * t + l16;
                    ak = mfma16(Qs[e], gg[r], ak);
                    av = mfma16(Ns[e], a[r], av);
                }
                acc1[t] = ak;
                acc2[t] = av;
            }
        } else {
            // dQ^T[d][i] += sum_j phi(K)[j][d] G^T[j][i]
#pragma unroll
            for (int t = 0; t < 4; t++) {
                f4 aq = acc1[t];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    aq = mfma16(Ks[(4 * g + r) * P::LD + c0 + 16 * t + l16], gg[r], aq);
                acc1[t] = aq;
            }
        }
        __syncthreads();   // the streamed tiles, dden and the partials are rewritten next
    }
    // row x0 + l16 of this job's outputs: phi' from the raw inputs
    const int row = x0 + l16;
    if (row < S) {
        const float* xr = (kjob ? Kx : Qx) + (rb + row) * D;
        float* g1 = (kjob ? dK : dQ) + (rb + row) * D;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int c = c0 + 16 * t + 4 * g;
            if (c < D) {
                f4 v = acc1[t];
                if constexpr (phi_rope(PHI)) {
                    // phi' at the rotated input, then the gradient rotated back
                    v = rope_phi_grad4<PHI>(v, load4c<VEC>(xr, c, D), row, c, rope_w);
                } else if constexpr (PHI != PHI_NONE) {
                    const f4 xv = load4c<VEC>(xr, c, D);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        v[i] *= Phi<PHI>::d(xv[i]);
                }
                store4<VEC>(g1, c, D, v);
            }
            if (kjob && c < E)
                store4<VEC>(dV + (rb + row) * E, c, E, acc2[t]);
        }
    }
}

// ---------------------------------------------------------------------------
// Final state of each sequence for the APIs that return it in S_buf / z_buf
// (the reference's running state ends there): S[d][e] = sum_s phi(K_s)[d] V_s[e],
// z[d] = sum_s phi(K_s)[d].  Workgroup (sequence, 64-row d tile, 64-column e
// tile) of four waves; wave w takes 16-row chunks w, w+4, ... and the four
// partial tiles are summed through LDS.  Lane (l16, g) holds phi(K) rows
// 4g + r of column d = 16dt + l16 and V rows 4g + r of column e = 16et + l16.
// ---------------------------------------------------------------------------
template <int PHI>
__global__ __launch_bounds__(256) void lin_wide_state_kernel(
    const float* __restrict__ K, const float* __restrict__ V, float* __restrict__ Sfin,
    float* __restrict__ zfin, int S, int D, int E, int sfin_de)
{
    __shared__ __attribute__((aligned(16))) float red[4][64 * 65];
    __shared__ float zred[4][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int ndt = (D + 63) / 64, net = (E + 63) / 64;
    const int seq = (int)(blockIdx.x / (ndt * net));
    const int rem = (int)(blockIdx.x % (ndt * net));
    const int d0 = 64 * (rem / net), e0 = 64 * (rem % net);
    const long rb = (long)seq * S;
    f4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
            acc[a][b] = f4zero();
    float zs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 16 * w; s0 < S; s0 += 64) {
        f4 kc[4], vc[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int s = s0 + 4 * g + r, d = d0 + 16 * dt + l16;
                const float x = (s < S && d < D) ? K[(rb + s) * D + d] : 0.0f;
                kc[dt][r] = (s < S && d < D) ? Phi<PHI>::f(x) : 0.0f;
            }
        }
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int s = s0 + 4 * g + r, e = e0 + 16 * et + l16;
                vc[et][r] = (s < S && e < E) ? V[(rb + s) * E + e] : 0.0f;
            }
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[dt][et] = mfma16(kc[dt][r], vc[et][r], acc[dt][et]);
            zs[dt] += kc[dt][0] + kc[dt][1] + kc[dt][2] + kc[dt][3];
        }
    }
    // lane (l16, g), element r of acc[dt][et] <-> d = 16dt + 4g + r, e = 16et + l16
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                red[w][(16 * dt + 4 * g + r) * 65 + 16 * et + l16] = acc[dt][et][r];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        const float zt = xrow_sum(zs[dt]);   // column d = 16dt + l16 over the wave's rows
        if (g == 0)
            zred[w][16 * dt + l16] = zt;
    }
    __syncthreads();
    for (int i = tid; i < 64 * 64; i += 256) {
        const int dl = i / 64, el = i % 64;
        const int d = d0 + dl, e = e0 + el;
        if (d < D && e < E) {
            const float v = red[0][dl * 65 + el] + red[1][dl * 65 + el] + red[2][dl * 65 + el] +
                            red[3][dl * 65 + el];
            Sfin[(long)seq * D * E + (sfin_de ? (long)d * E + e : (long)e * D + d)] = v;
        }
    }
    if (zfin != nullptr && e0 == 0 && tid < 64 && d0 + tid < D)
        zfin[(long)seq * D + d0 + tid] = zred[0][tid] + zred[1][tid] + zred[2][tid] + zred[3][tid];
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
bool lin_wide_ok(int D, int E)
{
    const int m = std::max(D, E);
    return D >= 1 && E >= 1 && m > 64 && m <= LIN_WIDE_MAX;
}

bool lin_quad_ok(int D, int E, long S)
{
    return lin_wide_ok(D, E) || (D >= 1 && E >= 1 && D <= 64 && E <= 64 && S <= LIN_QUAD_MAX_S);
}

static inline bool al16x(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (cached per device).
static int wide_cus()
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

// Key blocks per part of the forward: whole query blocks (PL = the block
// count) unless those jobs leave resident workgroup slots free (B' x blocks
// below one round); then the smallest power of two whose jobs fit one round,
// so the longest job is PL key blocks instead of S / 16.  Narrow widths
// (NW < 4) keep whole blocks: their blocks are cheap and plentiful.
template <int NW>
static int wide_fwd_pl(int Bq, int nqb)
{
    if (NW < 4 || nqb <= 1)
        return nqb;
    static int per_cu = 0;
    if (per_cu <= 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)lin_wide_fwd_kernel<PHI_NONE, NW, true>, 64 * NW, 0) !=
                hipSuccess || n <= 0)
            n = 1;
        per_cu = n;
    }
    const long slots = (long)per_cu * wide_cus();
    if ((long)Bq * nqb >= slots)
        return nqb;
    for (int pl = 1; pl < nqb; pl *= 2) {
        long units = 0;
        for (int qb = 0; qb < nqb; qb++)
            units += (qb + pl) / pl;
        if ((long)Bq * units <= slots)
            return pl;
    }
    return nqb;
}

template <int NW>
static size_t wide_fwd_ws(int Bq, int S, int E)
{
    const int nqb = (S + LWB - 1) / LWB;
    const int pl = wide_fwd_pl<NW>(Bq, nqb);
    const long pmax = (nqb + pl - 1) / pl;
    if (pmax <= 1)
        return 0;
    const size_t N = (size_t)Bq * S;
    return (size_t)pmax * N * ((size_t)E + 1) * sizeof(float);
}

// The block-score path (linquad.hip) takes every width above 64 whose scratch
// fits its budget; narrow heads keep the one-wave kernels here.
static bool wide_qs(int Bq, int S, int D, int E)
{
    return std::max(D, E) > 64 && lin_qs_ok(Bq, S, D, E);
}

bool lin_qs_path(int Bq, int S, int D, int E)
{
    return lin_quad_any(Bq, S, D, E) && wide_qs(Bq, S, D, E);
}

bool lin_quad_any(int Bq, int S, int D, int E)
{
    return lin_quad_ok(D, E, S) || (std::max(D, E) > LIN_WIDE_MAX && lin_qs_ok(Bq, S, D, E));
}

size_t lin_wide_ws_bytes(int Bq, int S, int D, int E)
{
    if (wide_qs(Bq, S, D, E))
        return lin_qs_bytes(Bq, S, D, E, 0);
    if (!lin_wide_ok(D, E))
        return 0;
    const int m = std::max(D, E);
    if (m <= 128)
        return 0;
    return m <= 256 ? wide_fwd_ws<4>(Bq, S, E) : wide_fwd_ws<8>(Bq, S, E);
}

size_t lin_wide_bwd_ws_bytes(int Bq, int S, int D, int E, int kinds)
{
    return wide_qs(Bq, S, D, E) ? lin_qs_bytes(Bq, S, D, E, kinds) : 0;
}

// ws: lin_wide_ws_bytes of scratch, or null (whole query blocks); z_cache
// needs whole blocks.
template <int PHI, int NW>
static hipError_t wide_fwd_t(const float* Q, const float* K, const float* V, float* O,
                             float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                             bool vec, void* ws, hipStream_t st)
{
    const int nqb = (S + LWB - 1) / LWB;
    const int PL = (zc == nullptr && ws != nullptr) ? wide_fwd_pl<NW>(Bq, nqb) : nqb;
    const int PMAX = (nqb + PL - 1) / PL;
    const long N = (long)Bq * S;
    float* wsO = PMAX > 1 ? (float*)ws : nullptr;
    float* wsD = PMAX > 1 ? wsO + (size_t)PMAX * N * E : nullptr;
    dim3 grid((unsigned)((long)nqb * PMAX * Bq)), block(64 * NW);
    {
        ProfScope ps(st, "lin_wide_fwd");
        if (vec)
            CXG_LAUNCH((lin_wide_fwd_kernel<PHI, NW, true>), grid, block, 0, st, Q, K, V, O,
                       den, zc, S, D, E, Bq, den_eps, PL, PMAX, wsO, wsD);
        else
            CXG_LAUNCH((lin_wide_fwd_kernel<PHI, NW, false>), grid, block, 0, st, Q, K, V, O,
                       den, zc, S, D, E, Bq, den_eps, PL, PMAX, wsO, wsD);
    }
    if (PMAX > 1) {
        ProfScope ps(st, "lin_wide_fin");
        CXG_LAUNCH(lin_wide_fin_kernel, dim3((unsigned)((N * E + 255) / 256)), dim3(256), 0, st,
                   wsO, wsD, O, den, S, E, Bq, PL, den_eps);
    }
    return hipGetLastError();
}

template <int PHI, int NW>
static hipError_t wide_bwd_t(const float* Q, const float* K, const float* V, const float* dnum,
                             const float* dden, float* dQ, float* dK, float* dV, int Bq, int S,
                             int D, int E, int kinds, bool vec, hipStream_t st, const float* Qx,
                             const float* Kx)
{
    const int nb = (S + LWB - 1) / LWB;
    dim3 grid((unsigned)((long)(kinds == 3 ? 2 : 1) * nb * Bq)), block(64 * NW);
    ProfScope ps(st, kinds == 3 ? "lin_wide_bwd" : kinds == 1 ? "lin_wide_dkdv" : "lin_wide_dq");
    const LinRopeArg<PHI> rope = lin_rope_arg<PHI>(D);
    if (vec)
        CXG_LAUNCH((lin_wide_bwd_kernel<PHI, NW, true>), grid, block, 0, st, Q, K, V,
                           dnum, dden, dQ, dK, dV, S, D, E, Bq, kinds, Qx, Kx, rope);
    else
        CXG_LAUNCH((lin_wide_bwd_kernel<PHI, NW, false>), grid, block, 0, st, Q, K, V,
                           dnum, dden, dQ, dK, dV, S, D, E, Bq, kinds, Qx, Kx, rope);
    return hipGetLastError();
}

template <int PHI>
static hipError_t wide_fwd_p(const float* Q, const float* K, const float* V, float* O,
                             float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                             bool vec, void* ws, hipStream_t st)
{
    const int m = std::max(D, E);
    if (m <= 64)
        return wide_fwd_t<PHI, 1>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
    if (m <= 128)
        return wide_fwd_t<PHI, 2>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
    if (m <= 256)
        return wide_fwd_t<PHI, 4>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
    return wide_fwd_t<PHI, 8>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
}

template <int PHI>
static hipError_t wide_bwd_p(const float* Q, const float* K, const float* V, const float* dnum,
                             const float* dden, float* dQ, float* dK, float* dV, int Bq, int S,
                             int D, int E, int kinds, bool vec, hipStream_t st, const float* Qx,
                             const float* Kx)
{
    const int m = std::max(D, E);
    if (m <= 64)
        return wide_bwd_t<PHI, 1>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st,
                                  Qx, Kx);
    if (m <= 128)
        return wide_bwd_t<PHI, 2>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st,
                                  Qx, Kx);
    if (m <= 256)
        return wide_bwd_t<PHI, 4>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st,
                                  Qx, Kx);
    return wide_bwd_t<PHI, 8>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st, Qx,
                              Kx);
}

hipError_t lin_wide_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                               float* den, float* zc, int den_eps, int Bq, int S, int D, int E,
                               void* ws, hipStream_t st)
{
    if (ws != nullptr && wide_qs(Bq, S, D, E) && phi != PHI_HEXP && !phi_rope(phi) && al16x(Q) &&
        al16x(K) && al16x(V) && al16x(O) && al16x(zc))
        return lin_qs_fwd_launch(phi, Q, K, V, O, den, zc, den_eps, Bq, S, D, E, ws, st);
    if (!lin_quad_ok(D, E, S))
        return hipErrorInvalidValue;   // above LIN_WIDE_MAX: the block-score path only
    const bool vec = D % 4 == 0 && E % 4 == 0 && al16x(Q) && al16x(K) && al16x(V) && al16x(O);
    if (phi == PHI_ELU1)
        return wide_fwd_p<PHI_ELU1>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
    if (phi == PHI_ELU1_LG)
        return wide_fwd_p<PHI_ELU1_LG>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
    return wide_fwd_p<PHI_NONE>(Q, K, V, O, den, zc, den_eps, Bq, S, D, E, vec, ws, st);
}

hipError_t lin_wide_bwd_launch(int phi, const float* Q, const float* K, const float* V,
                               const float* dnum, const float* dden, float* dQ, float* dK,
                               float* dV, int Bq, int S, int D, int E, int kinds, hipStream_t st,
                               const float* Qx, const float* Kx, void* ws)
{
    if (phi_rope(phi) != (Qx != nullptr && Kx != nullptr))
        return hipErrorInvalidValue;   // RoPE maps: features plus raw inputs; others: no raw
    if (Qx == nullptr) {
        Qx = Q;
        Kx = K;
    }
    if (ws != nullptr && wide_qs(Bq, S, D, E) && phi != PHI_HEXP && al16x(Q) && al16x(K) &&
        al16x(V) && al16x(dnum) && al16x(dQ) && al16x(dK) && al16x(dV) && al16x(Qx) && al16x(Kx))
        return lin_qs_bwd_launch(phi, Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, ws, st,
                                 Qx, Kx);
    if (!lin_quad_ok(D, E, S))
        return hipErrorInvalidValue;   // above LIN_WIDE_MAX: the block-score path only
    const bool vec = D % 4 == 0 && E % 4 == 0 && al16x(Q) && al16x(K) && al16x(V) &&
                     al16x(dnum) && al16x(dQ) && al16x(dK) && al16x(dV) && al16x(Qx) && al16x(Kx);
    if (phi == PHI_ELU1)
        return wide_bwd_p<PHI_ELU1>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st,
                                    Qx, Kx);
    if (phi == PHI_ELU1_LG)
        return wide_bwd_p<PHI_ELU1_LG>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec,
                                       st, Qx, Kx);
    if (phi == PHI_ELU1_ROPE)
        return wide_bwd_p<PHI_ELU1_ROPE>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds,
                                         vec, st, Qx, Kx);
    return wide_bwd_p<PHI_NONE>(Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, kinds, vec, st, Qx,
                                Kx);
}

// ---------------------------------------------------------------------------
// Features of the RoPE map for the quadratic form: F = phi(rot(X)) for Q and K
// (rows of B' sequences of S, width D even; pair i of row t rotated by
// t * 10000^(-2i/D), then two_stage's ELU+1).  Each row is rotated once here,
// where the quadratic-form kernels would rotate every streamed block again in
// each job that reads it.  A thread takes one column pair of FEAT_ROWS
// consecutive rows of both tensors (the pair's frequency read once, pairs
// moved as 8-byte loads when aligned).
// ---------------------------------------------------------------------------
constexpr int FEAT_ROWS = 4;   // rows per thread: the pair's frequency is read once

template <bool VEC>
__global__ __launch_bounds__(256) void lin_rope_feat_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, float* __restrict__ Fq,
    float* __restrict__ Fk, long rows, int S, int D, const LinRopeArg<PHI_ELU1_ROPE> rope)
{
    const int np = D / 2;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    const long rblk = idx / np;
    const int i = (int)(idx - rblk * np);
    const long r0 = rblk * FEAT_ROWS;
    if (r0 >= rows)
        return;
    const float w = rope.w[i];
    using F = Phi<PHI_ELU1_ROPE>;
    auto ld = [&](const float* a) {
        if constexpr (VEC)
            return *reinterpret_cast<const float2*>(a);
        return make_float2(a[0], a[1]);
    };
    auto st = [&](float* a, float2 v) {
        if constexpr (VEC) {
            *reinterpret_cast<float2*>(a) = v;
        } else {
            a[0] = v.x;
            a[1] = v.y;
        }
    };
    int pos = (int)(r0 % S);
#pragma unroll
    for (int k = 0; k < FEAT_ROWS; k++) {
        if (r0 + k < rows) {
            float sn, cs;
            sincos_rev((float)pos * w, &sn, &cs);
            const long off = (r0 + k) * D + 2 * i;
            const float2 q = ld(Q + off), kk = ld(K + off);
            st(Fq + off, make_float2(F::f(q.x * cs - q.y * sn), F::f(q.x * sn + q.y * cs)));
            st(Fk + off, make_float2(F::f(kk.x * cs - kk.y * sn), F::f(kk.x * sn + kk.y * cs)));
        }
        pos = (pos + 1 == S) ? 0 : pos + 1;
    }
}

hipError_t lin_rope_feat_launch(const float* Q, const float* K, float* Fq, float* Fk, int Bq,
                                int S, int D, hipStream_t st)
{
    if (D % 2 != 0 || D > LIN_ROPE_MAX_D)
        return hipErrorInvalidValue;
    const long rows = (long)Bq * S;
    const long n = (rows + FEAT_ROWS - 1) / FEAT_ROWS * (D / 2);
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    const bool vec = (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)Fq | (uintptr_t)Fk) & 7u) == 0;
    const LinRopeArg<PHI_ELU1_ROPE> rope = lin_rope_arg<PHI_ELU1_ROPE>(D);
    ProfScope ps(st, "lin_rope_feat");
    if (vec)
        CXG_LAUNCH(lin_rope_feat_kernel<true>, grid, block, 0, st, Q, K, Fq, Fk, rows, S, D,
                   rope);
    else
        CXG_LAUNCH(lin_rope_feat_kernel<false>, grid, block, 0, st, Q, K, Fq, Fk, rows, S, D,
                   rope);
    return hipGetLastError();
}

hipError_t lin_wide_state_launch(int phi, const float* K, const float* V, float* Sfin,
                                 float* zfin, int sfin_de, int Bq, int S, int D, int E,
                                 hipStream_t st)
{
    const long tiles = (long)((D + 63) / 64) * ((E + 63) / 64);
    dim3 grid((unsigned)(tiles * Bq)), block(256);
    ProfScope ps(st, "lin_wide_state");
    if (phi == PHI_ELU1)
        CXG_LAUNCH(lin_wide_state_kernel<PHI_ELU1>, grid, block, 0, st, K, V, Sfin, zfin,
                           S, D, E, sfin_de);
    else if (phi == PHI_ELU1_LG)
        CXG_LAUNCH(lin_wide_state_kernel<PHI_ELU1_LG>, grid, block, 0, st, K, V, Sfin,
                           zfin, S, D, E, sfin_de);
    else
        CXG_LAUNCH(lin_wide_state_kernel<PHI_NONE>, grid, block, 0, st, K, V, Sfin, zfin,
                           S, D, E, sfin_de);
    return hipGetLastError();
}

} // namespace cxg
