// mhawide.hip -- causal softmax attention for head dims 257..512 (gfx950, FP32 MFMA).
//
// GPT's attention (src/GPT/gpt_gpt.hpp:365-380 forward, :420-438 backward) is
// one head over the whole embedding: scores = Q K^T / sqrt(E) on (B*S) x (B*S)
// with a block-diagonal causal mask (gpt_cuda_kernels.cu:458-480, -1e10 on
// cross-batch and future entries), softmax, times V; the backward goes through
// softmax_backward (:131-173).  Per batch that is causal attention with H = 1
// and Dh = E.  The fused MHA kernels (mha.hip) cover Dh <= 256; the reference
// GPT's training configuration has E = 512 (gpt_train.cpp:139).  These kernels
// take 256 < Dh <= 512 with the same layout ((B*S, H*Dh) rows), scale, lse
// convention and backward contract as mha.hip.
//
// Design.  16 query rows (forward) or 16 keys (backward) per workgroup of
// eight waves (two per SIMD, one workgroup per compute unit by LDS); the head
// dim is split over the waves, 64 columns each, so the 16x16 score tile is
// eight partial products summed through LDS, and each wave
// keeps its own column slice of the O (forward) or dK/dV (backward)
// accumulators in registers.  Scores are formed transposed in the forward (a
// lane owns a query row: its online-softmax state is per lane).  The backward
// runs key-block jobs (dK, dV) and query-block jobs (dQ) side by side in one
// launch, each owning its outputs, so no atomics are needed.  Tiles stream
// through LDS with 16-byte row loads, fetched one block ahead.  When a shape
// has few query blocks for the device (under two per compute unit), the
// forward splits each block's keys into chunks over more workgroups and a
// merge kernel combines their partial softmax states.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>
#include <functional>
#include <queue>
#include <unordered_map>
#include <vector>

namespace cxg {

constexpr int WB = 16;                 // rows per tile (queries and keys)
constexpr int WIDE_DHP = 512;          // padded head dim
constexpr int WLD = WIDE_DHP + 4;      // LDS row stride of a staged tile
constexpr int WW = 8;                  // waves per workgroup (two per SIMD)
constexpr int WT = 64 * WW;            // threads per workgroup
constexpr int WSL = WIDE_DHP / WW;     // head-dim columns per wave
constexpr int WNT = WSL / 16;          // 16-column tiles per wave
constexpr int WU = WB * WIDE_DHP / 4 / WT;   // 16-byte units of a tile per thread

// Rows [r0, r0+16) x [0, Dh) of one head, WU 16-byte units per thread of WT
// (unit u = tid + WT k: row u / 128, column 4 (u % 128)): rows past S repeat
// row S-1 (clamped loads), columns past Dh are zeroed when stored.
struct WideRegs {
    f4 v[WU];
};

template <bool VEC>
__device__ __forceinline__ void wide_fetch(WideRegs& R, const float* __restrict__ head, long ld,
                                           int r0, int S, int Dh, int tid)
{
#pragma unroll
    for (int k = 0; k < WU; k++) {
        const int u = tid + WT * k;
        const int row = u / (WIDE_DHP / 4), c = 4 * (u % (WIDE_DHP / 4));
        R.v[k] = load4c<VEC>(head + (long)min(r0 + row, S - 1) * ld, c, Dh);
    }
}

__device__ __forceinline__ void wide_store(float* __restrict__ dst, const WideRegs& R, int Dh,
                                           int tid)
{
#pragma unroll
    for (int k = 0; k < WU; k++) {
        const int u = tid + WT * k;
        const int row = u / (WIDE_DHP / 4), c = 4 * (u % (WIDE_DHP / 4));
        *reinterpret_cast<f4*>(&dst[row * WLD + c]) = mask4(R.v[k], c, Dh, true);
    }
}

// ---------------------------------------------------------------------------
// forward: job = (bh, 16-query block, chunk of key blocks), latest query
// blocks first.  With few jobs (B*H*nqb well under two per compute unit) a
// query block's key blocks are cut into chunks of C (split-KV), so that the
// last blocks of a sequence, which see every key, do not set the kernel's
// length alone; a chunked block's jobs leave unnormalised partial states
// (o, m, l) in a workspace and mha_wide_merge_kernel combines them.
// C >= nqb: one chunk per query block, written directly.
// ---------------------------------------------------------------------------
constexpr int WREC = WB * WIDE_DHP + 2 * WB;   // partial record: o[16][512], m[16], l[16]
constexpr int WBREC = 2 * WB * WIDE_DHP;       // backward: dK (or dQ) rows, then dV rows

__host__ __device__ inline int wide_nch(int qb, int C) { return (qb + C) / C; }

template <bool VEC>
__global__ __launch_bounds__(WT) void mha_wide_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, float* __restrict__ part, int S, int H,
    int Dh, int BH, int C, float qscale)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * WB * WLD + WW * 256];
    float* Sp = lds + 4 * WB * WLD;   // partial scores [wave][lane * 4 + r]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int nqb = (S + WB - 1) / WB;
    const int ent = (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH);
    int qb = nqb - 1 - ent, ch = 0;
    if (C < nqb) {   // entries: query blocks from the last, each as its chunks
        qb = nqb - 1;
        ch = ent;
        while (ch >= wide_nch(qb, C)) {
            ch -= wide_nch(qb, C);
            qb--;
        }
    }
    const bool chunked = C < nqb && wide_nch(qb, C) > 1;
    const int kb0 = C < nqb ? ch * C : 0;
    const int kb1 = C < nqb ? min(qb + 1, kb0 + C) : qb + 1;
    const int b = bh / H, h = bh - b * H;
    const long ld = (long)H * Dh;
    const long hoff = (long)b * S * ld + (long)h * Dh;
    const int q0 = qb * WB, c0 = w * WSL;

    // this wave's column slice of Q rows q0 + l16 (pre-scaled by scale*log2e)
    f4 q[WNT], o[WNT];
    {
        const float* qrow = Q + hoff + (long)min(q0 + l16, S - 1) * ld;
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int c = c0 + 16 * t + 4 * g;
            q[t] = mask4(load4c<VEC>(qrow, c, Dh), c, Dh, true) * qscale;
            o[t] = f4zero();
        }
    }
    float m_run = -INFINITY, l_run = 0.0f;
    const int qi = q0 + l16;   // this lane's query row

    // key blocks are fetched one ahead into registers and stored to the
    // double-buffered LDS tiles at the top of their step
    WideRegs kr, vr;
    wide_fetch<VEC>(kr, K + hoff, ld, kb0 * WB, S, Dh, tid);
    wide_fetch<VEC>(vr, V + hoff, ld, kb0 * WB, S, Dh, tid);
    for (int kb = kb0; kb < kb1; kb++) {
        const int k0 = kb * WB;
        float* Ks = lds + ((kb - kb0) & 1) * 2 * WB * WLD;
        float* Vs = Ks + WB * WLD;
        wide_store(Ks, kr, Dh, tid);
        wide_store(Vs, vr, Dh, tid);
        __builtin_amdgcn_sched_barrier(0);
        const int kn = min(kb + 1, kb1 - 1) * WB;   // the last step refetches its own block
        wide_fetch<VEC>(kr, K + hoff, ld, kn, S, Dh, tid);
        wide_fetch<VEC>(vr, V + hoff, ld, kn, S, Dh, tid);
        __syncthreads();
        // S^T[j][i] over this wave's columns: lane i = l16, element r <-> key 4g + r
        // two accumulation chains (one wave per SIMD issues a single chain at
        // two thirds of the MFMA rate)
        f4 sp = f4zero(), sp2 = f4zero();
#pragma unroll
        for (int t = 0; t < WNT; t += 2) {
            const f4 kv = *reinterpret_cast<const f4*>(&Ks[l16 * WLD + c0 + 16 * t + 4 * g]);
            const f4 kv2 = *reinterpret_cast<const f4*>(&Ks[l16 * WLD + c0 + 16 * t + 16 + 4 * g]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sp = mfma16(kv[r], q[t][r], sp);
                sp2 = mfma16(kv2[r], q[t + 1][r], sp2);
            }
        }
        *reinterpret_cast<f4*>(&Sp[w * 256 + lane * 4]) = sp + sp2;
        __syncthreads();
        f4 s = f4zero();
#pragma unroll
        for (int u = 0; u < WW; u++)
            s += *reinterpret_cast<const f4*>(&Sp[u * 256 + lane * 4]);
        // causal and length masks, online softmax per query row (lane)
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int kj = k0 + 4 * g + r;
            s[r] = (kj <= qi && kj < S) ? s[r] : -INFINITY;
            mloc = fmaxf(mloc, s[r]);
        }
        const float m_new = fmaxf(m_run, xrow_max(mloc));
        const float alpha = fast_exp2(m_run - m_new);
        f4 p;
        float ploc = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = fast_exp2(s[r] - m_new);
            ploc += p[r];
        }
        l_run = l_run * alpha + xrow_sum(ploc);
        m_run = m_new;
        // O^T[d][i] += sum_j V[j][d] P[i][j] over this wave's columns
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            f4 a = o[t] * alpha;
#pragma unroll
            for (int r = 0; r < 4; r++)
                a = mfma16(Vs[(4 * g + r) * WLD + c0 + 16 * t + l16], p[r], a);
            o[t] = a;
        }
    }
    if (chunked) {
        float* rec = part + (long)blockIdx.x * WREC;
#pragma unroll
        for (int t = 0; t < WNT; t++)
            *reinterpret_cast<f4*>(&rec[l16 * WIDE_DHP + c0 + 16 * t + 4 * g]) = o[t];
        if (w == 0 && g == 0) {
            rec[WB * WIDE_DHP + l16] = m_run;
            rec[WB * WIDE_DHP + WB + l16] = l_run;
        }
    } else if (qi < S) {
        const float inv = 1.0f / l_run;
        if (O != nullptr) {
            float* orow = O + hoff + (long)qi * ld;
#pragma unroll
            for (int t = 0; t < WNT; t++)
                store4<VEC>(orow, c0 + 16 * t + 4 * g, Dh, o[t] * inv);
        }
        if (lse != nullptr && w == 0 && g == 0)
            lse[(long)bh * S + qi] = (m_run + fast_log2(l_run)) * kLn2;
    }
}

// ---------------------------------------------------------------------------
// backward: one launch, two kinds of job and no atomics.
//  * key jobs (bh, key block kb): for every query block from kb on, S and dP
//    (lane = key), P = exp2(S*c - lse2), dS = P (dP - Di) * scale, and over
//    this wave's columns dV^T += dO^T P, dK^T += Q^T dS; dK, dV stored at the end.
//  * query jobs (bh, query block qb): for every key block up to qb, S^T and
//    dP^T (lane = query), the same P and dS, and dQ^T += K^T dS^T; dQ stored.
// The query jobs recompute S and dP (96 MFMA per block pair and wave against
// the 32 dQ atomics per lane they replace: the float atomics of a dQ update per
// 16x16 block pair at Dh = 512 bounded the atomic version).  Jobs are ordered
// longest first within each kind; score partials over the waves' column slices
// are summed through LDS; the streamed tile is fetched one ahead.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(WT) void mha_wide_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ part, int S, int H, int Dh, int BH, int Cb, float qscale, float scale)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * WB * WLD + 2 * WW * 256 + 2 * WB];
    float* Ks = lds;                     // key job: its K, V; query job: the streamed K, V
    float* Vs = Ks + WB * WLD;
    float* Qs = Vs + WB * WLD;           // key job: the streamed Q, dO; query job: its Q, dO
    float* dOs = Qs + WB * WLD;
    float* Sp = dOs + WB * WLD;          // [wave][S, dP][lane * 4 + r]
    float* st = Sp + 2 * WW * 256;       // lse2[16], Di[16] of the current query block
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int nb = (S + WB - 1) / WB;
    const int ent = (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH);
    int L = nb - ent / 2, e = ent & 1;
    if (Cb < nb) {
        L = nb;
        e = ent;
        while (e >= 2 * wide_nch(L - 1, Cb)) {
            e -= 2 * wide_nch(L - 1, Cb);
            L--;
        }
    }
    const int nchL = Cb < nb ? wide_nch(L - 1, Cb) : 1;
    const bool kjob = e < nchL;
    const int chk = kjob ? e : e - nchL;
    const int blk = kjob ? nb - L : L - 1;
    const int b = bh / H, h = bh - b * H;
    const long ld = (long)H * Dh;
    const long hoff = (long)b * S * ld + (long)h * Dh;
    const int c0 = w * WSL, x0 = blk * WB;
    // the job's own tiles: K, V (key job) or Q, dO (query job)
    {
        WideRegs t;
        wide_fetch<VEC>(t, (kjob ? K : Q) + hoff, ld, x0, S, Dh, tid);
        wide_store(kjob ? Ks : Qs, t, Dh, tid);
        wide_fetch<VEC>(t, (kjob ? V : dO) + hoff, ld, x0, S, Dh, tid);
        wide_store(kjob ? Vs : dOs, t, Dh, tid);
    }
    auto load_stats = [&](int q0) {
        if (tid < WB) {
            const int qr = min(q0 + tid, S - 1);
            st[tid] = lse[(long)bh * S + qr] * kLog2e;
            st[WB + tid] = Di[(long)bh * S + qr];
        }
    };
    f4 acc1[WNT], acc2[WNT];   // key job: dK^T, dV^T; query job: dQ^T (acc1)
#pragma unroll
    for (int t = 0; t < WNT; t++) {
        acc1[t] = f4zero();
        acc2[t] = f4zero();
    }
    const int sfirst = kjob ? blk : 0;
    const int sbeg = sfirst + chk * (Cb < nb ? Cb : nb);
    const int send = Cb < nb ? min(sfirst + L, sbeg + Cb) : sfirst + L;
    const float* s1 = (kjob ? Q : K) + hoff;
    const float* s2 = (kjob ? dO : V) + hoff;
    float* d1 = kjob ? Qs : Ks;
    float* d2 = kjob ? dOs : Vs;
    if (!kjob)
        load_stats(x0);
    WideRegs r1, r2;
    wide_fetch<VEC>(r1, s1, ld, sbeg * WB, S, Dh, tid);
    wide_fetch<VEC>(r2, s2, ld, sbeg * WB, S, Dh, tid);
    for (int sb = sbeg; sb < send; sb++) {
        const int y0 = sb * WB;
        wide_store(d1, r1, Dh, tid);
        wide_store(d2, r2, Dh, tid);
        if (kjob)
            load_stats(y0);
        __builtin_amdgcn_sched_barrier(0);
        const int yn = min(sb + 1, send - 1) * WB;   // the last step refetches its own block
        wide_fetch<VEC>(r1, s1, ld, yn, S, Dh, tid);
        wide_fetch<VEC>(r2, s2, ld, yn, S, Dh, tid);
        __syncthreads();
        // key job: S[i][j], dP[i][j] (lane j = key, element r <-> query 4g + r);
        // query job: S^T, dP^T (lane i = query, element r <-> key 4g + r)
        f4 sp = f4zero(), dpp = f4zero();
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int c = c0 + 16 * t + 4 * g;
            const f4 qa = *reinterpret_cast<const f4*>(&Qs[l16 * WLD + c]);
            const f4 ka = *reinterpret_cast<const f4*>(&Ks[l16 * WLD + c]);
            const f4 oa = *reinterpret_cast<const f4*>(&dOs[l16 * WLD + c]);
            const f4 va = *reinterpret_cast<const f4*>(&Vs[l16 * WLD + c]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (kjob) {
                    sp = mfma16(qa[r], ka[r], sp);
                    dpp = mfma16(oa[r], va[r], dpp);
                } else {
                    sp = mfma16(ka[r], qa[r], sp);
                    dpp = mfma16(va[r], oa[r], dpp);
                }
            }
        }
        *reinterpret_cast<f4*>(&Sp[(2 * w) * 256 + lane * 4]) = sp;
        *reinterpret_cast<f4*>(&Sp[(2 * w + 1) * 256 + lane * 4]) = dpp;
        __syncthreads();
        f4 sv = f4zero(), dp = f4zero();
#pragma unroll
        for (int u = 0; u < WW; u++) {
            sv += *reinterpret_cast<const f4*>(&Sp[(2 * u) * 256 + lane * 4]);
            dp += *reinterpret_cast<const f4*>(&Sp[(2 * u + 1) * 256 + lane * 4]);
        }
        const int q0 = kjob ? y0 : x0, k0 = kjob ? x0 : y0;
        f4 p, ds;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qo = kjob ? 4 * g + r : l16;   // query row within the block
            const int kj = k0 + (kjob ? l16 : 4 * g + r);
            const int qi = q0 + qo;
            const bool ok = kj <= qi && qi < S && kj < S;
            p[r] = ok ? fast_exp2(sv[r] * qscale - st[qo]) : 0.0f;
            ds[r] = p[r] * (dp[r] - st[WB + qo]) * scale;
        }
        if (kjob) {
            // dV^T[d][j] += sum_i dO[i][d] P[i][j];  dK^T[d][j] += sum_i Q[i][d] dS[i][j]
#pragma unroll
            for (int t = 0; t < WNT; t++) {
                f4 ak = acc1[t], av = acc2[t];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int e = (4 * g + r) * WLD + c0 + 16 * t + l16;
                    ak = mfma16(Qs[e], ds[r], ak);
                    av = mfma16(dOs[e], p[r], av);
                }
                acc1[t] = ak;
                acc2[t] = av;
            }
        } else {
            // dQ^T[d][i] += sum_j K[j][d] dS[i][j]
#pragma unroll
            for (int t = 0; t < WNT; t++) {
                f4 a = acc1[t];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    a = mfma16(Ks[(4 * g + r) * WLD + c0 + 16 * t + l16], ds[r], a);
                acc1[t] = a;
            }
        }
        __syncthreads();   // the streamed tiles, stats and partials are rewritten next
    }
    if (nchL > 1) {
        float* rec = part + (long)blockIdx.x * WBREC;
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int c = c0 + 16 * t + 4 * g;
            *reinterpret_cast<f4*>(&rec[l16 * WIDE_DHP + c]) = acc1[t];
            if (kjob)
                *reinterpret_cast<f4*>(&rec[WB * WIDE_DHP + l16 * WIDE_DHP + c]) = acc2[t];
        }
        return;
    }
    const int row = x0 + l16;
    if (row < S) {
        const long ro = hoff + (long)row * ld;
#pragma unroll
        for (int t = 0; t < WNT; t++) {
            const int c = c0 + 16 * t + 4 * g;
            if (kjob) {
                store4<VEC>(dK + ro, c, Dh, acc1[t]);
                store4<VEC>(dV + ro, c, Dh, acc2[t]);
            } else {
                store4<VEC>(dQ + ro, c, Dh, acc1[t]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launchers
// Combine the chunks of every chunked query block: M = max m_c,
// L = sum 2^(m_c - M) l_c, O = sum 2^(m_c - M) o_c / L, lse = (M + log2 L) ln 2.
// Workgroup (query block, bh, column quarter); 16 threads form the per-row
// chunk weights 2^(m_c - M) / L in LDS, then each thread sums two float4
// columns of one row over the chunks.  Unchunked blocks return at once.
constexpr int WIDE_MAXCH = 256;   // chunks per query block: nqb < 512 and C >= 2 when split

__global__ __launch_bounds__(256) void mha_wide_merge_kernel(const float* __restrict__ part,
                                                            float* __restrict__ O,
                                                            float* __restrict__ lse, int S,
                                                            int H, int Dh, int BH, int C)
{
    __shared__ float wsh[WB][WIDE_MAXCH];
    const int nqb = (S + WB - 1) / WB;
    const int quarter = (int)(blockIdx.x & 3);
    const int job = (int)(blockIdx.x >> 2);
    const int qb = job / BH, bh = job - (job / BH) * BH;
    const int nch = wide_nch(qb, C);
    if (nch == 1)
        return;
    int e0 = 0;   // entry of the block's first chunk
    for (int q = nqb - 1; q > qb; q--)
        e0 += wide_nch(q, C);
    const float* rec0 = part + ((long)e0 * BH + bh) * WREC;
    const long cstride = (long)BH * WREC;   // between a block's consecutive chunks
    const int tid = threadIdx.x;
    if (tid < WB) {
        float M = -INFINITY;
        for (int j = 0; j < nch; j++)
            M = fmaxf(M, rec0[j * cstride + WB * WIDE_DHP + tid]);
        float L = 0.0f;
        for (int j = 0; j < nch; j++) {
            const float wgt = fast_exp2(rec0[j * cstride + WB * WIDE_DHP + tid] - M);
            wsh[tid][j] = wgt;
            L += wgt * rec0[j * cstride + WB * WIDE_DHP + WB + tid];
        }
        const float inv = 1.0f / L;
        for (int j = 0; j < nch; j++)
            wsh[tid][j] *= inv;
        const int qi = qb * WB + tid;
        if (lse != nullptr && quarter == 0 && qi < S)
            lse[(long)bh * S + qi] = (M + fast_log2(L)) * kLn2;
    }
    __syncthreads();
    if (O == nullptr)
        return;
    const int row = tid >> 4;
    const int c0 = quarter * (WIDE_DHP / 4) + 4 * (tid & 15), c1 = c0 + 64;
    f4 a0 = f4zero(), a1 = f4zero();
    for (int j = 0; j < nch; j++) {
        const float* rec = rec0 + j * cstride + row * WIDE_DHP;
        const float wgt = wsh[row][j];
        a0 += *reinterpret_cast<const f4*>(rec + c0) * wgt;
        a1 += *reinterpret_cast<const f4*>(rec + c1) * wgt;
    }
    const int qi = qb * WB + row;
    if (qi >= S)
        return;
    const int b = bh / H, h = bh - b * H;
    const long ld = (long)H * Dh;
    float* orow = O + (long)b * S * ld + (long)h * Dh + (long)qi * ld;
    const bool vec = Dh % 4 == 0 && (((uintptr_t)orow & 15u) == 0);
    for (int k = 0; k < 2; k++) {
        const int c = k ? c1 : c0;
        const f4 v = k ? a1 : a0;
        if (c >= Dh)
            continue;
        if (vec) {
            *reinterpret_cast<f4*>(orow + c) = v;
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (c + i < Dh)
                    orow[c + i] = v[i];
        }
    }
}

// Sum the chunks of every chunked backward job (jobs numbered like the
// backward's entries) into dK and dV, or dQ.  Workgroup (job, column quarter).
__global__ __launch_bounds__(256) void mha_wide_bsum_kernel(const float* __restrict__ part,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int S, int H, int Dh,
    int BH, int Cb)
{
    const int nb = (S + WB - 1) / WB;
    const int quarter = (int)(blockIdx.x & 3);
    const int job = (int)(blockIdx.x >> 2);
    const int bh = job % BH;
    const int kind = (job / BH) & 1;
    const int L = job / (2 * BH) + 1;
    const int nch = wide_nch(L - 1, Cb);
    if (nch == 1)
        return;
    int e0 = 0;
    for (int l = nb; l > L; l--)
        e0 += 2 * wide_nch(l - 1, Cb);
    e0 += kind ? nch : 0;
    const float* rec0 = part + ((long)e0 * BH + bh) * WBREC;
    const long cstride = (long)BH * WBREC;
    const int tid = threadIdx.x, row = tid >> 4;
    const int c0 = quarter * (WIDE_DHP / 4) + 4 * (tid & 15), c1 = c0 + 64;
    f4 a0 = f4zero(), a1 = f4zero(), b0 = f4zero(), b1 = f4zero();
    for (int j = 0; j < nch; j++) {
        const float* rec = rec0 + j * cstride + row * WIDE_DHP;
        a0 += *reinterpret_cast<const f4*>(rec + c0);
        a1 += *reinterpret_cast<const f4*>(rec + c1);
        if (kind == 0) {
            b0 += *reinterpret_cast<const f4*>(rec + WB * WIDE_DHP + c0);
            b1 += *reinterpret_cast<const f4*>(rec + WB * WIDE_DHP + c1);
        }
    }
    const int blk = kind ? L - 1 : nb - L;
    const int x = blk * WB + row;
    if (x >= S)
        return;
    const int b = bh / H, h = bh - b * H;
    const long ld = (long)H * Dh;
    const long ro = (long)b * S * ld + (long)h * Dh + (long)x * ld;
    for (int k = 0; k < 2; k++) {
        const int c = k ? c1 : c0;
        if (c >= Dh)
            continue;
        const f4 va = k ? a1 : a0, vb = k ? b1 : b0;
        for (int o = 0; o < (kind ? 1 : 2); o++) {
            float* dst = (kind ? dQ : (o ? dV : dK)) + ro;
            const f4 v = o ? vb : va;
            if (Dh % 4 == 0 && (((uintptr_t)dst & 15u) == 0)) {
                *reinterpret_cast<f4*>(dst + c) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (c + i < Dh)
                        dst[c + i] = v[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
static inline bool al16w(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Key-block chunk for the forward: list-schedule the jobs (heaviest query
// blocks first, one workgroup per compute unit, a job costing its key blocks
// plus ~0.6 of a block of set-up) for a few chunk sizes, charging a split
// for its merge, and keep the shortest.  Only when jobs are few: with two or
// more whole query blocks per compute unit the plain grid balances itself.
static int wide_fwd_chunk(int BH, int S)
{
    const int nqb = (S + WB - 1) / WB;
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if ((long)BH * nqb >= 2L * cus || nqb < 4)
        return nqb;
    // decisions cached per thread (the simulation is a few thousand heap steps)
    static thread_local std::unordered_map<long long, int> cache;
    const long long key = ((long long)BH << 40) ^ ((long long)S << 12) ^ cus;
    auto hit = cache.find(key);
    if (hit != cache.end())
        return hit->second;
    int best_c = nqb;
    double best = 0.0;
    bool first = true;
    for (int C : {nqb, 2, 3, 4, 5, 6, 8, 12, 16}) {
        if (!first && (C >= nqb || wide_nch(nqb - 1, C) > WIDE_MAXCH))
            continue;
        std::priority_queue<double, std::vector<double>, std::greater<double>> freeq;
        for (int i = 0; i < cus; i++)
            freeq.push(0.0);
        long parts = 0;
        for (int qb = nqb - 1; qb >= 0; qb--) {
            const int nch = C < nqb ? wide_nch(qb, C) : 1;
            for (int c = 0; c < nch; c++) {
                const int len = nch > 1 ? std::min(C, qb + 1 - c * C) : qb + 1;
                for (int b = 0; b < BH; b++) {
                    const double t = freeq.top();
                    freeq.pop();
                    freeq.push(t + len + 0.6);
                }
                if (nch > 1)
                    parts += BH;
            }
        }
        double t = 0.0;
        while (!freeq.empty()) {
            t = std::max(t, freeq.top());
            freeq.pop();
        }
        if (C < nqb)
            t += 1.0 + 0.1 * (double)parts / cus;   // merge launch and traffic
        if (first || t < best) {
            best = t;
            best_c = C;
        }
        first = false;
    }
    cache[key] = best_c;
    return best_c;
}

size_t mha_wide_fwd_ws_floats(int BH, int S)
{
    const int nqb = (S + WB - 1) / WB;
    const int C = wide_fwd_chunk(BH, S);
    if (C >= nqb)
        return 0;
    long nent = 0;
    for (int qb = 0; qb < nqb; qb++)
        nent += wide_nch(qb, C);
    return (size_t)nent * BH * WREC;
}

hipError_t mha_wide_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                               float* lse, int B, int S, int H, int Dh, float* part,
                               hipStream_t st)
{
    const int nqb = (S + WB - 1) / WB;
    const int BH = B * H;
    const int C = wide_fwd_chunk(BH, S);
    if (C < nqb && part == nullptr)
        return hipErrorInvalidValue;
    long nent = nqb;
    if (C < nqb) {
        nent = 0;
        for (int qb = 0; qb < nqb; qb++)
            nent += wide_nch(qb, C);
    }
    const float qscale = (1.0f / sqrtf((float)Dh)) * kLog2e;
    dim3 grid((unsigned)(nent * BH)), block(WT);
    const bool vec = Dh % 4 == 0 && al16w(Q) && al16w(K) && al16w(V) && al16w(O);
    {
        ProfScope ps(st, O != nullptr ? "mha_wide_fwd" : "mha_wide_stats");
        if (vec)
            CXG_LAUNCH(mha_wide_fwd_kernel<true>, grid, block, 0, st, Q, K, V, O, lse,
                               part, S, H, Dh, BH, C, qscale);
        else
            CXG_LAUNCH(mha_wide_fwd_kernel<false>, grid, block, 0, st, Q, K, V, O, lse,
                               part, S, H, Dh, BH, C, qscale);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || C >= nqb)
        return e;
    ProfScope ps(st, "mha_wide_merge");
    CXG_LAUNCH(mha_wide_merge_kernel, dim3((unsigned)((long)nqb * BH * 4)), dim3(256), 0, st,
                       part, O, lse, S, H, Dh, BH, C);
    return hipGetLastError();
}

// Backward stream chunk: with few jobs (2*B*H*nb under three per compute
// unit) the long key and query jobs are cut into chunks of nb/3 blocks (at
// least 2) whose partial dK/dV/dQ mha_wide_bsum_kernel adds up.  Tuned on
// B8 S256 E512 (nb = 16): chunks of 2..8 blocks gave 99.9, 95.0, 93.5,
// 86.7, 91.7, -, 101.9 us per fwd+bwd step against 95.1 unchunked; nb/3 = 5.
static int wide_bwd_chunk(int BH, int S)
{
    const int nb = (S + WB - 1) / WB;
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (2L * BH * nb >= 3L * cus || nb < 6)
        return nb;
    return std::max(2, nb / 3);
}

static long wide_bwd_entries(int nb, int Cb)
{
    long n = 0;
    for (int L = 1; L <= nb; L++)
        n += 2 * (Cb < nb ? wide_nch(L - 1, Cb) : 1);
    return n;
}

size_t mha_wide_bwd_ws_floats(int BH, int S)
{
    const int nb = (S + WB - 1) / WB;
    const int Cb = wide_bwd_chunk(BH, S);
    return Cb < nb ? (size_t)wide_bwd_entries(nb, Cb) * BH * WBREC : 0;
}

hipError_t mha_wide_bwd_launch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, float* part,
                               hipStream_t st)
{
    const int nb = (S + WB - 1) / WB;
    const int BH = B * H;
    const int Cb = wide_bwd_chunk(BH, S);
    if (Cb < nb && part == nullptr)
        return hipErrorInvalidValue;
    const float scale = 1.0f / sqrtf((float)Dh);
    dim3 grid((unsigned)(wide_bwd_entries(nb, Cb) * BH)), block(WT);
    const bool vec = Dh % 4 == 0 && al16w(Q) && al16w(K) && al16w(V) && al16w(dO) &&
                     al16w(dQ) && al16w(dK) && al16w(dV);
    {
        ProfScope ps(st, "mha_wide_bwd");
        if (vec)
            CXG_LAUNCH(mha_wide_bwd_kernel<true>, grid, block, 0, st, Q, K, V, dO, lse,
                               Di, dQ, dK, dV, part, S, H, Dh, BH, Cb, scale * kLog2e, scale);
        else
            CXG_LAUNCH(mha_wide_bwd_kernel<false>, grid, block, 0, st, Q, K, V, dO, lse,
                               Di, dQ, dK, dV, part, S, H, Dh, BH, Cb, scale * kLog2e, scale);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || Cb >= nb)
        return e;
    ProfScope ps(st, "mha_wide_bsum");
    CXG_LAUNCH(mha_wide_bsum_kernel, dim3((unsigned)(2L * nb * BH * 4)), dim3(256), 0, st,
                       part, dQ, dK, dV, S, H, Dh, BH, Cb);
    return hipGetLastError();
}

} // namespace cxg
