// linattn.hip -- causal linear ("kernel") attention for gfx950 (FP32 MFMA).
//
// Replaces the serial per-timestep scans of
//   two_stage_cuda::kernel_attn_fwd / _bwd_step1 / _bwd_dQ / _bwd_dKdV
//     (src/TwoStage/two_stage_cuda_kernels.cu:885-1809), phi = ELU+1 fused, and
//   linear_cuda::causal_linear_attention_fwd / _bwd_step1 / _bwd_dQ / _bwd_dKdV
//     (src/LinearAttention/linear_cuda_kernels.cu:10-298), phi applied outside,
// with a chunked parallel scan.
//
// Recurrences (per sequence; Q/K rows of width D, V/O rows of width E):
//   forward : S_t = sum_{s<=t} phi(K_s) V_s^T (D x E), z_t = sum_{s<=t} phi(K_s)
//             den_t = phi(Q_t).z_t, O_t = phi(Q_t)^T S_t / (den_t + 1e-8)
//   dQ      : dQ_t = (z_t dden_t + S_t dnum_t) * phi'(Q_t)
//   dK, dV  : S*_t = sum_{s>=t} phi(Q_s) dnum_s^T, z*_t = sum_{s>=t} dden_s phi(Q_s)
//             dV_t = S*_t^T phi(K_t), dK_t = (z*_t + S*_t V_t) * phi'(K_t)
//
// Fast path (D <= 64 and E <= 64, padded to 64): the sequence is cut into
// segments of L rows; one wave owns one segment and walks it in 16-row
// chunks, holding the 64x64 state in MFMA accumulator registers.  Per chunk
// the contribution of earlier chunks is one state product (phi(Q) S) and the
// contribution inside the chunk is a masked 16x16 product, all on
// v_mfma_f32_16x16x4_f32.  A segment's starting state comes from a
// per-segment aggregate kernel (lin_agg) followed by an exclusive scan over
// segments (lin_scan); with one segment per sequence both are skipped.
//
// Wider D/E take the generic kernels at the end of the file (one workgroup
// per sequence, serial over t, state in global scratch).
//
// Register layouts of a 16-row chunk (lane l, l16 = l%16, g = l/16, f4 element r):
//   R-layout:  v[ct][r] = M[t0 + l16][16ct + 4g + r]   (row per lane)
//   C-layout:  v[ct][r] = M[t0 + 4g + r][16ct + l16]   (column per lane)
#include "common.hpp"
#include "launch.hpp"
#include "linattn.hpp"

namespace cxg {

constexpr int LIN_THREADS = 256;
constexpr int LIN_WAVES = LIN_THREADS / 64;

template <int PHI>
struct Phi;
template <>
struct Phi<PHI_ELU1> {
    // two_stage_cuda_kernels.cu:1027-1031 / kernel_test.cpp:16-17
    static __device__ __forceinline__ float f(float x) { return x > 0.0f ? x + 1.0f : __expf(x); }
    static __device__ __forceinline__ float d(float x) { return x > 0.0f ? 1.0f : __expf(x); }
};
template <>
struct Phi<PHI_NONE> {
    static __device__ __forceinline__ float f(float x) { return x; }
    static __device__ __forceinline__ float d(float) { return 1.0f; }
};

// ---------------------------------------------------------------------------
// chunk loaders.  Rows >= S and columns >= ncol read as 0; APPLY_PHI maps the
// valid entries through phi and leaves padding at exactly 0.
// ---------------------------------------------------------------------------
template <bool VEC, int PHI, bool APPLY_PHI>
__device__ __forceinline__ void load_R(f4 (&v)[4], const float* __restrict__ M, long ld,
                                       long row, bool rok, int ncol, int g)
{
    const float* p = M + (rok ? row : 0) * ld;
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
        const int c = 16 * ct + 4 * g;
        f4 x = load4<VEC>(p, c, ncol, rok);
        if (APPLY_PHI) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                x[i] = (rok && c + i < ncol) ? Phi<PHI>::f(x[i]) : 0.0f;
        }
        v[ct] = x;
    }
}

template <int PHI, bool APPLY_PHI>
__device__ __forceinline__ void load_C(f4 (&v)[4], const float* __restrict__ M, long ld,
                                       long row0, int nvalid, int ncol, int l16)
{
    // rows row0 + r for r < nvalid are in range
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
        const int c = 16 * ct + l16;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = (r < nvalid) && (c < ncol);
            float x = ok ? M[(row0 + r) * ld + c] : 0.0f;
            if (APPLY_PHI)
                x = ok ? Phi<PHI>::f(x) : 0.0f;
            v[ct][r] = x;
        }
    }
}

// ---------------------------------------------------------------------------
// per-segment aggregates: dS = sum_s phi(X_s)^T Y_s (64 x 64), dz = sum_s w_s phi(X_s)
// (w = 1 when null).  Forward direction: X = K, Y = V.  Reverse: X = Q, Y = dnum,
// w = dden.  Written row-major [d][e] followed by z[d], LIN_WS floats per segment.
// ---------------------------------------------------------------------------
template <int PHI, bool VEC>
__global__ __launch_bounds__(LIN_THREADS) void lin_agg_kernel(
    const float* __restrict__ X, const float* __restrict__ Y, const float* __restrict__ w,
    float* __restrict__ ws, int Bq, int S, int D, int E, int nseg, int L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x * LIN_WAVES + wave;
    if (wid >= Bq * nseg)
        return;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L);
    const long rb = (long)seq * S;

    f4 St[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++)
            St[a][c] = f4zero();
    float zp[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    for (int t0 = tbeg; t0 < tend; t0 += 16) {
        const int nv = min(4, max(0, tend - (t0 + 4 * g)));
        f4 xC[4], yC[4];
        load_C<PHI, true>(xC, X, D, rb + t0 + 4 * g, nv, D, l16);
        load_C<PHI, false>(yC, Y, E, rb + t0 + 4 * g, nv, E, l16);
        float wr[4];
#pragma unroll
        for (int r = 0; r < 4; r++)
            wr[r] = (w == nullptr) ? 1.0f : (r < nv ? w[rb + t0 + 4 * g + r] : 0.0f);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                zp[dt] += wr[r] * xC[dt][r];
#pragma unroll
            for (int et = 0; et < 4; et++) {
                f4 acc = St[dt][et];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(xC[dt][r], yC[et][r], acc);
                St[dt][et] = acc;
            }
        }
    }
    float* P = ws + (long)wid * LIN_WS;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                P[(16 * dt + 4 * g + r) * 64 + 16 * et + l16] = St[dt][et][r];
        const float z = xrow_sum(zp[dt]);
        if (g == 0)
            P[4096 + 16 * dt + l16] = z;
    }
}

// Exclusive scan over the segments of each sequence, in place: forward
// (prefix of earlier segments) or reverse (suffix of later segments).
__global__ __launch_bounds__(256) void lin_scan_kernel(float* __restrict__ ws, int Bq, int nseg,
                                                      int reverse)
{
    const long j = (long)blockIdx.x * 256 + threadIdx.x;
    if (j >= (long)Bq * LIN_WS)
        return;
    const long seq = j / LIN_WS, e = j - seq * LIN_WS;
    float run = 0.0f;
    for (int k = 0; k < nseg; k++) {
        const int s = reverse ? nseg - 1 - k : k;
        const long idx = (seq * nseg + s) * LIN_WS + e;
        const float tmp = ws[idx];
        ws[idx] = run;
        run += tmp;
    }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int PHI, bool VEC>
__global__ __launch_bounds__(LIN_THREADS) void lin_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ den, float* __restrict__ zcache,
    const float* __restrict__ ws, float* __restrict__ Sfin, float* __restrict__ zfin,
    int sfin_de, int den_incl_eps, int Bq, int S, int D, int E, int nseg, int L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x * LIN_WAVES + wave;
    if (wid >= Bq * nseg)
        return;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L);
    const long rb = (long)seq * S;

    // state S[d][e]: St[dt][et] lane (e = 16et + l16), element r <-> d = 16dt + 4g + r
    // z[d]:          zr[dt]   element r <-> d = 16dt + 4g + r (same in every lane row)
    f4 St[4][4], zr[4];
    if (ws != nullptr) {
        const float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    St[dt][et][r] = P[(16 * dt + 4 * g + r) * 64 + 16 * et + l16];
            zr[dt] = *reinterpret_cast<const f4*>(P + 4096 + 16 * dt + 4 * g);
        }
    } else {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++)
                St[dt][et] = f4zero();
            zr[dt] = f4zero();
        }
    }

    for (int t0 = tbeg; t0 < tend; t0 += 16) {
        const long trow = rb + t0 + l16;
        const bool rok = t0 + l16 < tend;
        const int nv = min(4, max(0, tend - (t0 + 4 * g)));
        f4 q[4], kR[4], kC[4], vC[4];
        load_R<VEC, PHI, true>(q, Q, D, trow, rok, D, g);
        load_R<VEC, PHI, true>(kR, K, D, trow, rok, D, g);
        load_C<PHI, true>(kC, K, D, rb + t0 + 4 * g, nv, D, l16);
        load_C<PHI, false>(vC, V, E, rb + t0 + 4 * g, nv, E, l16);

        // A^T[s][t] = phi(K_s).phi(Q_t), lane t = l16, element r <-> s = 4g + r; keep s <= t
        f4 At = f4zero();
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                At = mfma16(kR[dt][r], q[dt][r], At);
        f4 Lt;   // lower-triangular ones, as the B operand of the z_cache product
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool keep = 4 * g + r <= l16;
            At[r] = keep ? At[r] : 0.0f;
            Lt[r] = keep ? 1.0f : 0.0f;
        }
        // z_t (R-layout of row t = l16) = z_prev + sum_{s<=t} phi(K_s)
        f4 zc[4];
        float dpart = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            f4 acc = zr[dt];
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(kC[dt][r], Lt[r], acc);
            zc[dt] = acc;
            dpart += q[dt][0] * acc[0] + q[dt][1] * acc[1] + q[dt][2] * acc[2] + q[dt][3] * acc[3];
        }
        const float dn = xrow_sum(dpart);        // den_t = phi(Q_t) . z_t
        const float inv = 1.0f / (dn + 1e-8f);
        if (rok) {
            if (g == 0)
                den[trow] = den_incl_eps ? dn + 1e-8f : dn;
            if (zcache != nullptr)
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
                    store4<VEC>(zcache + trow * D, 16 * dt + 4 * g, D, zc[dt]);
        }
        // next chunk's z = z_t of row 15
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                zr[dt][r] = __shfl(zc[dt][r], (lane & 48) | 15, 64);

        // O^T[e][t] = sum_d S[d][e] phi(Q_t)[d] + sum_s V_s[e] A^T[s][t]
#pragma unroll
        for (int et = 0; et < 4; et++) {
            f4 acc = f4zero();
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(St[dt][et][r], q[dt][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(vC[et][r], At[r], acc);
            if (rok)
                store4<VEC>(O + trow * E, 16 * et + 4 * g, E, acc * inv);
        }
        // S += phi(K)^T V
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int et = 0; et < 4; et++) {
                f4 acc = St[dt][et];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(kC[dt][r], vC[et][r], acc);
                St[dt][et] = acc;
            }
    }

    if (Sfin != nullptr && seg == nseg - 1) {
        // final state of the sequence: [d][e] (linear_cuda) or [e][d] (two_stage)
        float* Sp = Sfin + (long)seq * D * E;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int d = 16 * dt + 4 * g + r, e = 16 * et + l16;
                    if (d < D && e < E)
                        Sp[sfin_de ? (long)d * E + e : (long)e * D + d] = St[dt][et][r];
                }
        if (zfin != nullptr && l16 == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int d = 16 * dt + 4 * g + r;
                    if (d < D)
                        zfin[(long)seq * D + d] = zr[dt][r];
                }
    }
}

// ---------------------------------------------------------------------------
// backward step 1: dnum = dO / den, dden = -(sum_e dO*O) / den.  16 lanes per row.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void lin_step1_kernel(
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ den,
    float* __restrict__ dnum, float* __restrict__ dden, long N, int E)
{
    const long row = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int sub = threadIdx.x & 15;
    const bool ok = row < N;
    float acc = 0.0f, inv = 0.0f;
    if (ok) {
        inv = 1.0f / den[row];
        const long off = row * E;
        for (int c = 4 * sub; c < E; c += 64) {
            const f4 o = load4<VEC>(O + off, c, E, true);
            const f4 d = load4<VEC>(dO + off, c, E, true);
            acc += d[0] * o[0] + d[1] * o[1] + d[2] * o[2] + d[3] * o[3];
            store4<VEC>(dnum + off, c, E, d * inv);
        }
    }
    acc = row16_sum(acc);
    if (ok && sub == 0)
        dden[row] = -acc * inv;
}

// ---------------------------------------------------------------------------
// dQ (forward-direction scan)
// ---------------------------------------------------------------------------
template <int PHI, bool VEC>
__global__ __launch_bounds__(LIN_THREADS) void lin_dq_kernel(
    const float* __restrict__ K, const float* __restrict__ V, const float* __restrict__ dnum,
    const float* __restrict__ dden, const float* __restrict__ zcache, const float* __restrict__ Q,
    float* __restrict__ dQ, const float* __restrict__ ws, int Bq, int S, int D, int E, int nseg,
    int L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x * LIN_WAVES + wave;
    if (wid >= Bq * nseg)
        return;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L);
    const long rb = (long)seq * S;

    // state transposed: StT[et][dt] lane (d = 16dt + l16), element r <-> e = 16et + 4g + r
    f4 StT[4][4];
    if (ws != nullptr) {
        const float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                StT[et][dt] = *reinterpret_cast<const f4*>(P + (16 * dt + l16) * 64 + 16 * et + 4 * g);
    } else {
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                StT[et][dt] = f4zero();
    }

    for (int t0 = tbeg; t0 < tend; t0 += 16) {
        const long trow = rb + t0 + l16;
        const bool rok = t0 + l16 < tend;
        const int nv = min(4, max(0, tend - (t0 + 4 * g)));
        f4 kC[4], vR[4], vC[4], dnR[4], zcR[4], qR[4];
        load_C<PHI, true>(kC, K, D, rb + t0 + 4 * g, nv, D, l16);
        load_R<VEC, PHI, false>(vR, V, E, trow, rok, E, g);
        load_C<PHI, false>(vC, V, E, rb + t0 + 4 * g, nv, E, l16);
        load_R<VEC, PHI, false>(dnR, dnum, E, trow, rok, E, g);
        load_R<VEC, PHI, false>(zcR, zcache, D, trow, rok, D, g);
        if (PHI != PHI_NONE)
            load_R<VEC, PHI, false>(qR, Q, D, trow, rok, D, g);
        const float dd = rok ? dden[trow] : 0.0f;

        // G^T[s][t] = V_s . dnum_t, lane t = l16, element r <-> s = 4g + r; keep s <= t
        f4 G = f4zero();
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                G = mfma16(vR[et][r], dnR[et][r], G);
#pragma unroll
        for (int r = 0; r < 4; r++)
            G[r] = (4 * g + r <= l16) ? G[r] : 0.0f;

        // dQ^T[d][t] = z_t[d] dden_t + sum_e S[d][e] dnum_t[e] + sum_s phi(K_s)[d] G^T[s][t]
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            f4 acc = zcR[dt] * dd;
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(StT[et][dt][r], dnR[et][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(kC[dt][r], G[r], acc);
            if (PHI != PHI_NONE) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[i] *= Phi<PHI>::d(qR[dt][i]);
            }
            if (rok)
                store4<VEC>(dQ + trow * D, 16 * dt + 4 * g, D, acc);
        }
        // S^T += V^T phi(K)
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                f4 acc = StT[et][dt];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(vC[et][r], kC[dt][r], acc);
                StT[et][dt] = acc;
            }
    }
}

// ---------------------------------------------------------------------------
// dK, dV (reverse-direction scan)
// ---------------------------------------------------------------------------
template <int PHI, bool VEC>
__global__ __launch_bounds__(LIN_THREADS) void lin_dkdv_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dnum, const float* __restrict__ dden, float* __restrict__ dK,
    float* __restrict__ dV, const float* __restrict__ ws, int Bq, int S, int D, int E, int nseg,
    int L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x * LIN_WAVES + wave;
    if (wid >= Bq * nseg)
        return;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L);
    const long rb = (long)seq * S;

    // suffix state S*[d][e] in two layouts:
    //   Sd[dt][et]  lane (e = 16et + l16), element r <-> d = 16dt + 4g + r   (dV product)
    //   SdT[et][dt] lane (d = 16dt + l16), element r <-> e = 16et + 4g + r   (dK product)
    // z*[d]: zs[dt] element r <-> d = 16dt + 4g + r
    f4 Sd[4][4], SdT[4][4], zs[4];
    if (ws != nullptr) {
        const float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++) {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    Sd[dt][et][r] = P[(16 * dt + 4 * g + r) * 64 + 16 * et + l16];
                SdT[et][dt] = *reinterpret_cast<const f4*>(P + (16 * dt + l16) * 64 + 16 * et + 4 * g);
            }
            zs[dt] = *reinterpret_cast<const f4*>(P + 4096 + 16 * dt + 4 * g);
        }
    } else {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++) {
                Sd[dt][et] = f4zero();
                SdT[et][dt] = f4zero();
            }
            zs[dt] = f4zero();
        }
    }

    const int nchunk = (tend - tbeg + 15) / 16;
    for (int c = nchunk - 1; c >= 0; c--) {
        const int t0 = tbeg + 16 * c;
        const long trow = rb + t0 + l16;
        const bool rok = t0 + l16 < tend;
        const int nv = min(4, max(0, tend - (t0 + 4 * g)));
        f4 qR[4], qC[4], kraw[4], kR[4], vR[4], dnR[4], dnC[4];
        load_R<VEC, PHI, true>(qR, Q, D, trow, rok, D, g);
        load_C<PHI, true>(qC, Q, D, rb + t0 + 4 * g, nv, D, l16);
        load_R<VEC, PHI, false>(kraw, K, D, trow, rok, D, g);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                kR[dt][i] = (rok && 16 * dt + 4 * g + i < D) ? Phi<PHI>::f(kraw[dt][i]) : 0.0f;
        load_R<VEC, PHI, false>(vR, V, E, trow, rok, E, g);
        load_R<VEC, PHI, false>(dnR, dnum, E, trow, rok, E, g);
        load_C<PHI, false>(dnC, dnum, E, rb + t0 + 4 * g, nv, E, l16);
        f4 ddC;
#pragma unroll
        for (int r = 0; r < 4; r++)
            ddC[r] = r < nv ? dden[rb + t0 + 4 * g + r] : 0.0f;

        // M1^T[s][t] = phi(Q_s).phi(K_t); M2^T[s][t] = dnum_s.V_t + dden_s;
        // lane t = l16, element r <-> s = 4g + r; keep s >= t
        f4 M1 = f4zero(), M2 = f4zero();
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                M1 = mfma16(qR[ct][r], kR[ct][r], M1);
                M2 = mfma16(dnR[ct][r], vR[ct][r], M2);
            }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool keep = 4 * g + r >= l16;
            M1[r] = keep ? M1[r] : 0.0f;
            M2[r] = keep ? M2[r] + ddC[r] : 0.0f;
        }
        // dV^T[e][t] = sum_d S*[d][e] phi(K_t)[d] + sum_s dnum_s[e] M1^T[s][t]
#pragma unroll
        for (int et = 0; et < 4; et++) {
            f4 acc = f4zero();
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(Sd[dt][et][r], kR[dt][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(dnC[et][r], M1[r], acc);
            if (rok)
                store4<VEC>(dV + trow * E, 16 * et + 4 * g, E, acc);
        }
        // dK^T[d][t] = (z*[d] + sum_e S*[d][e] V_t[e] + sum_s phi(Q_s)[d] M2^T[s][t]) phi'(K_t[d])
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            f4 acc = zs[dt];
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(SdT[et][dt][r], vR[et][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(qC[dt][r], M2[r], acc);
            if (PHI != PHI_NONE) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[i] *= Phi<PHI>::d(kraw[dt][i]);
            }
            if (rok)
                store4<VEC>(dK + trow * D, 16 * dt + 4 * g, D, acc);
        }
        // S* += phi(Q)^T dnum (both layouts), z* += phi(Q)^T dden
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int et = 0; et < 4; et++) {
                f4 a = Sd[dt][et], b = SdT[et][dt];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    a = mfma16(qC[dt][r], dnC[et][r], a);
                    b = mfma16(dnC[et][r], qC[dt][r], b);
                }
                Sd[dt][et] = a;
                SdT[et][dt] = b;
            }
            f4 z = zs[dt];
#pragma unroll
            for (int r = 0; r < 4; r++)
                z = mfma16(qC[dt][r], ddC[r], z);
            zs[dt] = z;
        }
    }
}

// ---------------------------------------------------------------------------
// generic kernels (any D, E): one workgroup per sequence, serial over t.
// State S[d][e] lives in global scratch (Bq x D x E), z in LDS.
// ---------------------------------------------------------------------------
template <int PHI>
__global__ __launch_bounds__(256) void lin_fwd_generic_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ den, float* __restrict__ zcache,
    float* __restrict__ state, float* __restrict__ zfin, int den_incl_eps, int S, int D, int E)
{
    extern __shared__ float sm[];
    float* z = sm;            // D
    float* pq = sm + D;       // D: phi(Q_t)
    float* pk = sm + 2 * D;   // D: phi(K_t)
    float* red = sm + 3 * D;  // 256
    const int tid = threadIdx.x;
    const long seq = blockIdx.x;
    float* St = state + seq * (long)D * E;
    for (int i = tid; i < D * E; i += 256)
        St[i] = 0.0f;
    for (int i = tid; i < D; i += 256)
        z[i] = 0.0f;
    __syncthreads();
    for (int t = 0; t < S; t++) {
        const long row = seq * S + t;
        for (int d = tid; d < D; d += 256) {
            pq[d] = Phi<PHI>::f(Q[row * D + d]);
            pk[d] = Phi<PHI>::f(K[row * D + d]);
            z[d] += pk[d];
            if (zcache != nullptr)
                zcache[row * D + d] = z[d];
        }
        __syncthreads();
        for (int i = tid; i < D * E; i += 256) {
            const int d = i / E, e = i - d * E;
            St[i] += pk[d] * V[row * E + e];
        }
        float part = 0.0f;
        for (int d = tid; d < D; d += 256)
            part += pq[d] * z[d];
        red[tid] = part;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (tid < s)
                red[tid] += red[tid + s];
            __syncthreads();
        }
        const float dn = red[0];
        for (int e = tid; e < E; e += 256) {
            float num = 0.0f;
            for (int d = 0; d < D; d++)
                num += pq[d] * St[(long)d * E + e];
            O[row * E + e] = num / (dn + 1e-8f);
        }
        if (tid == 0)
            den[row] = den_incl_eps ? dn + 1e-8f : dn;
        __syncthreads();
    }
    if (zfin != nullptr)
        for (int d = tid; d < D; d += 256)
            zfin[seq * D + d] = z[d];
}

template <int PHI>
__global__ __launch_bounds__(256) void lin_dq_generic_kernel(
    const float* __restrict__ K, const float* __restrict__ V, const float* __restrict__ dnum,
    const float* __restrict__ dden, const float* __restrict__ zcache, const float* __restrict__ Q,
    float* __restrict__ dQ, float* __restrict__ state, int S, int D, int E)
{
    const int tid = threadIdx.x;
    const long seq = blockIdx.x;
    float* St = state + seq * (long)D * E;
    for (int i = tid; i < D * E; i += 256)
        St[i] = 0.0f;
    __syncthreads();
    for (int t = 0; t < S; t++) {
        const long row = seq * S + t;
        for (int i = tid; i < D * E; i += 256) {
            const int d = i / E, e = i - d * E;
            St[i] += Phi<PHI>::f(K[row * D + d]) * V[row * E + e];
        }
        __syncthreads();
        const float dd = dden[row];
        for (int d = tid; d < D; d += 256) {
            float acc = zcache[row * D + d] * dd;
            for (int e = 0; e < E; e++)
                acc += St[(long)d * E + e] * dnum[row * E + e];
            dQ[row * D + d] = acc * Phi<PHI>::d(Q[row * D + d]);
        }
        __syncthreads();
    }
}

template <int PHI>
__global__ __launch_bounds__(256) void lin_dkdv_generic_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dnum, const float* __restrict__ dden, float* __restrict__ dK,
    float* __restrict__ dV, float* __restrict__ state, int S, int D, int E)
{
    extern __shared__ float sm[];
    float* zs = sm;   // D
    const int tid = threadIdx.x;
    const long seq = blockIdx.x;
    float* St = state + seq * (long)D * E;
    for (int i = tid; i < D * E; i += 256)
        St[i] = 0.0f;
    for (int i = tid; i < D; i += 256)
        zs[i] = 0.0f;
    __syncthreads();
    for (int t = S - 1; t >= 0; t--) {
        const long row = seq * S + t;
        const float dd = dden[row];
        for (int i = tid; i < D * E; i += 256) {
            const int d = i / E, e = i - d * E;
            St[i] += Phi<PHI>::f(Q[row * D + d]) * dnum[row * E + e];
        }
        for (int d = tid; d < D; d += 256)
            zs[d] += Phi<PHI>::f(Q[row * D + d]) * dd;
        __syncthreads();
        for (int e = tid; e < E; e += 256) {
            float acc = 0.0f;
            for (int d = 0; d < D; d++)
                acc += St[(long)d * E + e] * Phi<PHI>::f(K[row * D + d]);
            dV[row * E + e] = acc;
        }
        for (int d = tid; d < D; d += 256) {
            float acc = zs[d];
            for (int e = 0; e < E; e++)
                acc += St[(long)d * E + e] * V[row * E + e];
            dK[row * D + d] = acc * Phi<PHI>::d(K[row * D + d]);
        }
        __syncthreads();
    }
}

// Copy a [d][e] state to the caller's layout ([d][e] or [e][d]).
__global__ void lin_state_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                      long Bq, int D, int E, int de)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= Bq * D * E)
        return;
    const long seq = i / ((long)D * E);
    const long rem = i - seq * D * E;
    const int d = (int)(rem / E), e = (int)(rem - (long)d * E);
    dst[seq * D * E + (de ? (long)d * E + e : (long)e * D + d)] = src[i];
}

// ---------------------------------------------------------------------------
// feature-map kernels (linear_cuda API): phi_elu and Hadamard+Exp
// ---------------------------------------------------------------------------
// phi_elu_fwd_kernel (linear_cuda_kernels.cu:305-325): (expf(x) - 1) + 1 kept as written.
__global__ void phi_elu_fwd_kernel(const float* __restrict__ x, float* __restrict__ phi, long N,
                                   int D, int E)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= N * D)
        return;
    const long n = i / D;
    const int j = (int)(i - n * D);
    float out = 0.0f;
    if (j < E) {
        const float xv = x[n * E + j];
        const float elu = xv > 0.0f ? xv : expf(xv) - 1.0f;
        out = elu + 1.0f;
    }
    phi[i] = out;
}

__global__ void phi_elu_bwd_kernel(const float* __restrict__ dphi, const float* __restrict__ x,
                                   float* __restrict__ dx, long N, int D, int E)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= N * E)
        return;
    const long n = i / E;
    const int j = (int)(i - n * E);
    const float xv = x[i];
    dx[i] = dphi[n * D + j] * (xv > 0.0f ? 1.0f : expf(xv));
}

// In-wave fast Walsh-Hadamard transform of a 64-vector held one element per
// lane: y_i = sum_j (-1)^popcount(i&j) x_j.
__device__ __forceinline__ float fwht64(float v, int lane)
{
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float u = __shfl_xor(v, m, 64);
        v = (lane & m) ? (u - v) : (v + u);
    }
    return v;
}

// One wave per (row, 64-column block); columns >= E of phi are zeroed by the
// extra blocks of the grid's x range.
__global__ __launch_bounds__(256) void phi_hexp_fwd_kernel(const float* __restrict__ x,
                                                          float* __restrict__ phi, long N, int D,
                                                          int E)
{
    const int lane = threadIdx.x & 63;
    const long w = ((long)blockIdx.x * 256 + threadIdx.x) >> 6;
    const int nblk = (D + 63) / 64;
    if (w >= N * nblk)
        return;
    const long n = w / nblk;
    const int blk = (int)(w - n * nblk);
    const int c = 64 * blk + lane;
    if (64 * blk + 64 <= E) {
        const float y = fwht64(x[n * E + c], lane);
        phi[n * D + c] = __expf(y * 0.125f);
    } else if (c < D) {
        phi[n * D + c] = 0.0f;
    }
}

__global__ __launch_bounds__(256) void phi_hexp_bwd_kernel(const float* __restrict__ dphi,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ dx, long N, int D,
                                                          int E)
{
    const int lane = threadIdx.x & 63;
    const long w = ((long)blockIdx.x * 256 + threadIdx.x) >> 6;
    const int nblk = E / 64;
    if (w >= N * nblk)
        return;
    const long n = w / nblk;
    const int blk = (int)(w - n * nblk);
    const int c = 64 * blk + lane;
    const float y = fwht64(x[n * E + c], lane);
    const float p = __expf(y * 0.125f);
    const float t = fwht64(dphi[n * D + c] * p, lane);
    dx[n * E + c] = t * 0.125f;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline bool al16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

LinPlan lin_plan(int Bq, int S, int D, int E)
{
    LinPlan p;
    p.fast = (D <= 64 && E <= 64);
    p.nseg = 1;
    p.L = S;
    if (p.fast) {
        const int nchunk = (S + 15) / 16;
        // enough waves to cover the chip a few times, segments of >= 1 chunk
        int want = (2048 + Bq - 1) / Bq;
        if (want < 1)
            want = 1;
        if (want > nchunk)
            want = nchunk;
        const int cps = (nchunk + want - 1) / want;   // chunks per segment
        p.L = 16 * cps;
        p.nseg = (S + p.L - 1) / p.L;
    }
    return p;
}

size_t lin_ws_bytes(const LinPlan& p, int Bq, int D, int E)
{
    if (!p.fast)
        return (size_t)Bq * D * E * sizeof(float);
    if (p.nseg <= 1)
        return 0;
    return (size_t)Bq * p.nseg * LIN_WS * sizeof(float);
}

template <int PHI>
static hipError_t agg_and_scan(const LinPlan& p, const float* X, const float* Y, const float* w,
                               float* ws, int Bq, int S, int D, int E, int reverse, bool vec,
                               hipStream_t st)
{
    const int nw = Bq * p.nseg;
    dim3 grid((unsigned)((nw + LIN_WAVES - 1) / LIN_WAVES)), block(LIN_THREADS);
    {
        ProfScope ps(st, "lin_agg");
        if (vec)
            hipLaunchKernelGGL((lin_agg_kernel<PHI, true>), grid, block, 0, st, X, Y, w, ws, Bq,
                               S, D, E, p.nseg, p.L);
        else
            hipLaunchKernelGGL((lin_agg_kernel<PHI, false>), grid, block, 0, st, X, Y, w, ws, Bq,
                               S, D, E, p.nseg, p.L);
    }
    {
        ProfScope ps(st, "lin_scan");
        const long n = (long)Bq * LIN_WS;
        hipLaunchKernelGGL(lin_scan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           ws, Bq, p.nseg, reverse);
    }
    return hipGetLastError();
}

template <int PHI>
static hipError_t fwd_impl(const float* Q, const float* K, const float* V, float* O, float* den,
                           float* zc, float* Sfin, float* zfin, int sfin_de, int den_eps, int Bq,
                           int S, int D, int E, void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E);
    if (!p.fast) {
        float* state = (float*)ws;
        const size_t sm = (size_t)(3 * D + 256) * sizeof(float);
        {
            ProfScope ps(st, "lin_fwd_generic");
            hipLaunchKernelGGL((lin_fwd_generic_kernel<PHI>), dim3(Bq), dim3(256), sm, st, Q, K,
                               V, O, den, zc, state, zfin, den_eps, S, D, E);
        }
        if (Sfin != nullptr) {
            const long n = (long)Bq * D * E;
            hipLaunchKernelGGL(lin_state_copy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                               0, st, state, Sfin, (long)Bq, D, E, sfin_de);
        }
        return hipGetLastError();
    }
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(Q) && al16(K) && al16(V) && al16(O) &&
                     al16(zc);
    float* wsf = (float*)ws;
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, K, V, nullptr, wsf, Bq, S, D, E, 0, vec, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    const int nw = Bq * p.nseg;
    dim3 grid((unsigned)((nw + LIN_WAVES - 1) / LIN_WAVES)), block(LIN_THREADS);
    ProfScope ps(st, "lin_fwd");
    if (vec)
        hipLaunchKernelGGL((lin_fwd_kernel<PHI, true>), grid, block, 0, st, Q, K, V, O, den, zc,
                           wsf, Sfin, zfin, sfin_de, den_eps, Bq, S, D, E, p.nseg, p.L);
    else
        hipLaunchKernelGGL((lin_fwd_kernel<PHI, false>), grid, block, 0, st, Q, K, V, O, den, zc,
                           wsf, Sfin, zfin, sfin_de, den_eps, Bq, S, D, E, p.nseg, p.L);
    return hipGetLastError();
}

hipError_t lin_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                          float* den, float* zc, float* Sfin, float* zfin, int sfin_de,
                          int den_eps, int Bq, int S, int D, int E, void* ws, hipStream_t st)
{
    if (phi == PHI_ELU1)
        return fwd_impl<PHI_ELU1>(Q, K, V, O, den, zc, Sfin, zfin, sfin_de, den_eps, Bq, S, D, E,
                                  ws, st);
    return fwd_impl<PHI_NONE>(Q, K, V, O, den, zc, Sfin, zfin, sfin_de, den_eps, Bq, S, D, E, ws,
                              st);
}

hipError_t lin_step1_launch(const float* O, const float* dO, const float* den, float* dnum,
                            float* dden, long N, int E, hipStream_t st)
{
    const bool vec = (E % 4 == 0) && al16(O) && al16(dO) && al16(dnum);
    dim3 grid((unsigned)((N * 16 + 255) / 256)), block(256);
    ProfScope ps(st, "lin_step1");
    if (vec)
        hipLaunchKernelGGL((lin_step1_kernel<true>), grid, block, 0, st, O, dO, den, dnum, dden,
                           N, E);
    else
        hipLaunchKernelGGL((lin_step1_kernel<false>), grid, block, 0, st, O, dO, den, dnum, dden,
                           N, E);
    return hipGetLastError();
}

template <int PHI>
static hipError_t dq_impl(const float* K, const float* V, const float* dnum, const float* dden,
                          const float* zc, const float* Q, float* dQ, int Bq, int S, int D, int E,
                          void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E);
    if (!p.fast) {
        ProfScope ps(st, "lin_dq_generic");
        hipLaunchKernelGGL((lin_dq_generic_kernel<PHI>), dim3(Bq), dim3(256), 0, st, K, V, dnum,
                           dden, zc, Q, dQ, (float*)ws, S, D, E);
        return hipGetLastError();
    }
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(K) && al16(V) && al16(dnum) &&
                     al16(zc) && al16(Q) && al16(dQ);
    float* wsf = (float*)ws;
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, K, V, nullptr, wsf, Bq, S, D, E, 0, vec, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    const int nw = Bq * p.nseg;
    dim3 grid((unsigned)((nw + LIN_WAVES - 1) / LIN_WAVES)), block(LIN_THREADS);
    ProfScope ps(st, "lin_dq");
    if (vec)
        hipLaunchKernelGGL((lin_dq_kernel<PHI, true>), grid, block, 0, st, K, V, dnum, dden, zc,
                           Q, dQ, wsf, Bq, S, D, E, p.nseg, p.L);
    else
        hipLaunchKernelGGL((lin_dq_kernel<PHI, false>), grid, block, 0, st, K, V, dnum, dden, zc,
                           Q, dQ, wsf, Bq, S, D, E, p.nseg, p.L);
    return hipGetLastError();
}

hipError_t lin_dq_launch(int phi, const float* K, const float* V, const float* dnum,
                         const float* dden, const float* zc, const float* Q, float* dQ, int Bq,
                         int S, int D, int E, void* ws, hipStream_t st)
{
    if (phi == PHI_ELU1)
        return dq_impl<PHI_ELU1>(K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, ws, st);
    return dq_impl<PHI_NONE>(K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, ws, st);
}

template <int PHI>
static hipError_t dkdv_impl(const float* Q, const float* K, const float* V, const float* dnum,
                            const float* dden, float* dK, float* dV, int Bq, int S, int D, int E,
                            void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E);
    if (!p.fast) {
        ProfScope ps(st, "lin_dkdv_generic");
        hipLaunchKernelGGL((lin_dkdv_generic_kernel<PHI>), dim3(Bq), dim3(256),
                           (size_t)D * sizeof(float), st, Q, K, V, dnum, dden, dK, dV, (float*)ws,
                           S, D, E);
        return hipGetLastError();
    }
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(Q) && al16(K) && al16(V) &&
                     al16(dnum) && al16(dK) && al16(dV);
    float* wsf = (float*)ws;
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, Q, dnum, dden, wsf, Bq, S, D, E, 1, vec, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    const int nw = Bq * p.nseg;
    dim3 grid((unsigned)((nw + LIN_WAVES - 1) / LIN_WAVES)), block(LIN_THREADS);
    ProfScope ps(st, "lin_dkdv");
    if (vec)
        hipLaunchKernelGGL((lin_dkdv_kernel<PHI, true>), grid, block, 0, st, Q, K, V, dnum, dden,
                           dK, dV, wsf, Bq, S, D, E, p.nseg, p.L);
    else
        hipLaunchKernelGGL((lin_dkdv_kernel<PHI, false>), grid, block, 0, st, Q, K, V, dnum, dden,
                           dK, dV, wsf, Bq, S, D, E, p.nseg, p.L);
    return hipGetLastError();
}

hipError_t lin_dkdv_launch(int phi, const float* Q, const float* K, const float* V,
                           const float* dnum, const float* dden, float* dK, float* dV, int Bq,
                           int S, int D, int E, void* ws, hipStream_t st)
{
    if (phi == PHI_ELU1)
        return dkdv_impl<PHI_ELU1>(Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, ws, st);
    return dkdv_impl<PHI_NONE>(Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, ws, st);
}

hipError_t phi_elu_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st)
{
    const long n = N * D;
    ProfScope ps(st, "phi_elu_fwd");
    hipLaunchKernelGGL(phi_elu_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x,
                       phi, N, D, E);
    return hipGetLastError();
}

hipError_t phi_elu_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D, int E,
                              hipStream_t st)
{
    const long n = N * E;
    ProfScope ps(st, "phi_elu_bwd");
    hipLaunchKernelGGL(phi_elu_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       dphi, x, dx, N, D, E);
    return hipGetLastError();
}

hipError_t phi_hexp_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st)
{
    const long waves = N * ((D + 63) / 64);
    ProfScope ps(st, "phi_hexp_fwd");
    hipLaunchKernelGGL(phi_hexp_fwd_kernel, dim3((unsigned)((waves * 64 + 255) / 256)), dim3(256),
                       0, st, x, phi, N, D, E);
    return hipGetLastError();
}

hipError_t phi_hexp_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D,
                               int E, hipStream_t st)
{
    const long waves = N * (E / 64);
    ProfScope ps(st, "phi_hexp_bwd");
    hipLaunchKernelGGL(phi_hexp_bwd_kernel, dim3((unsigned)((waves * 64 + 255) / 256)), dim3(256),
                       0, st, dphi, x, dx, N, D, E);
    return hipGetLastError();
}

} // namespace cxg
