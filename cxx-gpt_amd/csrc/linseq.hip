// linseq.hip -- segment records of short sequences in one pass, and the whole
// forward of sequences of at most 16 chunks in one launch (gfx950).
//
// The chunked linear-attention scans of the forward, dQ and dK/dV passes
// (linattn.hip) start each segment of a sequence from a record of the
// segments before it (forward, dQ) or after it (dK/dV): the 64x64 state sum
// sum_t phi(X_t)^T Y_t ([d][e]) and the z sum sum_t w_t phi(X_t) over those
// segments.  Long sequences form the records with two launches: per-segment
// aggregates (lin_agg), then a scan over each sequence's segments (lin_scan).
// For a sequence of a few hundred rows both are bound by start-up and memory
// round trips rather than by work.  Here two workgroups of 16 waves take one
// sequence, one per half of the state's columns:
//   1. wave w sums chunks [w cpw, (w+1) cpw) (cpw chunks per wave, a divisor
//      of the segment's chunk count, so a segment is a run of whole waves)
//      into a 64x32 MFMA accumulator, its operands read from global memory
//      directly in the MFMA column layout, a chunk's loads all in flight;
//   2. two passes over 16-column slices of the state: every wave puts its
//      slice in LDS, then thread j reads element j of all waves and walks them
//      in scan order, writing the records directly.
// Measured on MI355X at B' = 96, S = 256, D = E = 64 (8 segments of 2
// chunks): 10.8 us against 7.2 + 5.1 us for the pair.  The fused backward's
// records (lin_bagg + lin_bscan, which also form dnum and dden from O, dO and
// den) took no less time in this form and stay with the pair.
#include "common.hpp"
#include "launch.hpp"
#include "linattn.hpp"
#include "linattn_dev.hpp"

namespace cxg {

constexpr int SEQ_WAVES = 16;
constexpr int SEQ_THREADS = 64 * SEQ_WAVES;
constexpr int SEQ_SLOT = 1024 + 64;   // one wave's 16-column state slice + z

// Chunks per wave for a sequence of nch chunks in segments of cps chunks: the
// smallest divisor of cps that leaves at most SEQ_WAVES waves; 0 when neither
// 1 nor 2 does (the two-launch path then runs: with more chunks per wave this
// pass is slower than the pair).
int lin_seq_cpw(int nch, int cps)
{
    for (int d = 1; d <= 2; d++)
        if (cps % d == 0 && (nch + d - 1) / d <= SEQ_WAVES)
            return d;
    return 0;
}

// Buffer descriptor over n bytes from base: loads past the end read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seq_rsrc(const float* base, long n)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                             base != nullptr ? (int)n : 0, 0x00020000);
}

// Workgroup b -> (sequence, column half).  The dispatcher deals workgroups to
// the 8 XCDs round-robin (b % 8); b and b + 8 share an XCD and so its L2, and
// they take the two halves of one sequence, whose X rows the second then
// reads from L2.
__device__ __forceinline__ void seq_half(int b, int& seq, int& h)
{
    seq = (b >> 4) * 8 + (b & 7);
    h = (b >> 3) & 1;
}

// Records of sequence seq, state columns of tiles 2h, 2h+1 (and z from h = 0):
// REV = false exclusive prefix over segments, true exclusive suffix; w
// (nullable) weights z's rows (1 when null).
template <int PHI, bool REV, bool FW>
__global__ __launch_bounds__(SEQ_THREADS) void lin_seqrec_kernel(
    const float* __restrict__ X, const float* __restrict__ Y, const float* __restrict__ wgt,
    float* __restrict__ ws, int nseq, int S, int D, int E, int cpw, int wps, int nseg)
{
    __shared__ __attribute__((aligned(16))) float lds[SEQ_WAVES * SEQ_SLOT];
    int seq, h;
    seq_half(blockIdx.x, seq, h);
    if (seq >= nseq)
        return;
    if (FW) {   // compile-time widths
        D = 64;
        E = 64;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int nch = (S + 15) / 16;
    const int nw = (nch + cpw - 1) / cpw;
    const long rb = (long)seq * S;
    float* rec = ws + (long)seq * nseg * LIN_WS;

    // acc[dt][jj]: lane (l16, g), element r <-> state[d = 16dt + 4g + r][e = 16(2h + jj) + l16]
    f4 acc[4][2];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int jj = 0; jj < 2; jj++)
            acc[dt][jj] = f4zero();
    float zp[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // z partial of column 16dt + l16, rows 4g..4g+3

    // Descriptors over this sequence's rows (at most 2 * 16 * 16 rows of at
    // most 64 floats); with D = E = 64 rows past S read 0 through the range
    // check, so a chunk's loads need no clamp.
    const __amdgpu_buffer_rsrc_t rX = seq_rsrc(X + rb * D, (long)S * D * 4);
    const __amdgpu_buffer_rsrc_t rY = seq_rsrc(Y + rb * E, (long)S * E * 4);
    const __amdgpu_buffer_rsrc_t rw = seq_rsrc(wgt != nullptr ? wgt + rb : nullptr, (long)S * 4);
    const int c0 = wv * cpw, c1 = min(nch, c0 + cpw);
    for (int c = c0; c < c1; c++) {
        // Operands in the MFMA column layout: lane (l16, g), instruction r holds
        // row 16c + 4g + r, column 16 * tile + l16.
        float x[4][4], y[2][4], wr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 16 * c + 4 * g + r;
            const unsigned tr = FW ? (unsigned)t : (unsigned)min(t, S - 1);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int cx = FW ? 16 * k + l16 : min(16 * k + l16, D - 1);
                x[k][r] = buffer_load_f32(rX, (tr * (unsigned)D + cx) * 4u);
            }
#pragma unroll
            for (int jj = 0; jj < 2; jj++) {
                const int cy = FW ? 16 * (2 * h + jj) + l16 : min(16 * (2 * h + jj) + l16, E - 1);
                y[jj][r] = buffer_load_f32(rY, (tr * (unsigned)E + cy) * 4u);
            }
            wr[r] = wgt != nullptr ? buffer_load_f32(rw, tr * 4u) : 1.0f;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool rok = 16 * c + 4 * g + r < S;
            if constexpr (PHI == PHI_HEXP) {
                // row 16c + 4g + r: columns 16k + l16 over the 16-lane group
                float xr[4] = {x[0][r], x[1][r], x[2][r], x[3][r]};
                hexp_colC(xr, lane);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    x[k][r] = rok ? xr[k] : 0.0f;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    x[k][r] = (rok && (FW || 16 * k + l16 < D)) ? Phi<PHI>::f(x[k][r]) : 0.0f;
            }
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
                y[jj][r] = (rok && (FW || 16 * (2 * h + jj) + l16 < E)) ? y[jj][r] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int jj = 0; jj < 2; jj++)
                    acc[dt][jj] = mfma16(x[dt][r], y[jj][r], acc[dt][jj]);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                zp[dt] += wr[r] * x[dt][r];
    }
    float zs[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        zs[dt] = xrow_sum(zp[dt]);

    // Scan: pass jj publishes state columns of tile 2h + jj of every wave (slot
    // element (dt * 4 + r) * 64 + lane) and, in pass 0 of h = 0, z; thread j
    // then reads element j of every wave and walks them in scan order.
    const int j = threadIdx.x;
    const int jdt = j >> 8, jr = (j >> 6) & 3, jl = j & 63;
    const int jd = 16 * jdt + 4 * (jl >> 4) + jr;   // state row of element j
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
        float* slot = lds + wv * SEQ_SLOT;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                slot[(dt * 4 + r) * 64 + lane] = acc[dt][jj][r];
        if (jj == 0 && h == 0 && g == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                slot[1024 + 16 * dt + l16] = zs[dt];
        __syncthreads();
        const bool wz = jj == 0 && h == 0 && j < 64;   // this thread also walks z[j]
        float v[SEQ_WAVES], vz[SEQ_WAVES];
#pragma unroll
        for (int k = 0; k < SEQ_WAVES; k++) {
            v[k] = k < nw ? lds[k * SEQ_SLOT + j] : 0.0f;
            vz[k] = (wz && k < nw) ? lds[k * SEQ_SLOT + 1024 + j] : 0.0f;
        }
        float* rj = rec + jd * 64 + 16 * (2 * h + jj) + (jl & 15);   // [d][e] element of j
        float* rz = rec + 4096 + j;
        float run = 0.0f, runz = 0.0f;
        if (!REV) {
            // record s = sum over the waves of segments < s
            int pos = 0;
            long so = 0;
#pragma unroll
            for (int k = 0; k < SEQ_WAVES; k++) {
                if (k < nw) {
                    if (pos == 0) {
                        rj[so] = run;
                        if (wz)
                            rz[so] = runz;
                    }
                    run += v[k];
                    runz += vz[k];
                    if (++pos == wps) {
                        pos = 0;
                        so += LIN_WS;
                    }
                }
            }
        } else {
            // record s = sum over the waves of segments > s: walk down from the
            // last wave; the last wave of a segment writes its record first
            const int slast = (nw - 1) / wps;
            int pos = nw - 1 - slast * wps;   // position of wave k in its segment
            long so = (long)slast * LIN_WS;
#pragma unroll
            for (int k = SEQ_WAVES - 1; k >= 0; k--) {
                if (k < nw) {
                    if (k == nw - 1 || pos == wps - 1) {
                        rj[so] = run;
                        if (wz)
                            rz[so] = runz;
                    }
                    run += v[k];
                    runz += vz[k];
                    if (--pos < 0) {
                        pos = wps - 1;
                        so -= LIN_WS;
                    }
                }
            }
        }
        __syncthreads();   // the slots are rewritten by the next pass
    }
}

// two workgroups per sequence, in whole groups of 8 sequences (seq_half)
static unsigned seq_grid(int nseq) { return (unsigned)(16 * ((nseq + 7) / 8)); }

template <int PHI>
hipError_t lin_seqrec_launch(const float* X, const float* Y, const float* w, float* ws, int Bq,
                             int S, int D, int E, int L, int nseg, int reverse, hipStream_t st)
{
    const int nch = (S + 15) / 16, cps = L / 16;
    const int cpw = lin_seq_cpw(nch, cps);
    if (cpw == 0)
        return hipErrorInvalidValue;
    const int wps = cps / cpw;
    const bool fw = D == 64 && E == 64;
    if (PHI == PHI_HEXP && !fw)
        return hipErrorInvalidValue;
    const dim3 grid(seq_grid(Bq)), block(SEQ_THREADS);
    ProfScope ps(st, "lin_seqrec");
    if (reverse) {
        if (fw)
            CXG_LAUNCH((lin_seqrec_kernel<PHI, true, true>), grid, block, 0, st, X, Y, w,
                               ws, Bq, S, D, E, cpw, wps, nseg);
        else if constexpr (PHI != PHI_HEXP)
            CXG_LAUNCH((lin_seqrec_kernel<PHI, true, false>), grid, block, 0, st, X, Y, w,
                               ws, Bq, S, D, E, cpw, wps, nseg);
    } else {
        if (fw)
            CXG_LAUNCH((lin_seqrec_kernel<PHI, false, true>), grid, block, 0, st, X, Y, w,
                               ws, Bq, S, D, E, cpw, wps, nseg);
        else if constexpr (PHI != PHI_HEXP)
            CXG_LAUNCH((lin_seqrec_kernel<PHI, false, false>), grid, block, 0, st, X, Y,
                               w, ws, Bq, S, D, E, cpw, wps, nseg);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The whole forward of sequences of at most 16 chunks (S <= 256) at
// D = E = 64 in one launch: two workgroups of 16 waves per sequence (state
// columns halves h), wave c takes chunk c.
//   1. chunk c's state sum phi(K_c)^T V_c (its column half) and z sum, as the
//      records pass forms them;
//   2. exclusive prefix over the waves through LDS (two 32-column passes):
//      thread j walks element j across the waves, writes each wave's prefix
//      back into its slot and, on the way, the segment records the backward
//      may take, the anchors, the z table and the final state (context and
//      Sfin/zfin outputs, all nullable);
//   3. the chunk's outputs from its prefix state, as the chunked forward forms
//      them: A^T = phi(K_c) phi(Q_c)^T masked, den = phi(Q) . z_prev + row sums
//      of A, O = (phi(Q) S_prev + A V) / (den + 1e-8), z_cache rows.
// Replaces the records launch and the forward kernel (C3 S256: 10.8 + 15.2 us).
// ---------------------------------------------------------------------------
template <int PHI>
__global__ __launch_bounds__(SEQ_THREADS) void lin_seqfwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ den, float* __restrict__ zcache,
    float* __restrict__ rec, int nseg, int cps, float* __restrict__ Sfin,
    float* __restrict__ zfin, int sfin_de, float* __restrict__ ctot, float* __restrict__ ztab,
    float* __restrict__ anch, int den_eps, int nseq, int S)
{
    __shared__ __attribute__((aligned(16))) float lds[SEQ_WAVES * SEQ_SLOT];
    int seq, h;
    seq_half(blockIdx.x, seq, h);
    if (seq >= nseq)
        return;   // the whole workgroup
    const int lane = threadIdx.x & 63;
    const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // this wave's chunk
    const int l16 = lane & 15, g = lane >> 4;
    const int nch = (S + 15) / 16;
    const long rb = (long)seq * S;
    const __amdgpu_buffer_rsrc_t rQ = seq_rsrc(Q + rb * 64, (long)S * 64 * 4);
    const __amdgpu_buffer_rsrc_t rK = seq_rsrc(K + rb * 64, (long)S * 64 * 4);
    const __amdgpu_buffer_rsrc_t rV = seq_rsrc(V + rb * 64, (long)S * 64 * 4);

    // 1. column layout: lane (l16, g), instruction r <-> row 16c + 4g + r,
    // column 16k + l16 (rows past S, and chunks past the sequence, read 0)
    float x[4][4], y[2][4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const unsigned t = (unsigned)(16 * c + 4 * g + r);
#pragma unroll
        for (int k = 0; k < 4; k++)
            x[k][r] = buffer_load_f32(rK, (t * 64u + 16 * k + l16) * 4u);
#pragma unroll
        for (int jj = 0; jj < 2; jj++)
            y[jj][r] = buffer_load_f32(rV, (t * 64u + 16 * (2 * h + jj) + l16) * 4u);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const bool rok = 16 * c + 4 * g + r < S;
#pragma unroll
        for (int k = 0; k < 4; k++)
            x[k][r] = rok ? Phi<PHI>::f(x[k][r]) : 0.0f;
    }
    f4 acc[4][2];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            f4 a = f4zero();
#pragma unroll
            for (int r = 0; r < 4; r++)
                a = mfma16(x[dt][r], y[jj][r], a);
            acc[dt][jj] = a;   // state[d = 16dt + 4g + r][e = 16(2h + jj) + l16]
        }
    float zs[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        zs[dt] = xrow_sum((x[dt][0] + x[dt][1]) + (x[dt][2] + x[dt][3]));
    // 3's row-layout operands, requested now so that they arrive during the
    // scan: lane (row l16, g), columns 16dt + 4g .. +3
    const int trow = 16 * c + l16;
    const bool tok = trow < S;
    f4 qr[4], kr[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        qr[dt] = buffer_load_f4(rQ, ((unsigned)trow * 64u + 16 * dt + 4 * g) * 4u);
        kr[dt] = buffer_load_f4(rK, ((unsigned)trow * 64u + 16 * dt + 4 * g) * 4u);
    }

    // 2. exclusive prefix over the chunks
    const int j = threadIdx.x;
    const int jdt = j >> 8, jr = (j >> 6) & 3, jl = j & 63;
    const int jd = 16 * jdt + 4 * (jl >> 4) + jr;   // state row of element j
    const int nanch = lin_nanch(nch);
    float* slot = lds + c * SEQ_SLOT;
    f4 zrow[4];
    float zcol[4];
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                slot[(dt * 4 + r) * 64 + lane] = acc[dt][jj][r];
        if (jj == 0 && g == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                slot[1024 + 16 * dt + l16] = zs[dt];
        __syncthreads();
        {
            const int je = 16 * (2 * h + jj) + (jl & 15);   // state column of element j
            const bool wz = jj == 0 && j < 64;              // this thread also walks z[j]
            float run = 0.0f, runz = 0.0f;
            float* rs = rec != nullptr ? rec + (long)seq * nseg * LIN_WS : nullptr;   // segment 0
            float* an = anch != nullptr ? anch + (long)seq * nanch * LIN_ANCH : nullptr;
            float* zt = (ztab != nullptr && h == 0) ? ztab + (long)seq * nch * 64 : nullptr;
            int pos = 0;   // chunk k's position in its segment
#pragma unroll
            for (int k = 0; k < SEQ_WAVES; k++) {
                if (k < nch) {
                    float* sk = lds + k * SEQ_SLOT;
                    const float v = sk[j];
                    sk[j] = run;
                    if (rs != nullptr && pos == 0)
                        rs[jd * 64 + je] = run;
                    if (k > 0 && (k & (k - 1)) == 0 && an != nullptr)   // anchor before chunk 2^m
                        an[__builtin_ctz(k) * LIN_ANCH + jd * 64 + je] = run;
                    run += v;
                    if (wz) {
                        const float vz = sk[1024 + j];
                        sk[1024 + j] = runz;
                        if (h == 0 && rs != nullptr && pos == 0)
                            rs[4096 + j] = runz;
                        if (zt != nullptr)
                            zt[k * 64 + j] = runz;
                        runz += vz;
                    }
                    if (++pos == cps) {
                        pos = 0;
                        if (rs != nullptr)
                            rs += LIN_WS;
                    }
                }
            }
            if (ctot != nullptr)
                ctot[(long)seq * LIN_WS + jd * 64 + je] = run;
            if (Sfin != nullptr)
                Sfin[(long)seq * 4096 + (sfin_de ? jd * 64 + je : je * 64 + jd)] = run;
            if (wz && h == 0) {
                if (ctot != nullptr)
                    ctot[(long)seq * LIN_WS + 4096 + j] = runz;
                if (zfin != nullptr)
                    zfin[(long)seq * 64 + j] = runz;
            }
        }
        __syncthreads();
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc[dt][jj][r] = slot[(dt * 4 + r) * 64 + lane];   // now the prefix
        if (jj == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                zrow[dt] = *reinterpret_cast<const f4*>(&slot[1024 + 16 * dt + 4 * g]);
                zcol[dt] = slot[1024 + 16 * dt + l16];
            }
        __syncthreads();   // the slots are rewritten by the next pass
    }
    if (c >= nch)
        return;   // the wave (no barrier follows)

    // 3. outputs of chunk c
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qr[dt][i] = Phi<PHI>::f(qr[dt][i]);
            kr[dt][i] = tok ? Phi<PHI>::f(kr[dt][i]) : 0.0f;
        }
    // A^T[s = 4g + r][t = l16] = phi(K_s) . phi(Q_t), kept for s <= t
    f4 At = f4zero();
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            At = mfma16(kr[dt][i], qr[dt][i], At);
    float dpart = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        At[r] = (4 * g + r <= l16) ? At[r] : 0.0f;
        dpart += At[r];
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        dpart += (qr[dt][0] * zrow[dt][0] + qr[dt][1] * zrow[dt][1]) +
                 (qr[dt][2] * zrow[dt][2] + qr[dt][3] * zrow[dt][3]);
    const float dn = xrow_sum(dpart);
    const float inv = __builtin_amdgcn_rcpf(dn + 1e-8f);
    const __amdgpu_buffer_rsrc_t rO = buf_rsrc(O + (rb + 16 * c) * 64);
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
        // O^T[e = 16(2h + jj) + 4g + r][t = l16] = sum_d S[d][e] phi(Q_t)[d] + sum_s V_s[e] A^T[s][t]
        f4 o = f4zero();
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                o = mfma16(acc[dt][jj][r], qr[dt][r], o);
#pragma unroll
        for (int r = 0; r < 4; r++)
            o = mfma16(y[jj][r], At[r], o);
        buffer_store_f4(rO, tok ? (unsigned)(l16 * 64 + 16 * (2 * h + jj) + 4 * g) * 4u
                                : kDropOffset,
                        o * inv);
    }
    if (h == 0) {
        if (g == 0 && tok)
            den[rb + trow] = den_eps ? dn + 1e-8f : dn;
        if (zcache != nullptr) {
            // z_t = z before the chunk + inclusive prefix of phi(K) over the
            // chunk (phi(K) in the column layout again, from L2)
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                f4 xc;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = 16 * c + 4 * g + r;
                    const float xv = buffer_load_f32(rK, ((unsigned)t * 64u + 16 * dt + l16) * 4u);
                    xc[r] = t < S ? Phi<PHI>::f(xv) : 0.0f;
                }
                float tot;
                const f4 zp = col_prefix16(xc, tot, lane) + zcol[dt];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = 16 * c + 4 * g + r;
                    if (t < S)
                        zcache[(rb + t) * 64 + 16 * dt + l16] = zp[r];
                }
            }
        }
    }
}

bool lin_seqfwd_ok(int S) { return S >= 1 && (S + 15) / 16 <= SEQ_WAVES; }

template <int PHI>
hipError_t lin_seqfwd_launch(const float* Q, const float* K, const float* V, float* O, float* den,
                             float* zc, float* rec, int nseg, int L, float* Sfin, float* zfin,
                             int sfin_de, float* ctot, float* ztab, float* anch, int den_eps,
                             int Bq, int S, hipStream_t st)
{
    if (!lin_seqfwd_ok(S) || L % 16 != 0 || L <= 0)
        return hipErrorInvalidValue;
    const dim3 grid(seq_grid(Bq)), block(SEQ_THREADS);
    ProfScope ps(st, "lin_seqfwd");
    CXG_LAUNCH((lin_seqfwd_kernel<PHI>), grid, block, 0, st, Q, K, V, O, den, zc, rec, nseg, L / 16,
               Sfin, zfin, sfin_de, ctot, ztab, anch, den_eps, Bq, S);
    return hipGetLastError();
}

template hipError_t lin_seqfwd_launch<PHI_ELU1>(const float*, const float*, const float*, float*,
                                                float*, float*, float*, int, int, float*, float*,
                                                int, float*, float*, float*, int, int, int,
                                                hipStream_t);
template hipError_t lin_seqfwd_launch<PHI_NONE>(const float*, const float*, const float*, float*,
                                                float*, float*, float*, int, int, float*, float*,
                                                int, float*, float*, float*, int, int, int,
                                                hipStream_t);
template hipError_t lin_seqfwd_launch<PHI_ELU1_LG>(const float*, const float*, const float*,
                                                   float*, float*, float*, float*, int, int,
                                                   float*, float*, int, float*, float*, float*,
                                                   int, int, int, hipStream_t);

template hipError_t lin_seqrec_launch<PHI_ELU1>(const float*, const float*, const float*, float*,
                                                int, int, int, int, int, int, int, hipStream_t);
template hipError_t lin_seqrec_launch<PHI_NONE>(const float*, const float*, const float*, float*,
                                                int, int, int, int, int, int, int, hipStream_t);
template hipError_t lin_seqrec_launch<PHI_ELU1_LG>(const float*, const float*, const float*,
                                                   float*, int, int, int, int, int, int, int,
                                                   hipStream_t);
template hipError_t lin_seqrec_launch<PHI_HEXP>(const float*, const float*, const float*, float*,
                                                int, int, int, int, int, int, int, hipStream_t);

} // namespace cxg
