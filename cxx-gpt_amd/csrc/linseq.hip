// linseq.hip -- segment records of short sequences in one pass (gfx950).
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
