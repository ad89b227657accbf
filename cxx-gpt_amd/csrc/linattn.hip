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
// segments of L rows; a segment is walked in 16-row chunks with the 64x64
// state in MFMA accumulator registers (one wave per segment; the dK/dV scan
// splits a segment over two waves, one holding S* for dV and one S*^T for
// dK).  Per chunk, the contribution of earlier chunks is one state product
// and the contribution inside the chunk a masked 16x16 product, all on
// v_mfma_f32_16x16x4_f32.  A segment's starting state comes from a
// per-segment aggregate kernel (lin_agg) and an exclusive scan over segments
// (lin_scan); with one segment per sequence both are skipped.
//
// Memory pipeline: each chunk's rows are fetched with 16-byte row loads one
// chunk ahead (in flight while the current chunk computes).  The operands
// that need a row index as the MFMA contraction index (column layout) are
// re-read from a small LDS buffer the chunk is written to; buffers are private
// to a wave (or shared by the two waves of a dK/dV segment).
//
// Wider D/E take the generic kernels at the end of the file (one workgroup
// per sequence, serial over t, state in global scratch).
//
// Register layouts of a 16-row chunk (lane l, l16 = l%16, g = l/16, f4 element r):
//   R-layout:  v[ct][r] = M[t0 + l16][16ct + 4g + r]   (row per lane)
//   C-layout:  v[ct][r] = M[t0 + 4g + r][16ct + l16]   (column per lane)
#include "common.hpp"

#include <type_traits>
#include "launch.hpp"
#include "linattn.hpp"
#include "linattn_dev.hpp"

namespace cxg {

// ---------------------------------------------------------------------------
// Segment kernels.  A workgroup of NW waves owns one segment; the 64x64
// state is split between the waves by 32-column halves, so a wave keeps only
// a 64x32 slice in registers.  Each chunk's rows are loaded (one chunk ahead)
// by the wave that owns that input, transformed (phi, masks) and written to a
// double-buffered LDS stage; one barrier per chunk publishes the stage to
// the other waves.
// ---------------------------------------------------------------------------

// per-segment aggregates: dS = sum_s phi(X_s)^T Y_s (64 x 64), dz = sum_s w_s phi(X_s)
// (w = 1 when null).  Forward direction: X = K, Y = V.  Reverse: X = Q, Y = dnum,
// w = dden.  Written row-major [d][e] followed by z[d], LIN_WS floats per segment.
// Four waves: wave (h, half) accumulates columns e of tiles et = 2h, 2h+1 over
// one half of the segment's chunks (the two halves run side by side, which
// halves the chain of dependent chunk steps), and the halves are summed
// through LDS at the end.
// ---------------------------------------------------------------------------
constexpr int AGG_THREADS = 256;
constexpr int AGG_STAGE = 2 * CHUNK + 16;

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(AGG_THREADS) __attribute__((amdgpu_waves_per_eu(3))) void lin_agg_kernel(
    const float* __restrict__ X, const float* __restrict__ Y, const float* __restrict__ w,
    float* __restrict__ ws, int Bq, int S, int D, int E, int nseg, int L,
    const LinRopeArg<PHI> rope)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * AGG_STAGE];
    __shared__ float rope_w[phi_rope(PHI) ? 32 : 1];   // RoPE maps: X rows rotated first
    rope_tab_lds<PHI, 32>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar) wave index: the row ranges and descriptor bases
    // below derive from it
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = wv & 1, half = wv >> 1;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int sbeg = seg * L, send = min(S, sbeg + L);
    const int nch_all = (send - sbeg + 15) / 16;
    const int nh = (nch_all + 1) / 2;   // chunks of the first half (the second has nh or nh-1)
    // this half's rows [tbeg, tend); the second half of a one-chunk segment is empty
    const int tbeg = min(sbeg + 16 * nh * half, send);
    const int tend = half ? send : min(send, sbeg + 16 * nh);
    // clamp target for row loads: the half's last row, or the segment's for an empty half
    const int tlast = (tend > tbeg ? tend : send) - 1;
    const long rb = (long)seq * S;

    f4 St[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            St[a][j] = f4zero();
    float zp[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    // Wave (h, half) stages column tiles 2h, 2h+1 of X and Y for its half's
    // chunks (and every lane loads its row's w).  Two register sets, loaded
    // two chunks ahead of use; loads past the last chunk repeat it (clamped;
    // rows outside the half are masked to zero) and the w load goes through a
    // buffer descriptor (none when w is null: 0 is read), so every path issues
    // the same loads and the waits for each set stay exact.  Both halves step
    // through nh chunks (one barrier per step); a half with fewer chunks steps
    // through an empty one.
    const int tlc = tbeg + 16 * max(nh - 1, 0);
    const int tlcl = min(tlc, tlast);   // clamped fetch rows stay in the segment
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w != nullptr ? w + rb : nullptr);
    f4 xa[2], ya[2], xb[2], yb[2];
    float wa, wb;
    // Row loads are coalesced: wave h of the half takes chunk rows
    // 8h + 4i + l/16 (i = 0, 1), columns 4(l%16) .. +3, so each instruction
    // reads four whole rows.
    const int crow = 8 * h + (lane >> 4), ccol = 4 * (lane & 15);
    // D = E = 64: whole rows through descriptors based at the chunk's first
    // row (scalar), with small 32-bit lane offsets instead of 64-bit address
    // arithmetic per load
    auto fetch = [&](f4 (&fx)[2], f4 (&fy)[2], float& fw, int t0) {
        const __amdgpu_buffer_rsrc_t rXc = buf_rsrc(FW ? X + (rb + t0) * 64 : nullptr);
        const __amdgpu_buffer_rsrc_t rYc = buf_rsrc(FW ? Y + (rb + t0) * 64 : nullptr);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if constexpr (FW) {
                const unsigned o = (unsigned)(min(crow + 4 * i, tlast - t0) * 64 + ccol) * 4u;
                fx[i] = buffer_load_f4(rXc, o);
                fy[i] = buffer_load_f4(rYc, o);
            } else {
                const long r = rb + min(t0 + crow + 4 * i, tlast);
                fx[i] = load4c<VEC>(X + r * D, ccol, D);
                fy[i] = load4c<VEC>(Y + r * E, ccol, E);
            }
        }
        fw = buffer_load_f32(rw, (unsigned)min(t0 + l16, tlast) * 4u);
    };
    fetch(xa, ya, wa, min(tbeg, tlcl));
    fetch(xb, yb, wb, min(tbeg + 16, tlcl));
    float* stg = lds + half * 2 * AGG_STAGE;
    // WHOLE: the chunk is known to be whole (every chunk but the half's last),
    // so its row masks are left out
    auto chunk = [&](auto WHOLE, f4 (&ax)[2], f4 (&ay)[2], float& aw, int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = stg + (c & 1) * AGG_STAGE;
        float* bX = st;
        float* bY = st + CHUNK;
        float* bw = st + 2 * CHUNK;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const bool ok = decltype(WHOLE)::value || t0 + crow + 4 * i < tend;
            if constexpr (PHI == PHI_HEXP) {
                // the row's 64 columns lie in this lane's 16-lane group
                const f4 hx = hexp_row4(ax[i], lane);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ax[i][e] = ok ? hx[e] : 0.0f;
                    ay[i][e] = ok ? ay[i][e] : 0.0f;
                }
            } else {
                ax[i] = rot_row<PHI>(ax[i], t0 + crow + 4 * i, ccol, rope_w);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float xv = Phi<PHI>::f(ax[i][e]);
                    ax[i][e] = (ok && (FW || ccol + e < D)) ? xv : 0.0f;
                    ay[i][e] = (ok && (FW || ccol + e < E)) ? ay[i][e] : 0.0f;
                }
            }
            *reinterpret_cast<f4*>(&bX[(crow + 4 * i) * CLD + ccol]) = ax[i];
            *reinterpret_cast<f4*>(&bY[(crow + 4 * i) * CLD + ccol]) = ay[i];
        }
        if (h == 0 && g == 0)
            bw[l16] = w != nullptr ? aw : 1.0f;
        // Below the LDS writes, which read the set: refill it with chunk c+2.
        __builtin_amdgcn_sched_barrier(0);
        fetch(ax, ay, aw, min(t0 + 32, tlcl));
        __syncthreads();
        f4 xC[4], yC[2];
        getC(bX, xC, l16, g);
#pragma unroll
        for (int j = 0; j < 2; j++)
            yC[j] = colC(bY, 2 * h + j, l16, g);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f4 acc = St[dt][j];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(xC[dt][r], yC[j][r], acc);
                St[dt][j] = acc;
            }
        if (h == 0) {
            f4 wc;
#pragma unroll
            for (int r = 0; r < 4; r++)
                wc[r] = bw[4 * g + r];
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    zp[dt] += wc[r] * xC[dt][r];   // rows past the half hold xC = 0
        }
    };
    // Chunks whole in both halves: the second holds nh or nh - 1 chunks, its
    // last one possibly partial (the sequence's end); the remaining steps keep
    // the row masks.
    const int nwhole = (send - min(sbeg + 16 * nh, send)) / 16;
    int c = 0;
    for (; c + 2 <= nwhole; c += 2) {
        chunk(std::true_type{}, xa, ya, wa, c);
        chunk(std::true_type{}, xb, yb, wb, c + 1);
    }
    for (; c < nh; c += 2) {
        chunk(std::false_type{}, xa, ya, wa, c);
        if (c + 1 < nh)
            chunk(std::false_type{}, xb, yb, wb, c + 1);
    }

    // Sum the halves: the second publishes its state slice (and z partials)
    // through LDS, the first adds and writes the record.
    __syncthreads();   // every wave is done with the stages
    float* red = lds + h * (64 * 33);   // [lane][33]: 32 state values + z
    if (half == 1) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    red[lane * 33 + (dt * 2 + j) * 4 + r] = St[dt][j][r];
        }
        if (h == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                red[64 * 66 + lane * 4 + dt] = zp[dt];
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    St[dt][j][r] += red[lane * 33 + (dt * 2 + j) * 4 + r];
        }
        if (h == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                zp[dt] += red[64 * 66 + lane * 4 + dt];
        float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    P[(16 * dt + 4 * g + r) * 64 + 16 * (2 * h + j) + l16] = St[dt][j][r];
            if (h == 0) {
                const float z = xrow_sum(zp[dt]);
                if (g == 0)
                    P[4096 + 16 * dt + l16] = z;
            }
        }
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
    // Batches of SB segments: all loads of a batch are issued before its
    // stores, so the loop costs one memory round trip per batch rather than
    // one per segment.
    constexpr int SB = 8;
    float run = 0.0f;
    for (int k0 = 0; k0 < nseg; k0 += SB) {
        float v[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int k = min(k0 + u, nseg - 1);
            const int s = reverse ? nseg - 1 - k : k;
            v[u] = ws[(seq * nseg + s) * LIN_WS + e];
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            if (k0 + u < nseg) {
                const int k = k0 + u;
                const int s = reverse ? nseg - 1 - k : k;
                ws[(seq * nseg + s) * LIN_WS + e] = run;
                run += v[u];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// forward.  Wave h produces output columns of tiles et = 2h, 2h+1 and keeps
// that half of the state; both waves track z (wave 0 writes den and z_cache).
// ---------------------------------------------------------------------------
constexpr int FWD_THREADS = 128;
constexpr int FWD_STAGE = 3 * CHUNK;   // phi(Q), phi(K), V

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(FWD_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void lin_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ den, float* __restrict__ zcache,
    const float* __restrict__ ws, float* __restrict__ Sfin, float* __restrict__ zfin,
    float* __restrict__ ctot, float* __restrict__ ztab, float* __restrict__ anch, int sfin_de,
    int den_incl_eps, int Bq, int S, int D, int E, int nseg, int L, const LinRopeArg<PHI> rope)
{
    __shared__ __attribute__((aligned(16))) float lds[2 * FWD_STAGE + CHUNK];
    __shared__ float rope_w[phi_rope(PHI) ? 32 : 1];   // RoPE maps: Q, K rows rotated first
    rope_tab_lds<PHI, 32>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();
    const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L), tlast = tend - 1;
    const long rb = (long)seq * S;
    float* bZ = lds + 2 * FWD_STAGE;   // z rows for the z_cache store (each wave its tiles)
    // context for the fused backward (nullable): z before every chunk, [chunk][64]
    const __amdgpu_buffer_rsrc_t rzt =
        buf_rsrc(ztab != nullptr ? ztab + ((long)seq * ((S + 15) / 16) + tbeg / 16) * 64 : nullptr);

    // state slice S[d][e], et = 2h + j: St[dt][j] lane (e = 16et + l16), element r <-> d = 16dt + 4g + r
    // z (prefix of phi(K) before the chunk): zC[dt] = z[16dt + l16], zR[dt][i] = z[16dt + 4g + i]
    f4 St[4][2], zR[4];
    float zC[4];
    if (ws != nullptr) {
        const float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    St[dt][j][r] = P[(16 * dt + 4 * g + r) * 64 + 16 * (2 * h + j) + l16];
            zR[dt] = *reinterpret_cast<const f4*>(P + 4096 + 16 * dt + 4 * g);
            zC[dt] = P[4096 + 16 * dt + l16];
        }
    } else {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
                St[dt][j] = f4zero();
            zR[dt] = f4zero();
            zC[dt] = 0.0f;
        }
    }

    // Wave h stages column tiles 2h, 2h+1 of Q, K and V.  Two register sets,
    // loaded two chunks ahead of use: the set holding chunk c is written to
    // LDS at the start of chunk c and refilled with chunk c+2.  Loads past the
    // last chunk repeat it (clamped), and the stores are branch-free (buffer
    // descriptors, masked lanes dropped), so every path issues the same memory
    // instructions and the waits for each set stay exact.
    const int nch = (tend - tbeg + 15) / 16;
    const int tlc = tbeg + 16 * (nch - 1);   // first row of the last chunk
    f4 qa[2], ka[2], va[2], qb[2], kb[2], vb[2];
    auto fetch = [&](f4 (&fq)[2], f4 (&fk)[2], f4 (&fv)[2], int t0) {
        const int ro = min(l16, tlast - t0);
        // FW: descriptors based at the chunk's first row (scalar), lane
        // offsets of row ro, tile 2h
        const unsigned fvo = (unsigned)(ro * 64 + 32 * h + 4 * g) * 4u;
        const __amdgpu_buffer_rsrc_t rQs = buf_rsrc(FW ? Q + (rb + t0) * 64 : nullptr);
        const __amdgpu_buffer_rsrc_t rKs = buf_rsrc(FW ? K + (rb + t0) * 64 : nullptr);
        const __amdgpu_buffer_rsrc_t rVs = buf_rsrc(FW ? V + (rb + t0) * 64 : nullptr);
        if constexpr (PHI == PHI_HEXP) {
            // Hadamard+Exp transforms whole rows (D = 64): wave h takes chunk
            // rows 8h + 4i + g, columns 4 l16 .. +3, so that a row's 64 columns
            // lie in one 16-lane group
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const long r = rb + t0 + min(8 * h + 4 * i + g, tlast - t0);
                fq[i] = *reinterpret_cast<const f4*>(Q + r * 64 + 4 * l16);
                fk[i] = *reinterpret_cast<const f4*>(K + r * 64 + 4 * l16);
            }
        } else if constexpr (FW) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                fq[i] = buffer_load_f4(rQs, fvo + 64u * i);
                fk[i] = buffer_load_f4(rKs, fvo + 64u * i);
            }
        } else {
            ldRp<VEC, 2>(fq, Q + (rb + t0) * D, D, ro, D, g, 2 * h);
            ldRp<VEC, 2>(fk, K + (rb + t0) * D, D, ro, D, g, 2 * h);
        }
        if constexpr (FW) {
#pragma unroll
            for (int i = 0; i < 2; i++)
                fv[i] = buffer_load_f4(rVs, fvo + 64u * i);
        } else {
            ldRp<VEC, 2>(fv, V + (rb + t0) * E, E, ro, E, g, 2 * h);
        }
    };
    fetch(qa, ka, va, tbeg);
    fetch(qb, kb, vb, min(tbeg + 16, tlc));
    // WHOLE (a std::bool_constant): the chunk is known to be whole, so its
    // row masks are left out (only a sequence's last chunk can be partial)
    auto chunk = [&](auto WHOLE, f4 (&aq)[2], f4 (&ak)[2], f4 (&av)[2], int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = lds + (c & 1) * FWD_STAGE;
        float* bQ = st;
        float* bK = st + CHUNK;
        float* bV = st + 2 * CHUNK;
        const bool full = decltype(WHOLE)::value || t0 + 16 <= tend, rok = t0 + l16 < tend;
        // context: the state before chunk 2^k of the sequence is anchor k (a
        // wave-uniform branch taken log2(S / 16) times per sequence)
        const int cabs = tbeg / 16 + c;
        if (anch != nullptr && cabs > 0 && (cabs & (cabs - 1)) == 0) {
            float* R = anch + ((long)seq * lin_nanch((S + 15) / 16) + __builtin_ctz(cabs)) *
                                  LIN_ANCH;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        R[(16 * dt + 4 * g + r) * 64 + 16 * (2 * h + j) + l16] = St[dt][j][r];
        }
        // context: z before the chunk (lanes l16 = 0 of wave 0 store, others dropped)
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            buffer_store_f4(rzt, (h == 0 && l16 == 0) ? (unsigned)(c * 64 + 16 * dt + 4 * g) * 4u
                                                      : kDropOffset,
                            zR[dt]);
        if constexpr (PHI == PHI_HEXP) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int row = 8 * h + 4 * i + g;
                const bool ok = t0 + row < tend;
                const f4 hq = hexp_row4(aq[i], lane), hk = hexp_row4(ak[i], lane);
                *reinterpret_cast<f4*>(&bQ[row * CLD + 4 * l16]) = ok ? hq : f4zero();
                *reinterpret_cast<f4*>(&bK[row * CLD + 4 * l16]) = ok ? hk : f4zero();
            }
        } else {
            if constexpr (phi_rope(PHI))
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    aq[i] = rot_row<PHI>(aq[i], t0 + l16, 16 * (2 * h + i) + 4 * g, rope_w);
                    ak[i] = rot_row<PHI>(ak[i], t0 + l16, 16 * (2 * h + i) + 4 * g, rope_w);
                }
            finRp<PHI, true, FW, 2>(aq, full, rok, D, g, 2 * h);
            finRp<PHI, true, FW, 2>(ak, full, rok, D, g, 2 * h);
            putRp(bQ, aq, l16, g, 2 * h);
            putRp(bK, ak, l16, g, 2 * h);
        }
        finRp<PHI, false, FW, 2>(av, full, rok, E, g, 2 * h);
        putRp(bV, av, l16, g, 2 * h);
        // Below the LDS writes, which read the set: refill it with chunk c+2.
        __builtin_amdgcn_sched_barrier(0);
        fetch(aq, ak, av, min(t0 + 32, tlc));
        __syncthreads();
        f4 q[4], k[4];
        getR(bQ, q, l16, g);
        getR(bK, k, l16, g);

        // From here to the outputs the chunk is MFMA-dense: raised issue
        // priority lets this wave run ahead of the other workgroup's wave on its
        // SIMD while that one stages or waits (lin_fwd 116.3 -> 115.1 us at C3).
        __builtin_amdgcn_s_setprio(1);
        // A^T[s][t] = phi(K_s).phi(Q_t), lane t = l16, element r <-> s = 4g + r; keep s <= t
        f4 At = f4zero();
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                At = mfma16(k[dt][r], q[dt][r], At);
        // den_t = phi(Q_t).z_prev + sum_{s<=t in chunk} A[t][s]
        float dpart = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            At[r] = (4 * g + r <= l16) ? At[r] : 0.0f;
            dpart += At[r];
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            dpart += q[dt][0] * zR[dt][0] + q[dt][1] * zR[dt][1] + q[dt][2] * zR[dt][2] +
                     q[dt][3] * zR[dt][3];
        const float dn = xrow_sum(dpart);
        // hardware reciprocal (within 1 ulp) in place of a ten-instruction division
        const float inv = __builtin_amdgcn_rcpf(dn + 1e-8f);

        f4 kC[4], vC[2];
        getC(bK, kC, l16, g);
#pragma unroll
        for (int j = 0; j < 2; j++)
            vC[j] = colC(bV, 2 * h + j, l16, g);
        // z_t = z_prev + inclusive prefix of phi(K) over the chunk (column
        // layout); each wave turns its two column tiles into rows through
        // LDS for 16-byte stores
        f4 zp[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            float tot;
            zp[dt] = col_prefix16(kC[dt], tot, lane) + zC[dt];
            zC[dt] += tot;
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const f4 zw = h ? zp[2 + j] : zp[j];
#pragma unroll
            for (int r = 0; r < 4; r++)
                bZ[(4 * g + r) * CLD + 16 * (2 * h + j) + l16] = zw[r];
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                zR[dt][i] = __shfl(zC[dt], 4 * g + i, 64);

        // O^T[e][t] = sum_d S[d][e] phi(Q_t)[d] + sum_s V_s[e] A^T[s][t]
        f4 o[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            f4 acc = f4zero();
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(St[dt][j][r], q[dt][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(vC[j][r], At[r], acc);
            o[j] = acc * inv;
        }
        // S += phi(K)^T V (this wave's columns)
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f4 acc = St[dt][j];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(kC[dt][r], vC[j][r], acc);
                St[dt][j] = acc;
            }
        __builtin_amdgcn_s_setprio(0);
        // outputs of row t0 + l16: O and z_cache columns of this wave's two
        // tiles; den from wave 0
        const bool ok = full || rok;
        f4 zrow[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            zrow[j] = *reinterpret_cast<const f4*>(&bZ[l16 * CLD + 16 * (2 * h + j) + 4 * g]);
        const float dval = den_incl_eps ? dn + 1e-8f : dn;
        if constexpr (FW) {
            const __amdgpu_buffer_rsrc_t ro_ = buf_rsrc(O + (rb + t0) * E);
            const __amdgpu_buffer_rsrc_t rz_ = buf_rsrc(zcache != nullptr ? zcache + (rb + t0) * D
                                                                          : nullptr);
            const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(den + rb + t0);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const unsigned col = 16 * (2 * h + j) + 4 * g;
                buffer_store_f4(ro_, ok ? (unsigned)(l16 * E + col) * 4u : kDropOffset, o[j]);
                buffer_store_f4(rz_, ok ? (unsigned)(l16 * D + col) * 4u : kDropOffset, zrow[j]);
            }
            buffer_store_f32(rd_, (ok && h == 0 && g == 0) ? (unsigned)l16 * 4u : kDropOffset,
                             dval);
        } else if (ok) {
            float* orow = O + (rb + t0 + l16) * E;
#pragma unroll
            for (int j = 0; j < 2; j++)
                stR<VEC, FW>(orow, 16 * (2 * h + j) + 4 * g, E, o[j]);
            if (zcache != nullptr) {
                float* zrw = zcache + (rb + t0 + l16) * D;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    stR<VEC, FW>(zrw, 16 * (2 * h + j) + 4 * g, D, zrow[j]);
            }
            if (h == 0 && g == 0)
                den[rb + t0 + l16] = dval;
        }
    };
    int c = 0;
    for (; c + 2 < nch; c += 2) {
        chunk(std::true_type{}, qa, ka, va, c);
        chunk(std::true_type{}, qb, kb, vb, c + 1);
    }
    if (c < nch)
        chunk(std::false_type{}, qa, ka, va, c);
    if (c + 1 < nch)
        chunk(std::false_type{}, qb, kb, vb, c + 1);

    if (Sfin != nullptr && seg == nseg - 1) {
        // final state of the sequence: [d][e] (linear_cuda) or [e][d] (two_stage)
        float* Sp = Sfin + (long)seq * D * E;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int d = 16 * dt + 4 * g + r, e = 16 * (2 * h + j) + l16;
                    if (d < D && e < E)
                        Sp[sfin_de ? (long)d * E + e : (long)e * D + d] = St[dt][j][r];
                }
        if (zfin != nullptr && h == 0 && g == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                if (16 * dt + l16 < D)
                    zfin[(long)seq * D + 16 * dt + l16] = zC[dt];
    }
    if (ctot != nullptr && seg == nseg - 1) {
        // context: the sequence's final state as a segment record, [d][e] then z
        float* R = ctot + (long)seq * LIN_WS;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    R[(16 * dt + 4 * g + r) * 64 + 16 * (2 * h + j) + l16] = St[dt][j][r];
        if (h == 0 && g == 0)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                R[4096 + 16 * dt + l16] = zC[dt];
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
// dQ (forward-direction scan).  Wave h produces dQ columns of tiles dt = 2h,
// 2h+1 and keeps that half of the transposed state.
// ---------------------------------------------------------------------------
constexpr int DQ_THREADS = 128;
constexpr int DQ_STAGE = 3 * CHUNK + 16;   // phi(K), V, dnum chunks + dden rows

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(DQ_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void lin_dq_kernel(
    const float* __restrict__ K, const float* __restrict__ V, const float* __restrict__ dnum,
    const float* __restrict__ dden, const float* __restrict__ zcache, const float* __restrict__ Q,
    float* __restrict__ dQ, const float* __restrict__ ws, int Bq, int S, int D, int E, int nseg,
    int L)
{
    __shared__ __attribute__((aligned(16))) float lds[2 * DQ_STAGE];
    const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L), tlast = tend - 1;
    const long rb = (long)seq * S;
    constexpr bool HAS_Q = PHI != PHI_NONE;

    // transposed state slice, dt = 2h + j: StT[et][j] lane (d = 16dt + l16),
    // element r <-> e = 16et + 4g + r
    f4 StT[4][2];
    if (ws != nullptr) {
        const float* P = ws + (long)wid * LIN_WS;
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                StT[et][j] = *reinterpret_cast<const f4*>(P + (16 * (2 * h + j) + l16) * 64 + 16 * et + 4 * g);
    } else {
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                StT[et][j] = f4zero();
    }

    // Wave h loads column tiles 2h, 2h+1 of K, V, dnum, z_cache and Q (every
    // lane also its row's dden).  K, V and dnum go through LDS; z_cache and Q
    // are only needed in the row layout they are loaded in (row l16, the
    // wave's own column tiles), so they stay in registers.  The next chunk's
    // loads are issued unconditionally (clamped past the last chunk) and the
    // dQ stores are branch-free (buffer descriptor, masked lanes dropped), so
    // the waits for them stay exact.
    const int nch = (tend - tbeg + 15) / 16;
    const int tlc = tbeg + 16 * (nch - 1);   // first row of the last chunk
    f4 nk[2], nv[2], nn[2], nz[2], nq[2];
    float ndd = 0.0f;
    // D = E = 64: whole rows through descriptors based at the chunk's first
    // row (scalar), with small 32-bit lane offsets
    auto fetch = [&](int t0) {
        const int ro = min(l16, tlast - t0);
        if constexpr (FW) {
            const long cb = (rb + t0) * 64;
            const __amdgpu_buffer_rsrc_t rKs = buf_rsrc(K + cb), rVs = buf_rsrc(V + cb),
                                         rNs = buf_rsrc(dnum + cb), rZs = buf_rsrc(zcache + cb),
                                         rQs = buf_rsrc(HAS_Q ? Q + cb : nullptr);
            const unsigned vo = (unsigned)(ro * 64 + 32 * h + 4 * g) * 4u;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                nk[i] = buffer_load_f4(rKs, vo + 64u * i);
                nv[i] = buffer_load_f4(rVs, vo + 64u * i);
                nn[i] = buffer_load_f4(rNs, vo + 64u * i);
                nz[i] = buffer_load_f4(rZs, vo + 64u * i);
                if (HAS_Q)
                    nq[i] = buffer_load_f4(rQs, vo + 64u * i);
            }
        } else {
            ldRp<VEC, 2>(nk, K + (rb + t0) * D, D, ro, D, g, 2 * h);
            ldRp<VEC, 2>(nv, V + (rb + t0) * E, E, ro, E, g, 2 * h);
            ldRp<VEC, 2>(nn, dnum + (rb + t0) * E, E, ro, E, g, 2 * h);
            ldRp<VEC, 2>(nz, zcache + (rb + t0) * D, D, ro, D, g, 2 * h);
            if (HAS_Q)
                ldRp<VEC, 2>(nq, Q + (rb + t0) * D, D, ro, D, g, 2 * h);
        }
        ndd = dden[rb + t0 + ro];
    };
    fetch(tbeg);
    // WHOLE: the chunk is known to be whole (every chunk but a sequence's
    // last), so its row masks are left out
    auto body = [&](auto WHOLE, int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = lds + (c & 1) * DQ_STAGE;
        float* bK = st;
        float* bV = st + CHUNK;
        float* bN = st + 2 * CHUNK;
        float* bd = st + 3 * CHUNK;
        f4 ak[2], av[2], an[2], az[2], aq[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            ak[i] = nk[i];
            av[i] = nv[i];
            an[i] = nn[i];
            az[i] = nz[i];
            aq[i] = HAS_Q ? nq[i] : f4zero();
        }
        const float dd = ndd;
        fetch(min(t0 + 16, tlc));
        const bool full = decltype(WHOLE)::value || t0 + 16 <= tend, rok = t0 + l16 < tend;
        finRp<PHI, true, FW, 2>(ak, full, rok, D, g, 2 * h);
        finRp<PHI, false, FW, 2>(av, full, rok, E, g, 2 * h);
        finRp<PHI, false, FW, 2>(an, full, rok, E, g, 2 * h);
        putRp(bK, ak, l16, g, 2 * h);
        putRp(bV, av, l16, g, 2 * h);
        putRp(bN, an, l16, g, 2 * h);
        if (h == 0 && g == 0)
            bd[l16] = dd;
        __syncthreads();
        f4 v[4], dn[4];
        getR(bV, v, l16, g);
        getR(bN, dn, l16, g);

        // G^T[s][t] = V_s . dnum_t, lane t = l16, element r <-> s = 4g + r; keep s <= t
        f4 G = f4zero();
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                G = mfma16(v[et][r], dn[et][r], G);
#pragma unroll
        for (int r = 0; r < 4; r++)
            G[r] = (4 * g + r <= l16) ? G[r] : 0.0f;

        f4 vC[4], kC[2];
        getC(bV, vC, l16, g);
#pragma unroll
        for (int j = 0; j < 2; j++)
            kC[j] = colC(bK, 2 * h + j, l16, g);
        const float ddt = bd[l16];
        // dQ^T[d][t] = z_t[d] dden_t + sum_e S[d][e] dnum_t[e] + sum_s phi(K_s)[d] G^T[s][t]
        f4 dq[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            f4 acc = az[j] * ddt;
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(StT[et][j][r], dn[et][r], acc);
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc = mfma16(kC[j][r], G[r], acc);
            if (HAS_Q)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[i] *= Phi<PHI>::d(aq[j][i]);
            dq[j] = acc;
        }
        // S^T += V^T phi(K) (this wave's columns)
#pragma unroll
        for (int et = 0; et < 4; et++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f4 acc = StT[et][j];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(vC[et][r], kC[j][r], acc);
                StT[et][j] = acc;
            }
        const bool ok = full || rok;
        if constexpr (FW) {
            const __amdgpu_buffer_rsrc_t rq = buf_rsrc(dQ + (rb + t0) * D);
#pragma unroll
            for (int j = 0; j < 2; j++)
                buffer_store_f4(rq, ok ? (unsigned)(l16 * D + 16 * (2 * h + j) + 4 * g) * 4u
                                       : kDropOffset, dq[j]);
        } else if (ok) {
            float* qrow = dQ + (rb + t0 + l16) * D;
#pragma unroll
            for (int j = 0; j < 2; j++)
                stR<VEC, FW>(qrow, 16 * (2 * h + j) + 4 * g, D, dq[j]);
        }
    };
    for (int c = 0; c + 1 < nch; c++)
        body(std::true_type{}, c);
    if (nch > 0)
        body(std::false_type{}, nch - 1);
}

// ---------------------------------------------------------------------------
// dK, dV (reverse-direction scan).  Four waves per segment: waves 0/1 hold
// halves (by e columns) of S*[d][e] and produce dV, waves 2/3 hold halves (by
// d columns) of S*^T and z* and produce dK.
// ---------------------------------------------------------------------------
constexpr int DKDV_THREADS = 256;
constexpr int DKDV_STAGE = 4 * CHUNK + 16;   // phi(Q), phi(K), V, dnum chunks + dden rows

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(DKDV_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void lin_dkdv_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dnum, const float* __restrict__ dden, float* __restrict__ dK,
    float* __restrict__ dV, const float* __restrict__ ws, int Bq, int S, int D, int E, int nseg,
    int L)
{
    __shared__ __attribute__((aligned(16))) float lds[2 * DKDV_STAGE];   // double buffered
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const bool isV = w < 2;
    const int hh = w & 1;   // which 32-column half
    const int wid = blockIdx.x;   // segment
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L), tlast = tend - 1;
    const long rb = (long)seq * S;

    // dV waves: Sm[dt][j] = S*[d][e], et = 2hh + j: lane (e = 16et + l16), element r <-> d = 16dt + 4g + r
    // dK waves: Sm[et][j] = S*[d][e], dt = 2hh + j: lane (d = 16dt + l16), element r <-> e = 16et + 4g + r
    //           zs[j] element r <-> d = 16dt + 4g + r
    f4 Sm[4][2], zs[2];
    {
        const float* P = ws != nullptr ? ws + (long)wid * LIN_WS : nullptr;
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int half = 2 * hh + j;
                if (P == nullptr) {
                    Sm[a][j] = f4zero();
                } else if (isV) {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        Sm[a][j][r] = P[(16 * a + 4 * g + r) * 64 + 16 * half + l16];
                } else {
                    Sm[a][j] = *reinterpret_cast<const f4*>(P + (16 * half + l16) * 64 + 16 * a + 4 * g);
                }
            }
#pragma unroll
        for (int j = 0; j < 2; j++)
            zs[j] = (P != nullptr && !isV) ? *reinterpret_cast<const f4*>(P + 4096 + 16 * (2 * hh + j) + 4 * g)
                                           : f4zero();
    }

    // Wave w stages column tile w of Q, K, V and dnum (every lane also loads
    // its row's dden).  The next chunk's loads are issued unconditionally
    // (clamped to the first chunk) and the dK/dV stores are branch-free
    // (buffer descriptors, masked lanes dropped), so the waits for the loads
    // stay exact.
    f4 nq[1], nk[1], nv[1], nn[1];
    float ndd = 0.0f;
    // D = E = 64: whole rows through descriptors based at the chunk's first
    // row (scalar), with small 32-bit lane offsets
    auto fetch = [&](int t0) {
        const int ro = min(l16, tlast - t0);
        if constexpr (FW) {
            const long cb = (rb + t0) * 64;
            const unsigned vo = (unsigned)(ro * 64 + 16 * w + 4 * g) * 4u;
            nq[0] = buffer_load_f4(buf_rsrc(Q + cb), vo);
            nk[0] = buffer_load_f4(buf_rsrc(K + cb), vo);
            nv[0] = buffer_load_f4(buf_rsrc(V + cb), vo);
            nn[0] = buffer_load_f4(buf_rsrc(dnum + cb), vo);
        } else {
            ldRp<VEC, 1>(nq, Q + (rb + t0) * D, D, ro, D, g, w);
            ldRp<VEC, 1>(nk, K + (rb + t0) * D, D, ro, D, g, w);
            ldRp<VEC, 1>(nv, V + (rb + t0) * E, E, ro, E, g, w);
            ldRp<VEC, 1>(nn, dnum + (rb + t0) * E, E, ro, E, g, w);
        }
        ndd = dden[rb + t0 + ro];
    };
    const int nchunk = (tend - tbeg + 15) / 16;
    fetch(tbeg + 16 * (nchunk - 1));
    // WHOLE: the chunk is known to be whole (every chunk but a sequence's
    // last, which this walk takes first), so its row masks are left out
    auto body = [&](auto WHOLE, int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = lds + (c & 1) * DKDV_STAGE;
        float* bQ = st;
        float* bK = st + CHUNK;
        float* bV = st + 2 * CHUNK;
        float* bN = st + 3 * CHUNK;
        float* bd = st + 4 * CHUNK;
        f4 aq[1] = {nq[0]}, ak[1] = {nk[0]}, av[1] = {nv[0]}, an[1] = {nn[0]};
        const float dd = ndd;
        fetch(max(t0 - 16, tbeg));
        const bool full = decltype(WHOLE)::value || t0 + 16 <= tend, rok = t0 + l16 < tend;
        finRp<PHI, true, FW, 1>(aq, full, rok, D, g, w);
        finRp<PHI, true, FW, 1>(ak, full, rok, D, g, w);
        finRp<PHI, false, FW, 1>(av, full, rok, E, g, w);
        finRp<PHI, false, FW, 1>(an, full, rok, E, g, w);
        putRp(bQ, aq, l16, g, w);
        putRp(bK, ak, l16, g, w);
        putRp(bV, av, l16, g, w);
        putRp(bN, an, l16, g, w);
        if (w == 3 && g == 0)
            bd[l16] = rok ? dd : 0.0f;
        __syncthreads();

        if (isV) {
            f4 qR[4], kR[4], qC[4], dnC[2];
            getR(bQ, qR, l16, g);
            getR(bK, kR, l16, g);
            // M1^T[s][t] = phi(Q_s).phi(K_t); lane t = l16, element r <-> s = 4g + r; keep s >= t
            f4 M1 = f4zero();
#pragma unroll
            for (int ct = 0; ct < 4; ct++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    M1 = mfma16(qR[ct][r], kR[ct][r], M1);
#pragma unroll
            for (int r = 0; r < 4; r++)
                M1[r] = (4 * g + r >= l16) ? M1[r] : 0.0f;
            getC(bQ, qC, l16, g);
#pragma unroll
            for (int j = 0; j < 2; j++)
                dnC[j] = colC(bN, 2 * hh + j, l16, g);
            // dV^T[e][t] = sum_d S*[d][e] phi(K_t)[d] + sum_s dnum_s[e] M1^T[s][t]
            f4 dv[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f4 acc = f4zero();
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(Sm[dt][j][r], kR[dt][r], acc);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(dnC[j][r], M1[r], acc);
                dv[j] = acc;
            }
            // S* += phi(Q)^T dnum (this wave's columns)
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    f4 acc = Sm[dt][j];
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(qC[dt][r], dnC[j][r], acc);
                    Sm[dt][j] = acc;
                }
            const bool ok = full || rok;
            if constexpr (FW) {
                const __amdgpu_buffer_rsrc_t rv = buf_rsrc(dV + (rb + t0) * E);
#pragma unroll
                for (int j = 0; j < 2; j++)
                    buffer_store_f4(rv, ok ? (unsigned)(l16 * E + 16 * (2 * hh + j) + 4 * g) * 4u
                                           : kDropOffset, dv[j]);
            } else if (ok) {
                float* vrow = dV + (rb + t0 + l16) * E;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    stR<VEC, FW>(vrow, 16 * (2 * hh + j) + 4 * g, E, dv[j]);
            }
        } else {
            f4 vR[4], dnR[4], dnC[4], qC[2];
            getR(bV, vR, l16, g);
            getR(bN, dnR, l16, g);
            f4 ddC;
#pragma unroll
            for (int r = 0; r < 4; r++)
                ddC[r] = bd[4 * g + r];
            // M2^T[s][t] = dnum_s.V_t + dden_s; lane t = l16, element r <-> s = 4g + r; keep s >= t
            f4 M2 = f4zero();
#pragma unroll
            for (int ct = 0; ct < 4; ct++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    M2 = mfma16(dnR[ct][r], vR[ct][r], M2);
#pragma unroll
            for (int r = 0; r < 4; r++)
                M2[r] = (4 * g + r >= l16) ? M2[r] + ddC[r] : 0.0f;
            getC(bN, dnC, l16, g);
#pragma unroll
            for (int j = 0; j < 2; j++)
                qC[j] = colC(bQ, 2 * hh + j, l16, g);
            // dK^T[d][t] = (z*[d] + sum_e S*[d][e] V_t[e] + sum_s phi(Q_s)[d] M2^T[s][t]) phi'(K_t[d])
            f4 dk[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int dt = 2 * hh + j;
                f4 acc = zs[j];
#pragma unroll
                for (int et = 0; et < 4; et++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(Sm[et][j][r], vR[et][r], acc);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(qC[j][r], M2[r], acc);
                const f4 kv = *reinterpret_cast<const f4*>(&bK[l16 * CLD + 16 * dt + 4 * g]);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[i] *= Phi<PHI>::d_from_f(kv[i]);
                dk[j] = acc;
            }
            // S*^T += dnum^T phi(Q); z* += phi(Q)^T dden (column sums, VALU)
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    f4 acc = Sm[et][j];
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(dnC[et][r], qC[j][r], acc);
                    Sm[et][j] = acc;
                }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                float zp = qC[j][0] * ddC[0] + qC[j][1] * ddC[1] + qC[j][2] * ddC[2] +
                           qC[j][3] * ddC[3];
                zp = xrow_sum(zp);   // column total for d = 16dt + l16
#pragma unroll
                for (int i = 0; i < 4; i++)
                    zs[j][i] += __shfl(zp, 4 * g + i, 64);
            }
            const bool ok = full || rok;
            if constexpr (FW) {
                const __amdgpu_buffer_rsrc_t rk = buf_rsrc(dK + (rb + t0) * D);
#pragma unroll
                for (int j = 0; j < 2; j++)
                    buffer_store_f4(rk, ok ? (unsigned)(l16 * D + 16 * (2 * hh + j) + 4 * g) * 4u
                                           : kDropOffset, dk[j]);
            } else if (ok) {
                float* krow = dK + (rb + t0 + l16) * D;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    stR<VEC, FW>(krow, 16 * (2 * hh + j) + 4 * g, D, dk[j]);
            }
        }
    };
    if (nchunk > 0)
        body(std::false_type{}, nchunk - 1);
    for (int c = nchunk - 2; c >= 0; c--)
        body(std::true_type{}, c);
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
// z_cache for wide heads in the one-call backward (which receives no z_cache):
// z_t = sum_{s<=t} phi(K_s), row by row in fp32 as the forward forms it.  One
// thread per column of a sequence.
template <int PHI>
__global__ __launch_bounds__(256) void lin_zc_kernel(const float* __restrict__ K,
                                                    float* __restrict__ zc, int S, int D)
{
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D)
        return;
    const long base = (long)blockIdx.y * S * D + d;
    float z = 0.0f;
    for (int t = 0; t < S; t++) {
        z += Phi<PHI>::f(K[base + (long)t * D]);
        zc[base + (long)t * D] = z;
    }
}

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

// Vector forms (fwht64_f4, linattn_dev.hpp): each thread keeps HX rows'
// 16-byte loads in flight before any arithmetic.
constexpr int HX = 4;

// phi (N x D, D % 64 == 0): f4 unit u of a row is columns 4u .. 4u+3; blocks
// that lie within E transform x, the others are zero.  Units past the end
// repeat the last one (clamped) and are not stored.
__global__ __launch_bounds__(256) void phi_hexp_fwd_vec_kernel(const float* __restrict__ x,
                                                              float* __restrict__ phi, long N,
                                                              int D, int E)
{
    const int lane = threadIdx.x & 63;
    const long upr = D / 4, total = N * upr;
    const long u0 = (long)blockIdx.x * 256 * HX + threadIdx.x;
    f4 v[HX];
#pragma unroll
    for (int k = 0; k < HX; k++) {
        const long u = min(u0 + 256L * k, total - 1);
        const long n = u / upr;
        const int c = 4 * (int)(u - n * upr);
        v[k] = (c / 64) * 64 + 64 <= E ? *reinterpret_cast<const f4*>(x + n * E + c) : f4zero();
    }
#pragma unroll
    for (int k = 0; k < HX; k++) {
        const long u = u0 + 256L * k;
        const long uc = min(u, total - 1);
        const long n = uc / upr;
        const int c = 4 * (int)(uc - n * upr);
        const bool tr = (c / 64) * 64 + 64 <= E;   // uniform over the 16-lane group
        f4 y = fwht64_f4(v[k], lane, 0.125f);
#pragma unroll
        for (int i = 0; i < 4; i++)
            y[i] = tr ? __expf(y[i]) : 0.0f;
        if (u < total)
            *reinterpret_cast<f4*>(phi + n * D + c) = y;
    }
}

// dx (N x E, E % 64 == 0) = H (dphi * phi) / 8, phi recomputed from x.
__global__ __launch_bounds__(256) void phi_hexp_bwd_vec_kernel(const float* __restrict__ dphi,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ dx, long N,
                                                              int D, int E)
{
    // No multiply-add contraction: the product dphi * phi is rounded before the
    // transform's first (in-lane) additions, as in the one-element-per-lane
    // kernel, where a lane exchange separates them.
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const long upr = E / 4, total = N * upr;
    const long u0 = (long)blockIdx.x * 256 * HX + threadIdx.x;
    f4 xv[HX], gv[HX];
#pragma unroll
    for (int k = 0; k < HX; k++) {
        const long u = min(u0 + 256L * k, total - 1);
        const long n = u / upr;
        const int c = 4 * (int)(u - n * upr);
        xv[k] = *reinterpret_cast<const f4*>(x + n * E + c);
        gv[k] = *reinterpret_cast<const f4*>(dphi + n * D + c);
    }
#pragma unroll
    for (int k = 0; k < HX; k++) {
        const long u = u0 + 256L * k;
        const long uc = min(u, total - 1);
        const long n = uc / upr;
        const int c = 4 * (int)(uc - n * upr);
        f4 y = fwht64_f4(xv[k], lane, 0.125f);
#pragma unroll
        for (int i = 0; i < 4; i++)
            y[i] = gv[k][i] * __expf(y[i]);
        const f4 t = fwht64_f4(y, lane, 0.125f);
        if (u < total)
            *reinterpret_cast<f4*>(dx + n * E + c) = t;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline bool al16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (cached per device).
static int lin_cus()
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

// Workgroups of a pass's main kernel resident at once on the current device
// (occupancy of the D = E = 64 variant times the compute units), cached.
static int lin_slots(int pass)
{
    static int per_cu[4];
    if (pass == LIN_PASS_BWD)
        return lin_bwd_slots() * lin_cus();
    if (per_cu[pass] <= 0) {
        int n = 0;
        hipError_t e = hipErrorInvalidValue;
        if (pass == LIN_PASS_FWD)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)lin_fwd_kernel<PHI_ELU1, true, true>, FWD_THREADS, 0);
        else if (pass == LIN_PASS_DQ)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)lin_dq_kernel<PHI_ELU1, true, true>, DQ_THREADS, 0);
        else
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)lin_dkdv_kernel<PHI_ELU1, true, true>, DKDV_THREADS, 0);
        per_cu[pass] = (e == hipSuccess && n > 0) ? n : 4;
    }
    return per_cu[pass] * lin_cus();
}

LinPlan lin_plan(int Bq, int S, int D, int E, int pass)
{
    LinPlan p;
    p.pass = pass;
    p.quad = lin_quad_any(Bq, S, D, E);
    p.fast = !p.quad && (D <= 64 && E <= 64);
    p.nseg = 1;
    p.L = S;
    if (p.fast) {
        const int nchunk = (S + 15) / 16;
        // Segments per sequence (measured on MI355X at B' = 96): long
        // sequences (> 64 chunks) want one round of the main kernel's
        // resident workgroups (rounding up past it leaves a round that runs
        // almost empty; two rounds cost more in agg/scan and segment start-up
        // than they gain), shorter ones about three segment workgroups per
        // compute unit (the fused backward of sequences of at most 16 chunks
        // one and a half: at B' = 96, S = 256 four segments of four chunks
        // took 55.9 us a step against 57.8 with eight of two, 57.3 with two
        // of eight; at S = 1024 eight segments stay best); at least two
        // chunks per segment.
        const int target = nchunk > 64                                 ? lin_slots(pass)
                           : (pass == LIN_PASS_BWD && nchunk <= 16) ? 3 * lin_cus() / 2
                                                                      : 3 * lin_cus();
        int want = target / Bq;
        if (want > nchunk / 2)
            want = nchunk / 2;
        if (want < 1)
            want = 1;
        const int cps = (nchunk + want - 1) / want;   // chunks per segment
        p.L = 16 * cps;
        p.nseg = (S + p.L - 1) / p.L;
    }
    return p;
}

size_t lin_ws_bytes(const LinPlan& p, int Bq, int D, int E)
{
    if (p.quad)   // the forward's key parts or score blocks (p.L = S)
        return p.pass == LIN_PASS_FWD    ? lin_wide_ws_bytes(Bq, p.L, D, E)
               : p.pass == LIN_PASS_DQ   ? lin_wide_bwd_ws_bytes(Bq, p.L, D, E, 2)
               : p.pass == LIN_PASS_DKDV ? lin_wide_bwd_ws_bytes(Bq, p.L, D, E, 1)
                                         : lin_wide_bwd_ws_bytes(Bq, p.L, D, E, 3);
    if (!p.fast)
        return (size_t)Bq * D * E * sizeof(float);
    if (p.nseg <= 1)
        return 0;
    return (size_t)Bq * p.nseg * LIN_WS * sizeof(float);
}

// Fast-path kernel variant: 2 = D == E == 64 with 16-byte aligned rows, 1 = widths
// multiple of 4 and aligned, 0 = anything else.
static int lin_mode(bool vec, int D, int E) { return !vec ? 0 : (D == 64 && E == 64 ? 2 : 1); }

template <int PHI>
static hipError_t agg_and_scan(const LinPlan& p, const float* X, const float* Y, const float* w,
                               float* ws, int Bq, int S, int D, int E, int reverse, int mode,
                               hipStream_t st)
{
    // short sequences: one launch forms the scanned records (its column-layout
    // loads split RoPE's pairs across lanes, so the RoPE map takes the pair)
    if constexpr (!phi_rope(PHI))
        if (lin_seq_cpw((S + 15) / 16, p.L / 16) > 0)
            return lin_seqrec_launch<PHI>(X, Y, w, ws, Bq, S, D, E, p.L, p.nseg, reverse, st);
    const LinRopeArg<PHI> rope = lin_rope_arg<PHI>(D);
    dim3 grid((unsigned)(Bq * p.nseg)), block(AGG_THREADS);
    {
        ProfScope ps(st, "lin_agg");
        if (mode == 2)
            CXG_LAUNCH((lin_agg_kernel<PHI, true, true>), grid, block, 0, st, X, Y, w, ws,
                               Bq, S, D, E, p.nseg, p.L, rope);
        else if constexpr (PHI == PHI_HEXP)
            return hipErrorInvalidValue;   // D = E = 64 only
        else if (mode == 1)
            CXG_LAUNCH((lin_agg_kernel<PHI, true, false>), grid, block, 0, st, X, Y, w, ws,
                               Bq, S, D, E, p.nseg, p.L, rope);
        else
            CXG_LAUNCH((lin_agg_kernel<PHI, false, false>), grid, block, 0, st, X, Y, w,
                               ws, Bq, S, D, E, p.nseg, p.L, rope);
    }
    {
        ProfScope ps(st, "lin_scan");
        const long n = (long)Bq * LIN_WS;
        CXG_LAUNCH(lin_scan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           ws, Bq, p.nseg, reverse);
    }
    return hipGetLastError();
}

template <int PHI>
static hipError_t fwd_impl(const float* Q, const float* K, const float* V, float* O, float* den,
                           float* zc, float* Sfin, float* zfin, float* ctot, float* ztab,
                           float* anch, int sfin_de, int den_eps, int Bq, int S, int D, int E,
                           void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E, LIN_PASS_FWD);
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(Q) && al16(K) && al16(V) && al16(O) &&
                     al16(zc);
    const int mode = lin_mode(vec, D, E);
    if constexpr (PHI == PHI_HEXP) {
        // the fused Hadamard+Exp kernels: D = E = 64, 16-byte rows, the
        // chunked scan (the callers route other shapes through the
        // feature-map kernels)
        if (p.quad || !p.fast || mode != 2)
            return hipErrorInvalidValue;
    } else if (p.quad) {
        if (phi_rope(PHI))   // the callers form the features (lin_rope_feat_launch)
            return hipErrorInvalidValue;
        hipError_t e = lin_wide_fwd_launch(PHI, Q, K, V, O, den, zc, den_eps, Bq, S, D, E, ws,
                                           st);
        if (e == hipSuccess && Sfin != nullptr)
            e = lin_wide_state_launch(PHI, K, V, Sfin, zfin, sfin_de, Bq, S, D, E, st);
        return e;
    } else if (!p.fast) {
        if constexpr (phi_rope(PHI))
            return hipErrorInvalidValue;   // widths above 512: the callers rotate outside
        else {
        float* state = (float*)ws;
        const size_t sm = (size_t)(3 * D + 256) * sizeof(float);
        {
            ProfScope ps(st, "lin_fwd_generic");
            CXG_LAUNCH((lin_fwd_generic_kernel<PHI>), dim3(Bq), dim3(256), sm, st, Q, K,
                               V, O, den, zc, state, zfin, den_eps, S, D, E);
        }
        if (Sfin != nullptr) {
            const long n = (long)Bq * D * E;
            CXG_LAUNCH(lin_state_copy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                               0, st, state, Sfin, (long)Bq, D, E, sfin_de);
        }
        return hipGetLastError();
        }
    }
    float* wsf = (float*)ws;
    if constexpr (PHI == PHI_ELU1 || PHI == PHI_ELU1_LG || PHI == PHI_NONE) {
        // short sequences at D = E = 64: records and outputs in one launch
        // (the segment records still go to ws, where a context takes them)
        if (mode == 2 && lin_seqfwd_ok(S))
            return lin_seqfwd_launch<PHI>(Q, K, V, O, den, zc, p.nseg > 1 ? wsf : nullptr, p.nseg,
                                          p.L, Sfin, zfin, sfin_de, ctot, ztab, anch, den_eps, Bq,
                                          S, st);
    }
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, K, V, nullptr, wsf, Bq, S, D, E, 0, mode, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    dim3 grid((unsigned)(Bq * p.nseg)), block(FWD_THREADS);
    const LinRopeArg<PHI> rope = lin_rope_arg<PHI>(D);
    ProfScope ps(st, "lin_fwd");
    if (mode == 2)
        CXG_LAUNCH((lin_fwd_kernel<PHI, true, true>), grid, block, 0, st, Q, K, V, O, den, zc,
                           wsf, Sfin, zfin, ctot, ztab, anch, sfin_de, den_eps, Bq, S, D, E, p.nseg,
                           p.L, rope);
    else if constexpr (PHI == PHI_HEXP)
        return hipErrorInvalidValue;
    else if (mode == 1)
        CXG_LAUNCH((lin_fwd_kernel<PHI, true, false>), grid, block, 0, st, Q, K, V, O, den, zc,
                           wsf, Sfin, zfin, ctot, ztab, anch, sfin_de, den_eps, Bq, S, D, E, p.nseg,
                           p.L, rope);
    else
        CXG_LAUNCH((lin_fwd_kernel<PHI, false, false>), grid, block, 0, st, Q, K, V, O, den, zc,
                           wsf, Sfin, zfin, ctot, ztab, anch, sfin_de, den_eps, Bq, S, D, E, p.nseg,
                           p.L, rope);
    return hipGetLastError();
}

hipError_t lin_fwd_launch(int phi, const float* Q, const float* K, const float* V, float* O,
                          float* den, float* zc, float* Sfin, float* zfin, int sfin_de,
                          int den_eps, int Bq, int S, int D, int E, void* ws, hipStream_t st,
                          float* ctot, float* ztab, float* anch)
{
    if (phi == PHI_ELU1)
        return fwd_impl<PHI_ELU1>(Q, K, V, O, den, zc, Sfin, zfin, ctot, ztab, anch, sfin_de,
                                  den_eps, Bq, S, D, E, ws, st);
    if (phi == PHI_ELU1_LG)
        return fwd_impl<PHI_ELU1_LG>(Q, K, V, O, den, zc, Sfin, zfin, ctot, ztab, anch, sfin_de,
                                     den_eps, Bq, S, D, E, ws, st);
    if (phi == PHI_HEXP)
        return fwd_impl<PHI_HEXP>(Q, K, V, O, den, zc, Sfin, zfin, ctot, ztab, anch, sfin_de,
                                  den_eps, Bq, S, D, E, ws, st);
    if (phi == PHI_ELU1_ROPE)
        return fwd_impl<PHI_ELU1_ROPE>(Q, K, V, O, den, zc, Sfin, zfin, ctot, ztab, anch,
                                       sfin_de, den_eps, Bq, S, D, E, ws, st);
    return fwd_impl<PHI_NONE>(Q, K, V, O, den, zc, Sfin, zfin, ctot, ztab, anch, sfin_de,
                              den_eps, Bq, S, D, E, ws, st);
}

hipError_t lin_step1_launch(const float* O, const float* dO, const float* den, float* dnum,
                            float* dden, long N, int E, hipStream_t st)
{
    const bool vec = (E % 4 == 0) && al16(O) && al16(dO) && al16(dnum);
    dim3 grid((unsigned)((N * 16 + 255) / 256)), block(256);
    ProfScope ps(st, "lin_step1");
    if (vec)
        CXG_LAUNCH((lin_step1_kernel<true>), grid, block, 0, st, O, dO, den, dnum, dden,
                           N, E);
    else
        CXG_LAUNCH((lin_step1_kernel<false>), grid, block, 0, st, O, dO, den, dnum, dden,
                           N, E);
    return hipGetLastError();
}

template <int PHI>
static hipError_t dq_impl(const float* K, const float* V, const float* dnum, const float* dden,
                          const float* zc, const float* Q, float* dQ, int Bq, int S, int D, int E,
                          void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E, LIN_PASS_DQ);
    if (p.quad)   // the quadratic form needs no z_cache
        return lin_wide_bwd_launch(PHI, Q, K, V, dnum, dden, dQ, nullptr, nullptr, Bq, S, D, E, 2,
                                   st, nullptr, nullptr, ws);
    if (!p.fast) {
        ProfScope ps(st, "lin_dq_generic");
        CXG_LAUNCH((lin_dq_generic_kernel<PHI>), dim3(Bq), dim3(256), 0, st, K, V, dnum,
                           dden, zc, Q, dQ, (float*)ws, S, D, E);
        return hipGetLastError();
    }
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(K) && al16(V) && al16(dnum) &&
                     al16(zc) && al16(Q) && al16(dQ);
    const int mode = lin_mode(vec, D, E);
    float* wsf = (float*)ws;
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, K, V, nullptr, wsf, Bq, S, D, E, 0, mode, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    dim3 grid((unsigned)(Bq * p.nseg)), block(DQ_THREADS);
    ProfScope ps(st, "lin_dq");
    if (mode == 2)
        CXG_LAUNCH((lin_dq_kernel<PHI, true, true>), grid, block, 0, st, K, V, dnum, dden, zc,
                           Q, dQ, wsf, Bq, S, D, E, p.nseg, p.L);
    else if (mode == 1)
        CXG_LAUNCH((lin_dq_kernel<PHI, true, false>), grid, block, 0, st, K, V, dnum, dden, zc,
                           Q, dQ, wsf, Bq, S, D, E, p.nseg, p.L);
    else
        CXG_LAUNCH((lin_dq_kernel<PHI, false, false>), grid, block, 0, st, K, V, dnum, dden, zc,
                           Q, dQ, wsf, Bq, S, D, E, p.nseg, p.L);
    return hipGetLastError();
}

hipError_t lin_dq_launch(int phi, const float* K, const float* V, const float* dnum,
                         const float* dden, const float* zc, const float* Q, float* dQ, int Bq,
                         int S, int D, int E, void* ws, hipStream_t st)
{
    if (phi == PHI_ELU1)
        return dq_impl<PHI_ELU1>(K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, ws, st);
    if (phi == PHI_ELU1_LG)
        return dq_impl<PHI_ELU1_LG>(K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, ws, st);
    return dq_impl<PHI_NONE>(K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, ws, st);
}

template <int PHI>
static hipError_t dkdv_impl(const float* Q, const float* K, const float* V, const float* dnum,
                            const float* dden, float* dK, float* dV, int Bq, int S, int D, int E,
                            void* ws, hipStream_t st)
{
    const LinPlan p = lin_plan(Bq, S, D, E, LIN_PASS_DKDV);
    if (p.quad)
        return lin_wide_bwd_launch(PHI, Q, K, V, dnum, dden, nullptr, dK, dV, Bq, S, D, E, 1, st,
                                   nullptr, nullptr, ws);
    if (!p.fast) {
        ProfScope ps(st, "lin_dkdv_generic");
        CXG_LAUNCH((lin_dkdv_generic_kernel<PHI>), dim3(Bq), dim3(256),
                           (size_t)D * sizeof(float), st, Q, K, V, dnum, dden, dK, dV, (float*)ws,
                           S, D, E);
        return hipGetLastError();
    }
    const bool vec = (D % 4 == 0) && (E % 4 == 0) && al16(Q) && al16(K) && al16(V) &&
                     al16(dnum) && al16(dK) && al16(dV);
    const int mode = lin_mode(vec, D, E);
    float* wsf = (float*)ws;
    if (p.nseg > 1) {
        hipError_t e = agg_and_scan<PHI>(p, Q, dnum, dden, wsf, Bq, S, D, E, 1, mode, st);
        if (e != hipSuccess)
            return e;
    } else {
        wsf = nullptr;
    }
    dim3 grid((unsigned)(Bq * p.nseg)), block(DKDV_THREADS);
    ProfScope ps(st, "lin_dkdv");
    if (mode == 2)
        CXG_LAUNCH((lin_dkdv_kernel<PHI, true, true>), grid, block, 0, st, Q, K, V, dnum, dden,
                           dK, dV, wsf, Bq, S, D, E, p.nseg, p.L);
    else if (mode == 1)
        CXG_LAUNCH((lin_dkdv_kernel<PHI, true, false>), grid, block, 0, st, Q, K, V, dnum, dden,
                           dK, dV, wsf, Bq, S, D, E, p.nseg, p.L);
    else
        CXG_LAUNCH((lin_dkdv_kernel<PHI, false, false>), grid, block, 0, st, Q, K, V, dnum, dden,
                           dK, dV, wsf, Bq, S, D, E, p.nseg, p.L);
    return hipGetLastError();
}

hipError_t lin_dkdv_launch(int phi, const float* Q, const float* K, const float* V,
                           const float* dnum, const float* dden, float* dK, float* dV, int Bq,
                           int S, int D, int E, void* ws, hipStream_t st)
{
    if (phi == PHI_ELU1)
        return dkdv_impl<PHI_ELU1>(Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, ws, st);
    if (phi == PHI_ELU1_LG)
        return dkdv_impl<PHI_ELU1_LG>(Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, ws, st);
    return dkdv_impl<PHI_NONE>(Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, ws, st);
}

// One-call backward for heads wider than the fused kernels take: z_cache, step
// 1, dQ and dK/dV through the split kernels, with the intermediates in the
// workspace: zc (N x D), dnum (N x E), dden (N), then the scan scratch.
static size_t al256(size_t b) { return (b + 255) / 256 * 256; }

size_t lin_bwd_split_ws_bytes(int Bq, int S, int D, int E)
{
    const size_t N = (size_t)Bq * S;
    if (lin_quad_any(Bq, S, D, E))   // dnum, dden and the quadratic form's scratch
        return al256(N * E * 4) + al256(N * 4) + lin_wide_bwd_ws_bytes(Bq, S, D, E, 3);
    const size_t a = lin_ws_bytes(lin_plan(Bq, S, D, E, LIN_PASS_DQ), Bq, D, E);
    const size_t b = lin_ws_bytes(lin_plan(Bq, S, D, E, LIN_PASS_DKDV), Bq, D, E);
    return al256(N * D * 4) + al256(N * E * 4) + al256(N * 4) + (a > b ? a : b);
}

hipError_t lin_bwd_split_launch(int phi, const float* Q, const float* K, const float* V,
                                const float* O, const float* dO, const float* den, float* dQ,
                                float* dK, float* dV, int Bq, int S, int D, int E, void* ws,
                                hipStream_t st, const void* ctx)
{
    const size_t N = (size_t)Bq * S;
    char* p = (char*)ws;
    if (lin_quad_any(Bq, S, D, E)) {
        // step 1, then every gradient from the quadratic-form backward
        float* dnum = (float*)p;
        float* dden = (float*)(p + al256(N * E * 4));
        char* qws = p + al256(N * E * 4) + al256(N * 4);
        hipError_t e = lin_step1_launch(O, dO, den, dnum, dden, (long)N, E, st);
        if (e != hipSuccess)
            return e;
        if (ctx != nullptr)   // the block-score path with the forward's context
            return lin_qs_bwd_launch(phi, Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, 3, qws,
                                     st, nullptr, nullptr, ctx);
        return lin_wide_bwd_launch(phi, Q, K, V, dnum, dden, dQ, dK, dV, Bq, S, D, E, 3, st,
                                   nullptr, nullptr,
                                   lin_wide_bwd_ws_bytes(Bq, S, D, E, 3) ? qws : nullptr);
    }
    float* zc = (float*)p;
    p += al256(N * D * 4);
    float* dnum = (float*)p;
    p += al256(N * E * 4);
    float* dden = (float*)p;
    p += al256(N * 4);
    {
        ProfScope ps(st, "lin_zc");
        dim3 grid((unsigned)((D + 255) / 256), (unsigned)Bq);
        if (phi == PHI_ELU1)
            CXG_LAUNCH(lin_zc_kernel<PHI_ELU1>, grid, dim3(256), 0, st, K, zc, S, D);
        else if (phi == PHI_ELU1_LG)
            CXG_LAUNCH(lin_zc_kernel<PHI_ELU1_LG>, grid, dim3(256), 0, st, K, zc, S, D);
        else
            CXG_LAUNCH(lin_zc_kernel<PHI_NONE>, grid, dim3(256), 0, st, K, zc, S, D);
    }
    hipError_t e = lin_step1_launch(O, dO, den, dnum, dden, (long)N, E, st);
    if (e == hipSuccess)
        e = lin_dq_launch(phi, K, V, dnum, dden, zc, Q, dQ, Bq, S, D, E, p, st);
    if (e == hipSuccess)
        e = lin_dkdv_launch(phi, Q, K, V, dnum, dden, dK, dV, Bq, S, D, E, p, st);
    return e;
}

hipError_t phi_elu_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st)
{
    const long n = N * D;
    ProfScope ps(st, "phi_elu_fwd");
    CXG_LAUNCH(phi_elu_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x,
                       phi, N, D, E);
    return hipGetLastError();
}

hipError_t phi_elu_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D, int E,
                              hipStream_t st)
{
    const long n = N * E;
    ProfScope ps(st, "phi_elu_bwd");
    CXG_LAUNCH(phi_elu_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       dphi, x, dx, N, D, E);
    return hipGetLastError();
}

hipError_t phi_hexp_fwd_launch(const float* x, float* phi, long N, int D, int E, hipStream_t st)
{
    ProfScope ps(st, "phi_hexp_fwd");
    if (D % 64 == 0 && E % 4 == 0 && al16(x) && al16(phi)) {
        const long units = N * (D / 4);
        CXG_LAUNCH(phi_hexp_fwd_vec_kernel,
                           dim3((unsigned)((units + 256L * HX - 1) / (256L * HX))), dim3(256), 0,
                           st, x, phi, N, D, E);
        return hipGetLastError();
    }
    const long waves = N * ((D + 63) / 64);
    CXG_LAUNCH(phi_hexp_fwd_kernel, dim3((unsigned)((waves * 64 + 255) / 256)), dim3(256),
                       0, st, x, phi, N, D, E);
    return hipGetLastError();
}

hipError_t phi_hexp_bwd_launch(const float* dphi, const float* x, float* dx, long N, int D,
                               int E, hipStream_t st)
{
    ProfScope ps(st, "phi_hexp_bwd");
    if (E % 64 == 0 && D % 4 == 0 && al16(dphi) && al16(x) && al16(dx)) {
        const long units = N * (E / 4);
        CXG_LAUNCH(phi_hexp_bwd_vec_kernel,
                           dim3((unsigned)((units + 256L * HX - 1) / (256L * HX))), dim3(256), 0,
                           st, dphi, x, dx, N, D, E);
        return hipGetLastError();
    }
    const long waves = N * (E / 64);
    CXG_LAUNCH(phi_hexp_bwd_kernel, dim3((unsigned)((waves * 64 + 255) / 256)), dim3(256),
                       0, st, dphi, x, dx, N, D, E);
    return hipGetLastError();
}

} // namespace cxg
