// linbwd.hip -- fused backward of causal linear attention (gfx950, FP32 MFMA):
// step 1, dQ and dK/dV in one pass over each segment.
//
// Replaces the three-call backward of the reference's callers
//   kernel_attn_bwd_step1 -> _bwd_dQ -> _bwd_dKdV      (two_stage_gpt.hpp:149-157,
//     two_stage_cuda_kernels.cu:1190-1809, phi = ELU+1 fused)
//   causal_linear_attention_bwd_step1 -> _dQ -> _dKdV  (linear_gpt.hpp:154-167,
//     linear_cuda_kernels.cu:101-298, phi applied outside)
// for callers that can issue one call.  Q, K, V, O, dO and den are read once and
// dQ, dK, dV written once; dnum = dO / den and dden = -(dO . O) / den (the step-1
// outputs, two_stage_cuda_kernels.cu:1190-1248) never leave the chip, and no
// z_cache is needed.
//
// Per sequence (Q/K rows of width D, V/O rows of width E, D, E <= 64):
//   dQ_t = (z_t dden_t + S_t dnum_t) * phi'(Q_t)
//          S_t = sum_{s<=t} phi(K_s) V_s^T,  z_t = sum_{s<=t} phi(K_s)
//   dV_t = S*_t^T phi(K_t),  dK_t = (z*_t + S*_t V_t) * phi'(K_t)
//          S*_t = sum_{s>=t} phi(Q_s) dnum_s^T,  z*_t = sum_{s>=t} dden_s phi(Q_s)
//
// Structure.  Segments of L rows (16-row chunks), as in the split kernels.
//  * lin_bagg: per segment, the aggregate of phi(K)^T V and phi(K) (every
//    segment) and of phi(Q)^T dnum and dden phi(Q) (segments 1..), plus for
//    every chunk the exclusive within-segment prefix of phi(K) (the z table).
//  * lin_bscan: over the segments of a sequence, the first aggregate becomes an
//    inclusive prefix (its z part an exclusive one), the second an exclusive
//    suffix.
//  * lin_bwd: walks each segment's chunks from last to first.  S* and z* start
//    at the suffix of later segments and take in each chunk after its dK/dV
//    are formed.  S starts at the inclusive prefix at the segment end and gives
//    up each chunk's phi(K)^T V before that chunk's dQ is formed, so every row
//    is read once.  z is not recovered by subtraction (cancellation near a
//    segment start would reach ~1e-4 relative): a chunk's starting z is the
//    segment's exclusive prefix plus its z table entry, both forward sums.
//    The S subtraction is re-anchored: a chunk whose index within the sequence
//    is a power of two takes a forward-summed state (an anchor, written by the
//    forward's context or by lin_bagg) instead, and chunk 0 takes zero.  The
//    rounding error of S then stays relative to a state at most about twice
//    the size of S_t; subtracting from the segment end alone put it relative
//    to the whole segment's sum, and once V has a non-zero mean (|S| growing
//    like t) that exceeded the parity tolerance near the sequence start.
#include "common.hpp"
#include "launch.hpp"
#include "linattn.hpp"
#include "linattn_dev.hpp"

#include <algorithm>
#include <type_traits>

namespace cxg {

// Row-coalesced chunk loads: wave w of a 4-wave workgroup takes chunk rows
// 4w + lane/16, columns 4(lane%16) .. +3, so one instruction reads four whole
// 256-byte rows.  Rows past the segment are clamped (and zeroed after the
// load); columns past the width read a clamped copy and are zeroed too.
template <bool VEC, bool FW>
__device__ __forceinline__ f4 ld_row4(const float* __restrict__ base, long row, int ld, int col,
                                      int ncol)
{
    const f4 v = load4c<VEC>(base + row * ld, col, ncol);
    return FW ? v : mask4(v, col, ncol, true);
}

// The feature map of a row-coalesced f4 (lane: columns 4(lane%16) .. +3 of
// the row its 16-lane group shares): elementwise, or Hadamard+Exp over the row.
template <int PHI>
__device__ __forceinline__ f4 phi_row(f4 v, int lane)
{
    if constexpr (PHI == PHI_HEXP) {
        return hexp_row4(v, lane);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            v[i] = Phi<PHI>::f(v[i]);
        return v;
    }
}

// ---------------------------------------------------------------------------
// lin_bagg: per-segment aggregates.  Workgroups [0, Bq*nseg) form the prefix
// records (X = phi(K), Y = V, w = 1, z table; skipped when the forward's
// context supplies them); workgroups after that the suffix records of
// segments 1.. (X = phi(Q), Y = dnum, w = dden; segment 0's suffix aggregate
// is never used).  Records are row-major [d][e] plus z[d],
// LIN_WS floats.  Wave w accumulates output columns e of tile w over the
// segment's chunks, in forward order.
// ---------------------------------------------------------------------------
constexpr int BAGG_THREADS = 256;
constexpr int BAGG_STAGE = 2 * CHUNK + 16;

// One instance per workgroup kind: SUF is uniform over the workgroup, and each
// instance is straight-line code (no branch around its loads, so the waits on
// the loads in flight stay exact).
template <int PHI, bool VEC, bool FW, bool SUF>
__device__ __attribute__((always_inline)) inline void bagg_body(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ den,
    float* __restrict__ rec, float* __restrict__ ztab_seg, float* __restrict__ anch_seq,
    float* __restrict__ lds, int seq, int seg, int S, int D, int E, int L,
    const float* __restrict__ rope_w)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int tbeg = seg * L, tend = min(S, tbeg + L), tlast = tend - 1;
    const int nch = (tend - tbeg + 15) / 16;
    const int tlc = tbeg + 16 * (nch - 1);
    const long rb = (long)seq * S;
    const int lrow = 4 * w + g, lcol = 4 * l16;
    // z table entries of this segment's chunks (prefix records only)
    const __amdgpu_buffer_rsrc_t rz = buf_rsrc(SUF ? nullptr : ztab_seg);

    f4 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        acc[dt] = f4zero();
    // column totals of w * X, element r <-> d = 16w + 4g + r (the same in every
    // lane l16: an MFMA against a broadcast weight column)
    f4 zrun = f4zero();

    // raw rows: prefix records load K, V; suffix records Q, O, dO and den
    struct Set {
        f4 a, b, c;
        float dn;
    };
    // D = E = 64: whole rows through descriptors over the sequence (32-bit
    // offsets instead of 64-bit address arithmetic)
    const __amdgpu_buffer_rsrc_t rAs = buf_rsrc(FW ? (SUF ? Q : K) + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rBs = buf_rsrc(FW ? (SUF ? O : V) + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rCs = buf_rsrc(FW && SUF ? dO + rb * 64 : nullptr);
    auto fetch = [&](Set& s, int t0) {
        const int t = min(t0 + lrow, tlast);
        const long r = rb + t;
        if constexpr (FW) {
            const unsigned off = (unsigned)(t * 64 + lcol) * 4u;
            s.a = buffer_load_f4(rAs, off);
            s.b = buffer_load_f4(rBs, off);
            if constexpr (SUF) {
                s.c = buffer_load_f4(rCs, off);
                s.dn = den[r];
            }
        } else if constexpr (!SUF) {
            s.a = ld_row4<VEC, FW>(K, r, D, lcol, D);
            s.b = ld_row4<VEC, FW>(V, r, E, lcol, E);
        } else {
            s.a = ld_row4<VEC, FW>(Q, r, D, lcol, D);
            s.b = ld_row4<VEC, FW>(O, r, E, lcol, E);
            s.c = ld_row4<VEC, FW>(dO, r, E, lcol, E);
            s.dn = den[r];
        }
    };
    Set sa, sb;
    fetch(sa, tbeg);
    fetch(sb, min(tbeg + 16, tlc));
    // WHOLE: the chunk is known to be whole (every chunk but the segment's
    // last), so its row masks are left out
    auto chunk = [&](auto WHOLE, Set& s, int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = lds + (c & 1) * BAGG_STAGE;
        float* bX = st;
        float* bY = st + CHUNK;
        float* bw = st + 2 * CHUNK;
        const bool ok = decltype(WHOLE)::value || t0 + lrow < tend;
        f4 x, y;
        float wv;
        const f4 px = phi_row<PHI>(rot_row<PHI>(s.a, t0 + lrow, lcol, rope_w), lane);
        if constexpr (!SUF) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[i] = ok ? px[i] : 0.0f;
                y[i] = ok ? s.b[i] : 0.0f;
            }
            wv = 1.0f;
        } else {
            // the same reciprocal as the main backward's step 1
            const float inv = ok ? __builtin_amdgcn_rcpf(s.dn) : 0.0f;
            const float dot = row16_sum(s.c[0] * s.b[0] + s.c[1] * s.b[1] + s.c[2] * s.b[2] +
                                        s.c[3] * s.b[3]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                x[i] = ok ? px[i] : 0.0f;
                y[i] = s.c[i] * inv;
            }
            wv = -dot * inv;
        }
        if (!FW)
            x = mask4(x, lcol, D, true);   // phi(0) != 0: re-zero the padded columns
        *reinterpret_cast<f4*>(&bX[lrow * CLD + lcol]) = x;
        *reinterpret_cast<f4*>(&bY[lrow * CLD + lcol]) = y;
        bw[lrow] = wv;   // the row's 16 lanes store the same value
        // Below the LDS writes, which read the set: refill it with chunk c+2.
        __builtin_amdgcn_sched_barrier(0);
        fetch(s, min(t0 + 32, tlc));
        __syncthreads();
        f4 xC[4];
        getC(bX, xC, l16, g);
        const f4 yC = colC(bY, w, l16, g);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            f4 a = acc[dt];
#pragma unroll
            for (int r = 0; r < 4; r++)
                a = mfma16(xC[dt][r], yC[r], a);
            acc[dt] = a;
        }
        // Segment 0's prefix (anch_seq != null): the state before chunk c + 1 is
        // anchor k when c + 1 = 2^k lies inside the segment (a wave-uniform
        // branch taken log2(L / 16) times).
        if (anch_seq != nullptr && c + 1 < nch && ((c + 1) & c) == 0) {
            float* R = anch_seq + __builtin_ctz(c + 1) * LIN_ANCH;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    R[(16 * dt + 4 * g + r) * 64 + 16 * w + l16] = acc[dt][r];
        }
        // z table: the exclusive prefix before this chunk (lanes l16 = 0 store)
        buffer_store_f4(rz, l16 == 0 ? (unsigned)(c * 64 + 16 * w + 4 * g) * 4u : kDropOffset,
                        zrun);
        // zrun[d] += sum_t X[t][d] w_t
        const f4 xw = colC(bX, w, l16, g);
        const f4 wt = SUF ? *reinterpret_cast<const f4*>(&bw[4 * g]) : f4splat(1.0f);
#pragma unroll
        for (int r = 0; r < 4; r++)
            zrun = mfma16(xw[r], wt[r], zrun);
    };
    int c = 0;
    for (; c + 2 < nch; c += 2) {
        chunk(std::true_type{}, sa, c);
        chunk(std::true_type{}, sb, c + 1);
    }
    if (c < nch)
        chunk(std::false_type{}, sa, c);
    if (c + 1 < nch)
        chunk(std::false_type{}, sb, c + 1);

#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            rec[(16 * dt + 4 * g + r) * 64 + 16 * w + l16] = acc[dt][r];
    if (l16 == 0)
        *reinterpret_cast<f4*>(&rec[4096 + 16 * w + 4 * g]) = zrun;
}

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(BAGG_THREADS) void lin_bagg_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ den,
    float* __restrict__ wsP, float* __restrict__ wsB, float* __restrict__ ztab,
    float* __restrict__ anch, int nanch, int Bq, int S, int D, int E, int nseg, int L, int nchs,
    int with_prefix, const LinRopeArg<PHI> rope)
{
    __shared__ __attribute__((aligned(16))) float lds[2 * BAGG_STAGE];
    __shared__ float rope_w[phi_rope(PHI) ? 32 : 1];   // RoPE maps: Q, K rows rotated first
    rope_tab_lds<PHI, 32>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();
    const int nP = with_prefix ? Bq * nseg : 0;
    if ((int)blockIdx.x < nP) {
        const int seq = blockIdx.x / nseg, seg = blockIdx.x - seq * nseg;
        bagg_body<PHI, VEC, FW, false>(Q, K, V, O, dO, den, wsP + (long)blockIdx.x * LIN_WS,
                                       ztab + ((long)seq * nchs + seg * (L / 16)) * 64,
                                       seg == 0 && nanch > 0 ? anch + (long)seq * nanch * LIN_ANCH
                                                             : nullptr,
                                       lds, seq, seg, S, D, E, L, rope_w);
    } else {
        const int b = blockIdx.x - nP;
        const int seq = b / (nseg - 1), seg = 1 + (b - seq * (nseg - 1));
        bagg_body<PHI, VEC, FW, true>(Q, K, V, O, dO, den,
                                      wsB + ((long)seq * nseg + seg) * LIN_WS, nullptr, nullptr,
                                      lds, seq, seg, S, D, E, L, rope_w);
    }
}

// ---------------------------------------------------------------------------
// lin_bscan: per sequence and record element, over the segments.  Prefix
// records: inclusive for the state (the backward walk starts at the segment
// end), exclusive for z.  Suffix records: exclusive from the end (segment 0's
// record is only written).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void lin_bscan_kernel(float* __restrict__ wsP,
                                                       float* __restrict__ wsB, int Bq, int nseg,
                                                       int with_prefix)
{
    const long n = (long)Bq * LIN_WS;
    const long j = (long)blockIdx.x * 256 + threadIdx.x + (with_prefix ? 0 : n);
    if (j >= 2 * n)
        return;
    const bool suf = j >= n;
    const long k = suf ? j - n : j;
    const long seq = k / LIN_WS, e = k - seq * LIN_WS;
    float* base = (suf ? wsB : wsP) + seq * nseg * LIN_WS + e;
    const bool incl = !suf && e < 4096;
    // Batches of SB segments: all loads of a batch are issued before its stores.
    constexpr int SB = 8;
    const int cnt = suf ? nseg - 1 : nseg;   // records read
    float run = 0.0f;
    for (int k0 = 0; k0 < cnt; k0 += SB) {
        float v[SB];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const int q = min(k0 + u, cnt - 1);
            const int s = suf ? nseg - 1 - q : q;
            v[u] = base[(long)s * LIN_WS];
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            if (k0 + u < cnt) {
                const int q = k0 + u;
                const int s = suf ? nseg - 1 - q : q;
                const float nx = run + v[u];
                base[(long)s * LIN_WS] = incl ? nx : run;
                run = nx;
            }
        }
    }
    if (suf)
        base[0] = run;   // segment 0: the suffix of every later segment
}

// ---------------------------------------------------------------------------
// lin_bwd: the fused pass.  Four waves per segment; wave w owns
//   column tile w of S* (e = 16w..): forms dV columns e of tile w,
//   column tile w of S^T (d = 16w..): forms dQ columns d of tile w,
//   and dK columns d of tile w from S* rows d of tile w, which the waves
//   publish through LDS (each wave writes its updated S* slice at the start of
//   the next chunk, after the barrier that ends every read of the old one).
// The chunk's 16x16 products phi(Q)phi(K)^T and dnum V^T are split over the
// waves by 16-wide slices of the contraction and summed through LDS.
// ---------------------------------------------------------------------------
constexpr int BWD_THREADS = 256;
constexpr int BWD_STAGE = 4 * CHUNK + 16;   // phi(Q), phi(K), V, dnum chunks + dden rows
constexpr int SLD = 68;                     // row stride of the S* copy [d][e]
constexpr int BWD_LDS = 2 * BWD_STAGE + 64 * SLD + 4 * 3 * 256;

template <int PHI, bool VEC, bool FW>
__global__ __launch_bounds__(BWD_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void lin_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ den,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV,
    const float* __restrict__ wsP, const float* __restrict__ wsB, const float* __restrict__ ztab,
    const float* __restrict__ crec, const float* __restrict__ ctot, const float* __restrict__ anch,
    int nanch, int mf, int nsegf, int S, int D, int E, int nseg, int L, int nchs,
    const LinRopeArg<PHI> rope)
{
    // Hadamard+Exp: the chunk's dphi(Q) * phi(Q) and dphi(K) * phi(K), [t][d],
    // for the row transform that turns them into dQ and dK (see flush below)
    constexpr int HEXP_LDS = PHI == PHI_HEXP ? 2 * CHUNK : 0;
    __shared__ __attribute__((aligned(16))) float lds[BWD_LDS + HEXP_LDS];
    // RoPE maps: Q, K rows rotated as they are staged; dQ, dK (gradients with
    // respect to the rotated rows) rotated back before their stores
    __shared__ float rope_w[phi_rope(PHI) ? 32 : 1];
    rope_tab_lds<PHI, 32>(rope_w, rope);
    if constexpr (phi_rope(PHI))
        __syncthreads();
    float* sS = lds + 2 * BWD_STAGE;   // S* [d][e]
    float* sP = sS + 64 * SLD;         // partial products [wave][M1, X, X^T][lane * 4 + r]
    float* sH = lds + BWD_LDS;         // Hadamard+Exp only
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wid = blockIdx.x;
    const int seq = wid / nseg, seg = wid - seq * nseg;
    const int tbeg = seg * L, tend = min(S, tbeg + L), tlast = tend - 1;
    const long rb = (long)seq * S;
    const int lrow = 4 * w + g, lcol = 4 * l16;

    // StT[et]: lane (d = 16w + l16), element r <-> e = 16et + 4g + r of S^T (inclusive
    //          prefix at the segment end, then S before the current chunk)
    // Sm[dt]:  lane (e = 16w + l16), element r <-> d = 16dt + 4g + r of S* (suffix
    //          of the chunks after the current one)
    // zs, pz:  element r <-> d = 16w + 4g + r of z* and of z before the segment
    // With the forward's context (ctot != null) the segment-end state is the
    // record at the forward's segment boundary mf * (seg + 1) (or the final
    // state) and ztab holds absolute z, so the segment prefix of z is not added.
    f4 StT[4], Sm[4];
    const float* RP;
    if (ctot != nullptr) {
        const int e = min(mf * (seg + 1), nsegf);
        RP = e < nsegf ? crec + ((long)seq * nsegf + e) * LIN_WS : ctot + (long)seq * LIN_WS;
    } else {
        RP = wsP + (long)wid * LIN_WS;
    }
    const float* RB = wsB + (long)wid * LIN_WS;
#pragma unroll
    for (int a = 0; a < 4; a++) {
        StT[a] = *reinterpret_cast<const f4*>(RP + (16 * w + l16) * 64 + 16 * a + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; r++)
            Sm[a][r] = RB[(16 * a + 4 * g + r) * 64 + 16 * w + l16];
    }
    f4 zs = *reinterpret_cast<const f4*>(RB + 4096 + 16 * w + 4 * g);
    const f4 pz = ctot != nullptr ? f4zero()
                                  : *reinterpret_cast<const f4*>(RP + 4096 + 16 * w + 4 * g);

    const int nch = (tend - tbeg + 15) / 16;
    const float* zt0 = ztab + ((long)seq * nchs + tbeg / 16) * 64 + 16 * w + 4 * g;
    struct Set {
        f4 q, k, v, o, d, zt;
        float dn;
    };
    // D = E = 64: loads through buffer descriptors over this sequence's rows
    // (one uniform base per tensor, 32-bit row offsets)
    const __amdgpu_buffer_rsrc_t rQ = buf_rsrc(FW ? Q + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rK = buf_rsrc(FW ? K + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rV = buf_rsrc(FW ? V + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rO = buf_rsrc(FW ? O + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rdO = buf_rsrc(FW ? dO + rb * 64 : nullptr);
    const __amdgpu_buffer_rsrc_t rden = buf_rsrc(den + rb);
    auto fetch = [&](Set& s, int c) {
        const int t = min(tbeg + 16 * c + lrow, tlast);
        if constexpr (FW) {
            const unsigned off = (unsigned)(t * 64 + lcol) * 4u;
            s.q = buffer_load_f4(rQ, off);
            s.k = buffer_load_f4(rK, off);
            s.v = buffer_load_f4(rV, off);
            s.o = buffer_load_f4(rO, off);
            s.d = buffer_load_f4(rdO, off);
        } else {
            const long r = rb + t;
            s.q = ld_row4<VEC, FW>(Q, r, D, lcol, D);
            s.k = ld_row4<VEC, FW>(K, r, D, lcol, D);
            s.v = ld_row4<VEC, FW>(V, r, E, lcol, E);
            s.o = ld_row4<VEC, FW>(O, r, E, lcol, E);
            s.d = ld_row4<VEC, FW>(dO, r, E, lcol, E);
        }
        s.dn = buffer_load_f32(rden, (unsigned)t * 4u);
        s.zt = *reinterpret_cast<const f4*>(zt0 + (long)c * 64);
    };
    Set sa, sb;
    fetch(sa, nch - 1);
    fetch(sb, max(nch - 2, 0));
    // State anchors (forward-summed S before chunk 2^k of the sequence, [d][e],
    // k < nanch): the one for chunk c is loaded while chunk c + 1 is worked, into
    // `an` in StT's layout.  Every chunk issues the loads; for a chunk that is no
    // anchor the descriptor has no records and they return zeros without a
    // memory access, so the waits on the other loads stay exact.
    const int cb = tbeg / 16;
    auto is_anchor = [&](int ca) { return ca > 0 && (ca & (ca - 1)) == 0 && __builtin_ctz(ca) < nanch; };
    f4 an[4];
    auto fetch_anchor = [&](int ca) {
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc(
            is_anchor(ca) ? anch + ((long)seq * nanch + __builtin_ctz(ca)) * LIN_ANCH : nullptr);
#pragma unroll
        for (int a = 0; a < 4; a++)
            an[a] = buffer_load_f4(ra, (unsigned)((16 * w + l16) * 64 + 16 * a + 4 * g) * 4u);
    };
    fetch_anchor(cb + nch - 1);
    // Hadamard+Exp (D = E = 64): dQ_t = H (dphi(Q_t) * phi(Q_t)) / 8 transforms
    // whole rows, which the waves hold a 16-column tile of each.  A chunk's
    // products go to sH at its end and are transformed and stored, as whole
    // rows (lane: row 4w + g, columns 4 l16 .. +3), by the next chunk between
    // its two barriers (the first orders them after every wave's write, the
    // second before the next write); the last chunk's after the walk.  ht0:
    // first row of the chunk pending in sH, -1 for none.
    int ht0 = -1;
    auto flush = [&]() __attribute__((always_inline)) {
        const f4 hq = *reinterpret_cast<const f4*>(&sH[lrow * CLD + lcol]);
        const f4 hk = *reinterpret_cast<const f4*>(&sH[CHUNK + lrow * CLD + lcol]);
        const f4 tq = fwht64_f4(hq, lane, 0.125f);
        const f4 tk = fwht64_f4(hk, lane, 0.125f);
        const unsigned off = (ht0 >= 0 && ht0 + lrow < tend)
                                 ? (unsigned)((ht0 + lrow) * 64 + lcol) * 4u
                                 : kDropOffset;
        buffer_store_f4(buf_rsrc(dQ + rb * 64), off, tq);
        buffer_store_f4(buf_rsrc(dK + rb * 64), off, tk);
    };
    // WHOLE: the chunk is known to be whole (every chunk but the segment's
    // last, which this walk takes first), so its row masks are left out
    auto chunk = [&](auto WHOLE, Set& s, int c) __attribute__((always_inline)) {
        const int t0 = tbeg + 16 * c;
        float* st = lds + (c & 1) * BWD_STAGE;
        float* bQ = st;
        float* bK = st + CHUNK;
        float* bV = st + 2 * CHUNK;
        float* bN = st + 3 * CHUNK;
        float* bd = st + 4 * CHUNK;
        {
            // step 1 for this wave's four rows, phi, row masks; stage the chunk.
            // 1/den through the hardware reciprocal (within 1 ulp; the exact
            // division costs ten VALU instructions, which on gfx950 add to the
            // chunk's MFMA time).  Rows past the end exist only in a
            // sequence's last, partial chunk (a wave-uniform branch).
            const bool ok = decltype(WHOLE)::value || t0 + lrow < tend;
            const float inv = ok ? __builtin_amdgcn_rcpf(s.dn) : 0.0f;
            const float dot = row16_sum(s.d[0] * s.o[0] + s.d[1] * s.o[1] + s.d[2] * s.o[2] +
                                        s.d[3] * s.o[3]);
            f4 q = phi_row<PHI>(rot_row<PHI>(s.q, t0 + lrow, lcol, rope_w), lane);
            f4 k = phi_row<PHI>(rot_row<PHI>(s.k, t0 + lrow, lcol, rope_w), lane);
            f4 v = s.v;
            if (!decltype(WHOLE)::value && t0 + 16 > tend) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    q[i] = ok ? q[i] : 0.0f;
                    k[i] = ok ? k[i] : 0.0f;
                    v[i] = ok ? v[i] : 0.0f;
                }
            }
            if (!FW) {
                q = mask4(q, lcol, D, true);
                k = mask4(k, lcol, D, true);
            }
            *reinterpret_cast<f4*>(&bQ[lrow * CLD + lcol]) = q;
            *reinterpret_cast<f4*>(&bK[lrow * CLD + lcol]) = k;
            *reinterpret_cast<f4*>(&bV[lrow * CLD + lcol]) = v;
            *reinterpret_cast<f4*>(&bN[lrow * CLD + lcol]) = s.d * inv;
            bd[lrow] = -dot * inv;   // the row's 16 lanes store the same value
        }
        const f4 zb = pz + s.zt;   // z before the chunk, columns d of tile w
        // Below the LDS writes, which read the set: refill it with chunk c-2.
        __builtin_amdgcn_sched_barrier(0);
        fetch(s, max(c - 2, 0));
        __syncthreads();
        if constexpr (PHI == PHI_HEXP)
            flush();   // the previous chunk's dQ, dK rows

        // partial products over the contraction slice of tile w:
        //   M1[s][t] = phi(Q_s).phi(K_t),  X[s][t] = dnum_s.V_t
        {
            const f4 qRw = *reinterpret_cast<const f4*>(&bQ[l16 * CLD + 16 * w + 4 * g]);
            const f4 kRw = *reinterpret_cast<const f4*>(&bK[l16 * CLD + 16 * w + 4 * g]);
            const f4 nRw = *reinterpret_cast<const f4*>(&bN[l16 * CLD + 16 * w + 4 * g]);
            const f4 vRw = *reinterpret_cast<const f4*>(&bV[l16 * CLD + 16 * w + 4 * g]);
            f4 m1 = f4zero(), x = f4zero();
#pragma unroll
            for (int r = 0; r < 4; r++) {
                m1 = mfma16(qRw[r], kRw[r], m1);
                x = mfma16(nRw[r], vRw[r], x);
            }
            *reinterpret_cast<f4*>(&sP[(3 * w) * 256 + lane * 4]) = m1;
            *reinterpret_cast<f4*>(&sP[(3 * w + 1) * 256 + lane * 4]) = x;
            // X^T in the accumulator layout: X[s][t] (lane t, element s - 4g) goes
            // to lane (t / 4) * 16 + s, element t % 4
#pragma unroll
            for (int r = 0; r < 4; r++)
                sP[(3 * w + 2) * 256 + ((l16 >> 2) * 16 + 4 * g + r) * 4 + (l16 & 3)] = x[r];
        }
        // This wave's S* slice (it took in chunk c+1 last step) for the dK of
        // chunk c: written after the barrier above, which every wave passes only
        // once its reads of the previous copy (dK of chunk c+1) are done.
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                sS[(16 * dt + 4 * g + r) * SLD + 16 * w + l16] = Sm[dt][r];
        __syncthreads();
        // The products below are the MFMA-heavy part of the chunk: the wave
        // issues ahead of the other workgroup's wave on its SIMD while that one
        // stages or waits (measured: 4% faster at C3).
        __builtin_amdgcn_s_setprio(1);
        // lane t = l16, element r <-> s = 4g + r:
        //   M1 (keep s >= t), M2 = X + dden_s (s >= t), G = X^T + dden_t (s <= t)
        f4 M1 = f4zero(), X = f4zero(), Xt = f4zero();
#pragma unroll
        for (int u = 0; u < 4; u++) {
            M1 += *reinterpret_cast<const f4*>(&sP[(3 * u) * 256 + lane * 4]);
            X += *reinterpret_cast<const f4*>(&sP[(3 * u + 1) * 256 + lane * 4]);
            Xt += *reinterpret_cast<const f4*>(&sP[(3 * u + 2) * 256 + lane * 4]);
        }
        const f4 ddS = *reinterpret_cast<const f4*>(&bd[4 * g]);
        const float ddT = bd[l16];
        f4 M2, G;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int sr = 4 * g + r;
            M1[r] = sr >= l16 ? M1[r] : 0.0f;
            M2[r] = sr >= l16 ? X[r] + ddS[r] : 0.0f;
            G[r] = sr <= l16 ? Xt[r] + ddT : 0.0f;
        }
        const bool okt = decltype(WHOLE)::value || t0 + l16 < tend;
        const unsigned soff = (unsigned)(l16 * 64 + 16 * w + 4 * g);   // FW store offsets

        // dV^T[e][t] = sum_d S*[d][e] phi(K_t)[d] + sum_{s>=t} dnum_s[e] M1[s][t]
        f4 kR[4];
        getR(bK, kR, l16, g);
        const f4 nCw = colC(bN, w, l16, g);
        {
            f4 dv = f4zero();
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    dv = mfma16(Sm[dt][r], kR[dt][r], dv);
#pragma unroll
            for (int r = 0; r < 4; r++)
                dv = mfma16(nCw[r], M1[r], dv);
            if constexpr (FW) {
                buffer_store_f4(buf_rsrc(dV + (rb + t0) * E), okt ? soff * 4u : kDropOffset, dv);
            } else if (okt) {
                store4<VEC>(dV + (rb + t0 + l16) * E, 16 * w + 4 * g, E, dv);
            }
        }
        // dK^T[d][t] = (z*[d] + sum_e S*[d][e] V_t[e] + sum_{s>=t} phi(Q_s)[d] M2[s][t]) phi'(K_t[d])
        const f4 qCw = colC(bQ, w, l16, g);
        {
            f4 vR[4];
            getR(bV, vR, l16, g);
            f4 dk = zs;
#pragma unroll
            for (int et = 0; et < 4; et++) {
                const f4 sT = *reinterpret_cast<const f4*>(&sS[(16 * w + l16) * SLD + 16 * et + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    dk = mfma16(sT[r], vR[et][r], dk);
            }
#pragma unroll
            for (int r = 0; r < 4; r++)
                dk = mfma16(qCw[r], M2[r], dk);
            const f4 kRw = *reinterpret_cast<const f4*>(&bK[l16 * CLD + 16 * w + 4 * g]);
            if constexpr (PHI == PHI_HEXP) {
                *reinterpret_cast<f4*>(&sH[CHUNK + l16 * CLD + 16 * w + 4 * g]) = dk * kRw;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    dk[i] *= Phi<PHI>::d_from_f(kRw[i]);
                dk = rot_row<PHI>(dk, t0 + l16, 16 * w + 4 * g, rope_w, -1.0f);
            }
            if constexpr (PHI == PHI_HEXP) {
            } else if constexpr (FW) {
                buffer_store_f4(buf_rsrc(dK + (rb + t0) * D), okt ? soff * 4u : kDropOffset, dk);
            } else if (okt) {
                store4<VEC>(dK + (rb + t0 + l16) * D, 16 * w + 4 * g, D, dk);
            }
        }
        // S^T gives up the chunk: S^T[e][d] -= sum_t V_t[e] phi(K_t)[d]
        const f4 kCw = colC(bK, w, l16, g);
        {
            f4 vC[4];
            getC(bV, vC, l16, g);
            const f4 nk = -kCw;
#pragma unroll
            for (int et = 0; et < 4; et++) {
                f4 a = StT[et];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    a = mfma16(vC[et][r], nk[r], a);
                StT[et] = a;
            }
            // re-anchor: chunk 0 of the sequence starts from zero, an anchor chunk
            // from its forward-summed state; then request the next chunk's anchor
            // (wave-uniform branches: taken at log2(S / 16) + 1 chunks)
            const int ca = cb + c;
            if (ca == 0) {
#pragma unroll
                for (int et = 0; et < 4; et++)
                    StT[et] = f4zero();
            } else if (is_anchor(ca)) {
#pragma unroll
                for (int et = 0; et < 4; et++)
                    StT[et] = an[et];
            }
            fetch_anchor(ca - 1);
        }
        // dQ^T[d][t] = (z_t[d] dden_t + sum_e S[d][e] dnum_t[e]) phi'(Q_t[d]), with
        // z_t = zb + sum_{s<=t} phi(K_s) and S_t = S + sum_{s<=t} phi(K_s) V_s^T:
        //   = (zb[d] dden_t + sum_e S[d][e] dnum_t[e] + sum_{s<=t} phi(K_s)[d] G[s][t]) phi'
        {
            f4 nR[4];
            getR(bN, nR, l16, g);
            f4 dq = zb * ddT;
#pragma unroll
            for (int et = 0; et < 4; et++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    dq = mfma16(StT[et][r], nR[et][r], dq);
#pragma unroll
            for (int r = 0; r < 4; r++)
                dq = mfma16(kCw[r], G[r], dq);
            const f4 qRw = *reinterpret_cast<const f4*>(&bQ[l16 * CLD + 16 * w + 4 * g]);
            if constexpr (PHI == PHI_HEXP) {
                *reinterpret_cast<f4*>(&sH[l16 * CLD + 16 * w + 4 * g]) = dq * qRw;
                ht0 = t0;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    dq[i] *= Phi<PHI>::d_from_f(qRw[i]);
                dq = rot_row<PHI>(dq, t0 + l16, 16 * w + 4 * g, rope_w, -1.0f);
            }
            if constexpr (PHI == PHI_HEXP) {
            } else if constexpr (FW) {
                buffer_store_f4(buf_rsrc(dQ + (rb + t0) * D), okt ? soff * 4u : kDropOffset, dq);
            } else if (okt) {
                store4<VEC>(dQ + (rb + t0 + l16) * D, 16 * w + 4 * g, D, dq);
            }
        }
        // S* += phi(Q)^T dnum (columns e of tile w); z* += phi(Q)^T dden (columns d of tile w)
        {
            f4 qC[4];
            getC(bQ, qC, l16, g);
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                f4 a = Sm[dt];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    a = mfma16(qC[dt][r], nCw[r], a);
                Sm[dt] = a;
            }
            // z*[d] += sum_t phi(Q_t)[d] dden_t: an MFMA whose every output column is
            // the same, in zs's layout
#pragma unroll
            for (int r = 0; r < 4; r++)
                zs = mfma16(qCw[r], ddS[r], zs);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    chunk(std::false_type{}, sa, nch - 1);   // the segment's last chunk
    int c = nch - 2;
    for (; c >= 1; c -= 2) {
        chunk(std::true_type{}, sb, c);
        chunk(std::true_type{}, sa, c - 1);
    }
    if (c == 0)
        chunk(std::true_type{}, sb, 0);
    if constexpr (PHI == PHI_HEXP) {
        __syncthreads();
        flush();
    }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The fused kernels take D, E <= 64 and address a sequence's rows with 32-bit
// byte offsets; short sequences take the quadratic form instead.
bool lin_bwd_fused_ok(int D, int E, long S)
{
    return D >= 1 && E >= 1 && D <= 64 && E <= 64 && S >= 1 && S < (1L << 22) &&
           !lin_quad_ok(D, E, S);
}

int lin_bwd_slots()
{
    static int per_cu = 0;
    if (per_cu <= 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)lin_bwd_kernel<PHI_ELU1, true, true>, BWD_THREADS, 0) !=
                hipSuccess ||
            n <= 0)
            n = 2;
        per_cu = n;
    }
    return per_cu;
}

// Anchors kept without a context: those inside the first backward segment
// (later segments start from their own end prefix), formed by lin_bagg.
static int bwd_nanch_noctx(const LinPlan& p, int S)
{
    const long nchs = (S + 15) / 16;
    return lin_nanch(std::min<long>(p.L / 16, nchs));
}

size_t lin_bwd_ws_bytes(const LinPlan& p, int Bq, int S)
{
    const long nchs = (S + 15) / 16;
    return ((size_t)2 * Bq * p.nseg * LIN_WS + (size_t)Bq * nchs * 64 +
            (size_t)Bq * bwd_nanch_noctx(p, S) * LIN_ANCH) *
           sizeof(float);
}

size_t lin_ctx_bytes(int Bq, int S, int D, int E)
{
    if (lin_qs_path(Bq, S, D, E))
        return lin_qs_ctx_bytes(Bq, S, D, E);
    if (!lin_bwd_fused_ok(D, E, S))
        return 0;
    const LinPlan pf = lin_plan(Bq, S, D, E, LIN_PASS_FWD);
    const long nchs = (S + 15) / 16;
    return ((size_t)Bq * (pf.nseg + 1) * LIN_WS + (size_t)Bq * nchs * 64 +
            (size_t)Bq * lin_nanch(nchs) * LIN_ANCH) *
           sizeof(float);
}

LinCtx lin_ctx_split(void* ctx, int Bq, int S, int D, int E)
{
    const LinPlan pf = lin_plan(Bq, S, D, E, LIN_PASS_FWD);
    const long nchs = (S + 15) / 16;
    LinCtx c;
    c.rec = (float*)ctx;
    c.tot = c.rec + (size_t)Bq * pf.nseg * LIN_WS;
    c.zt = c.tot + (size_t)Bq * LIN_WS;
    c.anch = c.zt + (size_t)Bq * nchs * 64;
    return c;
}

// Launch context: with the forward's context (c.tot != null) the prefix
// records and the z table come from it and only the suffix aggregates are
// formed; mf forward segments make one backward segment.
struct BwdArgs {
    float *wsP, *wsB, *zt, *anch;   // anch: the anchors lin_bagg forms (no context)
    LinCtx c;
    int mf, nsegf;
};

template <int PHI, bool VEC, bool FW>
static void bwd_launch_t(const LinPlan& p, const float* Q, const float* K, const float* V,
                         const float* O, const float* dO, const float* den, float* dQ, float* dK,
                         float* dV, const BwdArgs& a, int Bq, int S, int D, int E, hipStream_t st)
{
    const int nchs = (S + 15) / 16;
    const bool pre = a.c.tot == nullptr;
    // anchors: the context's (every 2^k below the sequence's chunk count), or
    // those lin_bagg forms inside the first segment
    const int nanch = pre ? bwd_nanch_noctx(p, S) : lin_nanch(nchs);
    const unsigned nb = (unsigned)((pre ? Bq * p.nseg : 0) + Bq * (p.nseg - 1));
    const LinRopeArg<PHI> rope = lin_rope_arg<PHI>(D);
    if (nb > 0) {
        ProfScope ps(st, "lin_bagg");
        CXG_LAUNCH((lin_bagg_kernel<PHI, VEC, FW>), dim3(nb), dim3(BAGG_THREADS), 0, st,
                           Q, K, V, O, dO, den, a.wsP, a.wsB, a.zt, a.anch, pre ? nanch : 0, Bq,
                           S, D, E, p.nseg, p.L, nchs, pre ? 1 : 0, rope);
    }
    {
        ProfScope ps(st, "lin_bscan");
        const long n = (pre ? 2L : 1L) * Bq * LIN_WS;
        CXG_LAUNCH(lin_bscan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           a.wsP, a.wsB, Bq, p.nseg, pre ? 1 : 0);
    }
    ProfScope ps(st, "lin_bwd");
    CXG_LAUNCH((lin_bwd_kernel<PHI, VEC, FW>), dim3((unsigned)(Bq * p.nseg)),
                       dim3(BWD_THREADS), 0, st, Q, K, V, O, dO, den, dQ, dK, dV, a.wsP, a.wsB,
                       pre ? a.zt : a.c.zt, a.c.rec, a.c.tot, pre ? a.anch : a.c.anch, nanch,
                       a.mf, a.nsegf, S, D, E, p.nseg, p.L, nchs, rope);
}

template <int PHI>
static void bwd_dispatch(const LinPlan& p, const float* Q, const float* K, const float* V,
                         const float* O, const float* dO, const float* den, float* dQ, float* dK,
                         float* dV, const BwdArgs& a, int Bq, int S, int D, int E, hipStream_t st)
{
    const bool vec = D % 4 == 0 && E % 4 == 0 && al16(Q) && al16(K) && al16(V) && al16(O) &&
                     al16(dO) && al16(dQ) && al16(dK) && al16(dV);
    if (vec && D == 64 && E == 64)
        bwd_launch_t<PHI, true, true>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else if constexpr (PHI == PHI_HEXP)
        return;   // D = E = 64 with 16-byte rows only (checked by the launcher)
    else if (vec)
        bwd_launch_t<PHI, true, false>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else
        bwd_launch_t<PHI, false, false>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
}

// Backward segments: the backward's own plan, or with a context whole groups
// of mf forward segments (so every backward segment ends on a boundary whose
// prefix record the forward kept), about as many as the backward's own plan.
static LinPlan bwd_plan(int Bq, int S, int D, int E, bool with_ctx, int* mf, int* nsegf)
{
    LinPlan p = lin_plan(Bq, S, D, E, LIN_PASS_BWD);
    *mf = 1;
    *nsegf = 0;
    if (with_ctx) {
        const LinPlan pf = lin_plan(Bq, S, D, E, LIN_PASS_FWD);
        *nsegf = pf.nseg;
        *mf = max(1, pf.nseg / max(1, p.nseg));
        p.L = pf.L * *mf;
        p.nseg = (pf.nseg + *mf - 1) / *mf;
    }
    return p;
}

hipError_t lin_bwd_fused_launch(int phi, const float* Q, const float* K, const float* V,
                                const float* O, const float* dO, const float* den, float* dQ,
                                float* dK, float* dV, int Bq, int S, int D, int E, void* ws,
                                hipStream_t st, const void* ctx)
{
    BwdArgs a;
    const LinPlan p = bwd_plan(Bq, S, D, E, ctx != nullptr, &a.mf, &a.nsegf);
    a.wsP = (float*)ws;
    a.wsB = a.wsP + (size_t)Bq * p.nseg * LIN_WS;
    a.zt = a.wsB + (size_t)Bq * p.nseg * LIN_WS;
    a.anch = a.zt + (size_t)Bq * ((S + 15) / 16) * 64;
    a.c = ctx != nullptr ? lin_ctx_split(const_cast<void*>(ctx), Bq, S, D, E)
                         : LinCtx{nullptr, nullptr, nullptr, nullptr};
    if (phi == PHI_HEXP && !(D == 64 && E == 64 && al16(Q) && al16(K) && al16(V) && al16(O) &&
                             al16(dO) && al16(dQ) && al16(dK) && al16(dV)))
        return hipErrorInvalidValue;
    if (phi == PHI_ELU1)
        bwd_dispatch<PHI_ELU1>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else if (phi == PHI_ELU1_LG)
        bwd_dispatch<PHI_ELU1_LG>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else if (phi == PHI_HEXP)
        bwd_dispatch<PHI_HEXP>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else if (phi == PHI_ELU1_ROPE)
        bwd_dispatch<PHI_ELU1_ROPE>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    else
        bwd_dispatch<PHI_NONE>(p, Q, K, V, O, dO, den, dQ, dK, dV, a, Bq, S, D, E, st);
    return hipGetLastError();
}

size_t lin_bwd_fused_ws_bytes(int Bq, int S, int D, int E, bool with_ctx)
{
    int mf, nsegf;
    return lin_bwd_ws_bytes(bwd_plan(Bq, S, D, E, with_ctx, &mf, &nsegf), Bq, S);
}

} // namespace cxg
