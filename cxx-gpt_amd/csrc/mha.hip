// mha.hip -- fused causal softmax multi-head attention for gfx950 (FP32 MFMA).
//
// Replaces two_stage_cuda::fused_mha_fwd / fused_mha_bwd
// (src/TwoStage/two_stage_cuda_kernels.cu:285-326, :830-882) and every kernel
// they dispatch to (primary, tiled long-sequence, warp and scratch
// fallbacks).  One algorithm covers every sequence length: K/V stream
// through LDS in 64-row tiles with an online softmax, and the backward pass
// recomputes the probabilities tile by tile, so no S x S buffer exists at any
// length.
//
// Layout: Q/K/V/O/dO/dQ/dK/dV are (B*S, H*Dh) row-major; head h of row r is
// [(r*H + h)*Dh, +Dh).  lse and Di are [B*H][S].
//
// Work decomposition.  A workgroup has 4*NSPLIT waves: four "row groups" of
// 16 rows times NSPLIT "splits", so two waves share each SIMD and hide one
// another's LDS / exp / memory latency behind MFMA work.
//   forward : a workgroup owns 64 query rows of one (b,h); wave (qg, ks) owns
//             queries 16qg..16qg+15 and keys [64/NSPLIT * ks, +64/NSPLIT) of
//             every 64-key tile, keeping its own online-softmax state; the
//             NSPLIT partial states are merged through LDS at the end.
//             Scores are computed transposed (S^T = K Q^T) so a lane holds one
//             query and the softmax statistics need one cross-row shuffle.
//   backward: a workgroup owns 64 key rows of one (b,h); wave (kg, qs) owns
//             keys 16kg..16kg+15 (K/V in registers) and rows
//             [BM/NSPLIT * qs, +BM/NSPLIT) of every BM-row query tile; it
//             accumulates partial dK^T/dV^T in registers (summed over the
//             splits through LDS at the end) and adds dQ = dS K into the
//             zero-initialised dQ with float atomics.
// The flat grid index is (tile * B*H + bh): heavy causal tiles dispatch first,
// and when B*H is a multiple of 8 all tiles of a head share an XCD (and its
// L2), since workgroups are dealt to the 8 XCDs round-robin.
#include "common.hpp"
#include "launch.hpp"

#include <math.h>

namespace cxg {

constexpr int MHA_BM = 64;   // query rows per tile
constexpr int MHA_BN = 64;   // key rows per tile

// ROWS x DHP fp32 tile of one head, held in registers between its global load
// and its LDS store (so the next tile's loads overlap the current tile's math).
// Thread tid of NT owns f4 units u = tid + i*NT: row u / (DHP/4), column
// 4*(u % (DHP/4)).  Rows past S repeat row S-1 and columns past Dh repeat real
// columns (load4c).
template <int DHP, int ROWS, int NT, bool VEC>
struct TileRegs {
    static constexpr int CPR = DHP / 4;   // f4 units per row
    static constexpr int NU = ROWS * CPR;
    static constexpr int UPT = (NU + NT - 1) / NT;
    f4 r[UPT];

    __device__ __forceinline__ void load(const float* __restrict__ X, long base, long rs,
                                         int row0, int S, int Dh, int tid)
    {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = min(tid + i * NT, NU - 1);
            const int row = u / CPR, c = 4 * (u - row * CPR);
            const int gr = min(row0 + row, S - 1);
            r[i] = load4c<VEC>(X + base + (long)gr * rs, c, Dh);
        }
    }
    // row-major [row][c] with row stride LD floats
    template <int LD>
    __device__ __forceinline__ void store(float* __restrict__ T, int tid) const
    {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + i * NT;
            if (NU % NT == 0 || u < NU) {
                const int row = u / CPR, c = 4 * (u - row * CPR);
                *reinterpret_cast<f4*>(&T[row * LD + c]) = r[i];
            }
        }
    }
    // transposed [c][row] with row stride LD floats
    template <int LD>
    __device__ __forceinline__ void store_t(float* __restrict__ T, int tid) const
    {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + i * NT;
            if (NU % NT == 0 || u < NU) {
                const int row = u / CPR, c = 4 * (u - row * CPR);
                T[(c + 0) * LD + row] = r[i][0];
                T[(c + 1) * LD + row] = r[i][1];
                T[(c + 2) * LD + row] = r[i][2];
                T[(c + 3) * LD + row] = r[i][3];
            }
        }
    }
};

// ----------------------------------------------------------------------------
// forward (and statistics-only) kernel
// ----------------------------------------------------------------------------
template <int DHP, int NSPLIT>
struct FwdSmem {
    static constexpr int KS = DHP + 4;      // Ks[key][d] row stride (floats)
    static constexpr int MS = DHP + 4;      // merge record: o[DHP], m, l
    static constexpr int TILES = 2 * MHA_BN * KS;   // Ks and Vs, both [key][d]
    static constexpr bool DB = DHP <= 64;    // double-buffered K/V tiles
    static constexpr int MERGE = (NSPLIT - 1) * MHA_BM * MS;
    static constexpr int FLOATS = (DB ? 2 : 1) * TILES > MERGE ? (DB ? 2 : 1) * TILES : MERGE;
};

template <int DHP, int NSPLIT, bool VEC, bool WRITE_O>
__global__ __launch_bounds__(256 * NSPLIT) void mha_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int S, int H, int Dh, int BH, int nqb,
    float qscale)
{
    using SM = FwdSmem<DHP, NSPLIT>;
    constexpr int NT = 256 * NSPLIT;
    constexpr int KS = SM::KS, MS = SM::MS;
    constexpr int NDT = DHP / 16;
    constexpr int NKT = 4 / NSPLIT;   // 16-key blocks per wave per tile
    __shared__ __attribute__((aligned(16))) float smem[SM::FLOATS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int qg = wave & 3, ks = wave >> 2;
    const int qi = blockIdx.x / BH, bh = blockIdx.x - qi * BH;
    const int qb = nqb - 1 - qi;
    const int b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;

    const int myq = qb * MHA_BM + qg * 16 + l16;
    const bool qok = myq < S;
    // B operand of S^T = K Q^T: lane holds Q[myq][16*dt + 4*g + r], pre-scaled
    // by scale*log2(e) so scores land in the exp2 domain; zero past Dh.
    f4 qreg[NDT];
    {
        const float* qrow = Q + base + (long)(qok ? myq : 0) * rs;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            qreg[dt] = load4<VEC>(qrow, 16 * dt + 4 * g, Dh, qok) * qscale;
    }
    f4 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
        oacc[dt] = f4zero();
    float m_run = -1e30f, l_run = 0.0f;

    const int nkb = qb + 1;   // causal: key tiles 0..qb (MHA_BM == MHA_BN)
    // One key tile of math on the tiles in LDS (Ks, Vs: [key][d], row stride KS).
    auto tile_math = [&](const float* __restrict__ Ks, const float* __restrict__ Vs, int kb) {
        const int k0 = kb * MHA_BN;
        // S^T block kt of this wave: lane holds query l16, keys k0 + 16*kt + 4*g + r.
        // The NKT key blocks run as interleaved accumulation chains.
        f4 sacc[NKT];
#pragma unroll
        for (int kk = 0; kk < NKT; kk++)
            sacc[kk] = f4zero();
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
            for (int kk = 0; kk < NKT; kk++) {
                const int kt = ks * NKT + kk;
                const f4 kv = *reinterpret_cast<const f4*>(&Ks[(16 * kt + l16) * KS + 16 * dt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    sacc[kk] = mfma16(kv[r], qreg[dt][r], sacc[kk]);
            }
        }
        if (kb == qb) {   // diagonal tile: causal mask key > query
#pragma unroll
            for (int kk = 0; kk < NKT; kk++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (k0 + 16 * (ks * NKT + kk) + 4 * g + r > myq)
                        sacc[kk][r] = -INFINITY;
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < NKT; kk++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                mloc = fmaxf(mloc, sacc[kk][r]);
        mloc = xrow_max(mloc);
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = fast_exp2(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int kk = 0; kk < NKT; kk++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = fast_exp2(sacc[kk][r] - m_new);
                sacc[kk][r] = p;
                psum += p;
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (WRITE_O) {
            // O^T += V^T P^T: A = V^T[d = 16dt + l16][key = 16kt + 4g + r], read
            // as single floats from the row-major V tile; B = P^T from sacc.
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                f4 acc = oacc[dt] * alpha;
#pragma unroll
                for (int kk = 0; kk < NKT; kk++) {
                    const int kt = ks * NKT + kk;
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(Vs[(16 * kt + 4 * g + r) * KS + 16 * dt + l16], sacc[kk][r], acc);
                }
                oacc[dt] = acc;
            }
        }
    };
    // Narrow heads (DB) run a four-deep pipeline: two register stages, loaded
    // from global memory three tiles ahead of use, feed two LDS buffers; tile
    // kb+1 is written to LDS while tile kb is consumed, one barrier per tile.
    // Wider heads use one LDS buffer (two barriers per tile) and one register
    // stage (none for the widest).
    TileRegs<DHP, MHA_BN, NT, VEC> kr, vr;
    auto load_kv = [&](TileRegs<DHP, MHA_BN, NT, VEC>& kx, TileRegs<DHP, MHA_BN, NT, VEC>& vx,
                       int kb) {
        kx.load(K, base, rs, kb * MHA_BN, S, Dh, tid);
        if (WRITE_O)
            vx.load(V, base, rs, kb * MHA_BN, S, Dh, tid);
    };
    auto store_kv = [&](const TileRegs<DHP, MHA_BN, NT, VEC>& kx,
                        const TileRegs<DHP, MHA_BN, NT, VEC>& vx, float* buf) {
        kx.template store<KS>(buf, tid);
        if (WRITE_O)
            vx.template store<KS>(buf + MHA_BN * KS, tid);
    };
    load_kv(kr, vr, 0);
    if constexpr (SM::DB) {
        TileRegs<DHP, MHA_BN, NT, VEC> kr1, vr1;
        if (nkb > 1)
            load_kv(kr1, vr1, 1);
        store_kv(kr, vr, smem);
        if (nkb > 2)
            load_kv(kr, vr, 2);
        __syncthreads();
        // Iteration kb: registers (kx, vx) hold tile kb+1; they go to LDS
        // buffer (kb+1)&1 and are refilled with tile kb+3.
        auto step = [&](TileRegs<DHP, MHA_BN, NT, VEC>& kx, TileRegs<DHP, MHA_BN, NT, VEC>& vx,
                        int kb) {
            const float* cur = smem + (kb & 1) * SM::TILES;
            if (kb + 1 < nkb) {
                store_kv(kx, vx, smem + ((kb + 1) & 1) * SM::TILES);
                if (kb + 3 < nkb)
                    load_kv(kx, vx, kb + 3);
            }
            tile_math(cur, cur + MHA_BN * KS, kb);
            __syncthreads();
        };
        for (int kb = 0; kb < nkb; kb += 2) {
            step(kr1, vr1, kb);
            if (kb + 1 < nkb)
                step(kr, vr, kb + 1);
        }
    } else {
        constexpr bool PREFETCH = DHP <= 128;
        for (int kb = 0; kb < nkb; kb++) {
            if (!PREFETCH && kb > 0)
                load_kv(kr, vr, kb);
            __syncthreads();
            store_kv(kr, vr, smem);
            __syncthreads();
            if (PREFETCH && kb + 1 < nkb)
                load_kv(kr, vr, kb + 1);
            tile_math(smem, smem + MHA_BN * KS, kb);
        }
    }
    float l_tot = xrow_sum(l_run);

    if (NSPLIT > 1) {
        // Merge the key splits: split ks > 0 publishes (o, m, l) per query row,
        // split 0 rescales everything to the common maximum.
        float* mb = smem;
        __syncthreads();   // every wave is done with the K/V tiles
        const int qrow = qg * 16 + l16;
        if (ks > 0) {
            float* rec = mb + ((ks - 1) * MHA_BM + qrow) * MS;
            if (WRITE_O)
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
                    *reinterpret_cast<f4*>(&rec[16 * dt + 4 * g]) = oacc[dt];
            if (g == 0) {
                rec[DHP] = m_run;
                rec[DHP + 1] = l_tot;
            }
        }
        __syncthreads();
        if (ks > 0)
            return;
        float m_all = m_run;
#pragma unroll
        for (int j = 1; j < NSPLIT; j++)
            m_all = fmaxf(m_all, mb[((j - 1) * MHA_BM + qrow) * MS + DHP]);
        const float a0 = fast_exp2(m_run - m_all);
        l_tot *= a0;
        if (WRITE_O)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                oacc[dt] = oacc[dt] * a0;
#pragma unroll
        for (int j = 1; j < NSPLIT; j++) {
            const float* rec = mb + ((j - 1) * MHA_BM + qrow) * MS;
            const float aj = fast_exp2(rec[DHP] - m_all);
            l_tot += rec[DHP + 1] * aj;
            if (WRITE_O)
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
                    oacc[dt] += *reinterpret_cast<const f4*>(&rec[16 * dt + 4 * g]) * aj;
        }
        m_run = m_all;
    }
    if (qok) {
        if (WRITE_O) {
            const float inv = 1.0f / l_tot;
            float* orow = O + base + (long)myq * rs;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                store4<VEC>(orow, 16 * dt + 4 * g, Dh, oacc[dt] * inv);
        }
        if (lse != nullptr && g == 0)
            lse[(long)bh * S + myq] = (m_run + fast_log2(l_tot)) * kLn2;
    }
}

// ----------------------------------------------------------------------------
// backward pre-pass: Di = rowsum(dO * O) (the reference's gs, kernel_test.cpp:76-78)
// and dQ = 0.  16 lanes per (row, head) segment.
// ----------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void mha_bwd_prep_kernel(
    const float* __restrict__ O, const float* __restrict__ dO, float* __restrict__ Di,
    float* __restrict__ dQ, int S, int H, int Dh, long nseg)
{
    const long seg = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int sub = threadIdx.x & 15;
    const bool ok = seg < nseg;
    float acc = 0.0f;
    if (ok) {
        const long off = seg * Dh;   // segment (b*S + s)*H + h starts at seg*Dh
        for (int c = 4 * sub; c < Dh; c += 64) {
            const f4 o = load4<VEC>(O + off, c, Dh, true);
            const f4 d = load4<VEC>(dO + off, c, Dh, true);
            acc += o[0] * d[0] + o[1] * d[1] + o[2] * d[2] + o[3] * d[3];
            store4<VEC>(dQ + off, c, Dh, f4zero());
        }
    }
    acc = row16_sum(acc);
    if (ok && sub == 0) {
        const long row = seg / H;
        const int h = (int)(seg - row * H);
        const long b = row / S;
        const long s = row - b * S;
        Di[(b * H + h) * (long)S + s] = acc;
    }
}

// ----------------------------------------------------------------------------
// backward main kernel.  BM query rows per tile (64, or 32 for the widest
// heads so the LDS tiles fit in 160 KB), split over NSPLIT wave groups.
// ----------------------------------------------------------------------------
template <int DHP, int BM>
struct BwdSmem {
    static constexpr int QS = DHP + 4;      // Qs/dOs [q][d] row stride
    static constexpr int TS = MHA_BN + 4;   // Kt [d][key] and dSs [q][key] row stride
    // Narrow heads double-buffer the query-side tiles (Q, dO, lse, Di, dS) so
    // one barrier per query tile suffices.
    static constexpr bool DB = DHP <= 64;
    static constexpr int NB = DB ? 2 : 1;
    static constexpr int STAGE = 2 * BM * QS + BM * TS + 2 * BM;   // Q, dO, dS, lse, Di
    static constexpr int FLOATS = DHP * TS + NB * STAGE;
};

template <int DHP, int BM, int NSPLIT, bool VEC>
__global__ __launch_bounds__(256 * NSPLIT) void mha_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int S, int H, int Dh,
    int BH, int nkb, float scale, float c2)
{
    using SM = BwdSmem<DHP, BM>;
    constexpr int NT = 256 * NSPLIT;
    constexpr int NW = NT / 64;
    constexpr int NDT = DHP / 16;
    constexpr int NQT = BM / 16;        // 16-row query blocks per tile
    constexpr int NQW = NQT / NSPLIT;   // ... per wave
    constexpr int QS = SM::QS, TS = SM::TS;
    static_assert(NQW >= 1, "query split too fine for BM");
    __shared__ __attribute__((aligned(16))) float smem[SM::FLOATS];
    float* Kt = smem;
    // Stage i: Qs [BM][QS], dOs [BM][QS], dSs [BM][TS], lse_s [BM], di_s [BM].
    auto stage = [&](int i) { return smem + DHP * TS + i * SM::STAGE; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int kg = wave & 3, qs = wave >> 2;
    const int kb = blockIdx.x / BH, bh = blockIdx.x - kb * BH;
    const int b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;
    const int k0 = kb * MHA_BN;
    const int mykey = k0 + kg * 16 + l16;
    const bool kok = mykey < S;

    // B operands for S = Q K^T and dP = dO V^T: K/V[mykey][16dt + 4g + r], zero past Dh.
    f4 kreg[NDT], vreg[NDT];
    {
        const long off = base + (long)(kok ? mykey : 0) * rs;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            kreg[dt] = load4<VEC>(K + off, 16 * dt + 4 * g, Dh, kok);
            vreg[dt] = load4<VEC>(V + off, 16 * dt + 4 * g, Dh, kok);
        }
    }
    // K^T tile for the dQ product, written from the K operand registers by
    // the waves of query split 0 (their key blocks kg cover the tile).
    if (qs == 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                Kt[(16 * dt + 4 * g + r) * TS + kg * 16 + l16] = kreg[dt][r];
    }

    f4 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        dk[dt] = f4zero();
        dv[dt] = f4zero();
    }

    const int nqb = (S + BM - 1) / BM;
    // A query tile in registers on its way to LDS: Q and dO rows, and the
    // tile's lse and Di entries (lse is scaled by log2 e on its way to LDS).
    struct QTile {
        TileRegs<DHP, BM, NT, VEC> q, d;
        float lse, di;
    };
    auto load_q = [&](QTile& t, int q0) {
        t.q.load(Q, base, rs, q0, S, Dh, tid);
        t.d.load(dO, base, rs, q0, S, Dh, tid);
        if (tid < BM) {   // rows past S repeat row S-1; their P is masked to 0
            const long i = (long)bh * S + min(q0 + tid, S - 1);
            t.lse = lse[i];   // scaled at the LDS store: no use of loaded data here,
            t.di = Di[i];     // so the loads stay in flight
        }
    };
    auto store_q = [&](const QTile& t, float* st) {
        t.q.template store<QS>(st, tid);
        t.d.template store<QS>(st + BM * QS, tid);
        if (tid < BM) {
            st[2 * BM * QS + BM * TS + tid] = t.lse * kLog2e;
            st[2 * BM * QS + BM * TS + BM + tid] = t.di;
        }
    };
    // S = Q K^T and dP = dO V^T for this wave's query blocks (lane holds key
    // l16, queries 16qt + 4g + r); dS goes to LDS for the dQ product, then
    // dV^T += dO^T P and dK^T += Q^T dS accumulate in registers.
    auto key_side = [&](float* st, int q0) {
        const float* Qs = st;
        const float* dOs = st + BM * QS;
        float* dSs = st + 2 * BM * QS;
        const float* lse_s = st + 2 * BM * QS + BM * TS;
        const float* di_s = lse_s + BM;
        const bool diag = q0 < k0 + MHA_BN;   // tile touches the causal boundary
        // Query blocks are taken QI at a time so that 2*QI accumulation
        // chains interleave on the MFMA pipe.
        constexpr int QI = NQW <= 2 ? NQW : 1;
        f4 P[NQW], dS[NQW];
#pragma unroll
        for (int q1 = 0; q1 < NQW; q1 += QI) {
            f4 sa[QI], da[QI];
#pragma unroll
            for (int j = 0; j < QI; j++)
                sa[j] = da[j] = f4zero();
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                for (int j = 0; j < QI; j++) {
                    const int qt = qs * NQW + q1 + j;
                    const f4 qa = *reinterpret_cast<const f4*>(&Qs[(16 * qt + l16) * QS + 16 * dt + 4 * g]);
                    const f4 oa = *reinterpret_cast<const f4*>(&dOs[(16 * qt + l16) * QS + 16 * dt + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        sa[j] = mfma16(qa[r], kreg[dt][r], sa[j]);
                        da[j] = mfma16(oa[r], vreg[dt][r], da[j]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < QI; j++) {
                const int qq = q1 + j, qt = qs * NQW + qq;
                const f4 l4 = *reinterpret_cast<const f4*>(&lse_s[16 * qt + 4 * g]);
                const f4 d4 = *reinterpret_cast<const f4*>(&di_s[16 * qt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int q = q0 + 16 * qt + 4 * g + r;
                    const bool ok = (!diag || mykey <= q) && q < S;
                    const float p = ok ? fast_exp2(sa[j][r] * c2 - l4[r]) : 0.0f;
                    P[qq][r] = p;
                    dS[qq][r] = p * (da[j][r] - d4[r]);
                    dSs[(16 * qt + 4 * g + r) * TS + kg * 16 + l16] = dS[qq][r];
                }
            }
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            f4 av = dv[dt], ak = dk[dt];
#pragma unroll
            for (int qq = 0; qq < NQW; qq++) {
                const int qt = qs * NQW + qq;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = (16 * qt + 4 * g + r) * QS + 16 * dt + l16;
                    av = mfma16(dOs[row], P[qq][r], av);
                    ak = mfma16(Qs[row], dS[qq][r], ak);
                }
            }
            dv[dt] = av;
            dk[dt] = ak;
        }
    };
    // dQ tiles (qt, dt) of the query block, dealt round-robin to the waves:
    // dS (LDS) x K (LDS, transposed), added into dQ with float atomics.  A
    // wave's jobs share qt (NW is a multiple of NQT), so pairs of jobs run as
    // two interleaved MFMA chains over one read of the dS operand.
    constexpr int NJOB = NQT * NDT;
    constexpr int NJ = (NJOB + NW - 1) / NW;   // jobs per wave (the last may be empty)
    static_assert(NW % NQT == 0, "dQ jobs of a wave must share their query block");
    auto dq_store = [&](const f4& acc, int q0, int qt, int dt) {
        const int d = 16 * dt + l16;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int q = q0 + 16 * qt + 4 * g + r;
            if (q < S && d < Dh)
                atomic_add_f32(dQ + base + (long)q * rs + d, acc[r] * scale);
        }
    };
    auto query_side = [&](const float* st, int q0) {
        const float* dSs = st + 2 * BM * QS;
        const int qt = wave % NQT;
        const float* arow = dSs + (16 * qt + l16) * TS + 4 * g;
        if constexpr (NJ % 2 == 0) {
#pragma unroll
            for (int i = 0; i < NJ; i += 2) {
                const int dt0 = (wave + i * NW) / NQT, dt1 = (wave + (i + 1) * NW) / NQT;
                const float* b0 = Kt + (16 * dt0 + l16) * TS + 4 * g;
                const float* b1 = Kt + (16 * dt1 + l16) * TS + 4 * g;
                f4 acc0 = f4zero(), acc1 = f4zero();
#pragma unroll
                for (int kt = 0; kt < 4; kt++) {
                    const f4 a = *reinterpret_cast<const f4*>(arow + 16 * kt);
                    const f4 u = *reinterpret_cast<const f4*>(b0 + 16 * kt);
                    const f4 v = *reinterpret_cast<const f4*>(b1 + 16 * kt);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        acc0 = mfma16(a[r], u[r], acc0);
                        acc1 = mfma16(a[r], v[r], acc1);
                    }
                }
                dq_store(acc0, q0, qt, dt0);
                dq_store(acc1, q0, qt, dt1);
            }
        } else {
            for (int job = wave; job < NJOB; job += NW) {
                const int dt = job / NQT;
                const float* b0 = Kt + (16 * dt + l16) * TS + 4 * g;
                f4 acc = f4zero();
#pragma unroll
                for (int kt = 0; kt < 4; kt++) {
                    const f4 a = *reinterpret_cast<const f4*>(arow + 16 * kt);
                    const f4 u = *reinterpret_cast<const f4*>(b0 + 16 * kt);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(a[r], u[r], acc);
                }
                dq_store(acc, q0, qt, dt);
            }
        }
    };

    const int qb0 = k0 / BM;
    QTile t0;
    t0.lse = t0.di = 0.0f;
    load_q(t0, qb0 * BM);
    if constexpr (SM::DB) {
        // Four-deep pipeline: two register stages loaded three query tiles
        // ahead of use, two LDS stages.  Tile qb is in stage qb&1 when
        // iteration qb starts.  The iteration writes dS into its own stage
        // (the dQ jobs read it after the barrier) and, once its own S/dP/dV/dK
        // work is issued, tile qb+1 into the Q/dO/lse/Di part of the other
        // stage: that part was last read before the previous barrier, and the
        // dQ jobs of iteration qb-1 still running on other waves read only the
        // other stage's dS part.  Writing the next tile after the key-side
        // work, rather than at the top, leaves the dQ atomics and loads of the
        // previous iteration time to drain before the wait for its registers.
        QTile t1;
        t1.lse = t1.di = 0.0f;
        if (qb0 + 1 < nqb)
            load_q(t1, (qb0 + 1) * BM);
        store_q(t0, stage(qb0 & 1));
        if (qb0 + 2 < nqb)
            load_q(t0, (qb0 + 2) * BM);
        __syncthreads();
        // Iteration qb: registers tx hold tile qb+1 and are refilled with qb+3.
        auto step = [&](QTile& tx, int qb) {
            const int q0 = qb * BM;
            float* cur = stage(qb & 1);
            key_side(cur, q0);
            if (qb + 1 < nqb) {
                store_q(tx, stage((qb + 1) & 1));
                if (qb + 3 < nqb)
                    load_q(tx, q0 + 3 * BM);
            }
            __syncthreads();
            query_side(cur, q0);
        };
        for (int qb = qb0; qb < nqb; qb += 2) {
            step(t1, qb);
            if (qb + 1 < nqb)
                step(t0, qb + 1);
        }
    } else {
        constexpr bool PREFETCH = DHP <= 128;
        float* st = stage(0);
        for (int qb = qb0; qb < nqb; qb++) {
            const int q0 = qb * BM;
            if (!PREFETCH && qb > qb0)
                load_q(t0, q0);
            __syncthreads();
            store_q(t0, st);
            __syncthreads();
            if (PREFETCH && qb + 1 < nqb)
                load_q(t0, q0 + BM);
            key_side(st, q0);
            __syncthreads();
            query_side(st, q0);
        }
    }

    if (NSPLIT > 1) {
        // Sum the per-split partial dK^T/dV^T: splits qs > 0 publish through
        // LDS (reusing the Q/dO tiles), split 0 adds and stores.
        constexpr int RS = 2 * DHP + 4;   // record per (split, key): dk[DHP], dv[DHP]
        static_assert((NSPLIT - 1) * MHA_BN * RS <= SM::FLOATS,
                      "dK/dV reduction buffer does not fit");
        float* rb = smem;
        __syncthreads();   // every wave is done with the tiles
        const int krow = kg * 16 + l16;
        if (qs > 0) {
            float* rec = rb + ((qs - 1) * MHA_BN + krow) * RS;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                *reinterpret_cast<f4*>(&rec[16 * dt + 4 * g]) = dk[dt];
                *reinterpret_cast<f4*>(&rec[DHP + 16 * dt + 4 * g]) = dv[dt];
            }
        }
        __syncthreads();
        if (qs > 0)
            return;
#pragma unroll
        for (int j = 1; j < NSPLIT; j++) {
            const float* rec = rb + ((j - 1) * MHA_BN + krow) * RS;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                dk[dt] += *reinterpret_cast<const f4*>(&rec[16 * dt + 4 * g]);
                dv[dt] += *reinterpret_cast<const f4*>(&rec[DHP + 16 * dt + 4 * g]);
            }
        }
    }
    if (kok) {
        const long off = base + (long)mykey * rs;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            store4<VEC>(dK + off, 16 * dt + 4 * g, Dh, dk[dt] * scale);
            store4<VEC>(dV + off, 16 * dt + 4 * g, Dh, dv[dt]);
        }
    }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Wave groups per workgroup: two per SIMD wherever registers allow.
template <int DHP>
struct MhaSplits {
    static constexpr int FWD = DHP <= 128 ? 2 : 1;
    static constexpr int BWD = DHP <= 64 ? 2 : 1;
    static constexpr int BWD_BM = DHP <= 128 ? 64 : 32;
};

template <int DHP, bool VEC>
static hipError_t fwd_dispatch2(const float* Q, const float* K, const float* V, float* O,
                                float* lse, int B, int S, int H, int Dh, hipStream_t st)
{
    constexpr int NS = MhaSplits<DHP>::FWD;
    const int BH = B * H;
    const int nqb = (S + MHA_BM - 1) / MHA_BM;
    const float qscale = (1.0f / sqrtf((float)Dh)) * kLog2e;
    dim3 grid((unsigned)(nqb * BH)), block(256 * NS);
    if (O != nullptr) {
        ProfScope ps(st, "mha_fwd");
        hipLaunchKernelGGL((mha_fwd_kernel<DHP, NS, VEC, true>), grid, block, 0, st, Q, K, V, O,
                           lse, S, H, Dh, BH, nqb, qscale);
    } else {
        ProfScope ps(st, "mha_stats");
        hipLaunchKernelGGL((mha_fwd_kernel<DHP, NS, VEC, false>), grid, block, 0, st, Q, K, V, O,
                           lse, S, H, Dh, BH, nqb, qscale);
    }
    return hipGetLastError();
}

template <int DHP>
static hipError_t fwd_dispatch(const float* Q, const float* K, const float* V, float* O,
                               float* lse, int B, int S, int H, int Dh, hipStream_t st)
{
    const bool vec = (Dh % 4 == 0) && aligned16(Q) && aligned16(K) && aligned16(V) &&
                     (O == nullptr || aligned16(O));
    if (vec)
        return fwd_dispatch2<DHP, true>(Q, K, V, O, lse, B, S, H, Dh, st);
    return fwd_dispatch2<DHP, false>(Q, K, V, O, lse, B, S, H, Dh, st);
}

hipError_t mha_fwd_launch(const float* Q, const float* K, const float* V, float* O, float* lse,
                          int B, int S, int H, int Dh, hipStream_t st)
{
    if (Dh <= 16)
        return fwd_dispatch<16>(Q, K, V, O, lse, B, S, H, Dh, st);
    if (Dh <= 32)
        return fwd_dispatch<32>(Q, K, V, O, lse, B, S, H, Dh, st);
    if (Dh <= 64)
        return fwd_dispatch<64>(Q, K, V, O, lse, B, S, H, Dh, st);
    if (Dh <= 128)
        return fwd_dispatch<128>(Q, K, V, O, lse, B, S, H, Dh, st);
    return fwd_dispatch<256>(Q, K, V, O, lse, B, S, H, Dh, st);
}

hipError_t mha_bwd_prep_launch(const float* O, const float* dO, float* Di, float* dQ, int B,
                               int S, int H, int Dh, hipStream_t st)
{
    const long nseg = (long)B * S * H;
    dim3 grid((unsigned)((nseg * 16 + 255) / 256)), block(256);
    ProfScope ps(st, "mha_bwd_prep");
    const bool vec = (Dh % 4 == 0) && aligned16(O) && aligned16(dO) && aligned16(dQ);
    if (vec)
        hipLaunchKernelGGL((mha_bwd_prep_kernel<true>), grid, block, 0, st, O, dO, Di, dQ, S, H,
                           Dh, nseg);
    else
        hipLaunchKernelGGL((mha_bwd_prep_kernel<false>), grid, block, 0, st, O, dO, Di, dQ, S,
                           H, Dh, nseg);
    return hipGetLastError();
}

template <int DHP>
static hipError_t bwd_dispatch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st)
{
    constexpr int NS = MhaSplits<DHP>::BWD, BM = MhaSplits<DHP>::BWD_BM;
    const int BH = B * H;
    const int nkb = (S + MHA_BN - 1) / MHA_BN;
    const float scale = 1.0f / sqrtf((float)Dh);
    dim3 grid((unsigned)(nkb * BH)), block(256 * NS);
    const bool vec = (Dh % 4 == 0) && aligned16(Q) && aligned16(K) && aligned16(V) &&
                     aligned16(dO) && aligned16(dK) && aligned16(dV);
    ProfScope ps(st, "mha_bwd");
    if (vec)
        hipLaunchKernelGGL((mha_bwd_kernel<DHP, BM, NS, true>), grid, block, 0, st, Q, K, V, dO,
                           lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e);
    else
        hipLaunchKernelGGL((mha_bwd_kernel<DHP, BM, NS, false>), grid, block, 0, st, Q, K, V, dO,
                           lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e);
    return hipGetLastError();
}

hipError_t mha_bwd_main_launch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st)
{
    if (Dh <= 16)
        return bwd_dispatch<16>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 32)
        return bwd_dispatch<32>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 64)
        return bwd_dispatch<64>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 128)
        return bwd_dispatch<128>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    return bwd_dispatch<256>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
}

} // namespace cxg
