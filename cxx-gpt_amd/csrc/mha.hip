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
    static constexpr int VS = MHA_BN + 4;   // Vt[d][key] row stride
    static constexpr int MS = DHP + 4;      // merge record: o[DHP], m, l
    static constexpr int TILES = MHA_BN * KS + DHP * VS;
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
    constexpr int KS = SM::KS, VS = SM::VS, MS = SM::MS;
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
    // One key tile of math on the tile in LDS (Ks, Vt).
    auto tile_math = [&](const float* __restrict__ Ks, const float* __restrict__ Vt, int kb) {
        const int k0 = kb * MHA_BN;
        // S^T block kt of this wave: lane holds query l16, keys k0 + 16*kt + 4*g + r.
        f4 sacc[NKT];
#pragma unroll
        for (int kk = 0; kk < NKT; kk++) {
            const int kt = ks * NKT + kk;
            f4 acc = f4zero();
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const f4 kv = *reinterpret_cast<const f4*>(&Ks[(16 * kt + l16) * KS + 16 * dt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(kv[r], qreg[dt][r], acc);
            }
            if (kb == qb) {   // diagonal tile: causal mask key > query
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (k0 + 16 * kt + 4 * g + r > myq)
                        acc[r] = -INFINITY;
            }
            sacc[kk] = acc;
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
            // O^T += V^T P^T: A = V^T[d = 16dt + l16][key], B = P^T from sacc.
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                f4 acc = oacc[dt] * alpha;
#pragma unroll
                for (int kk = 0; kk < NKT; kk++) {
                    const int kt = ks * NKT + kk;
                    const f4 vv = *reinterpret_cast<const f4*>(&Vt[(16 * dt + l16) * VS + 16 * kt + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(vv[r], sacc[kk][r], acc);
                }
                oacc[dt] = acc;
            }
        }
    };
    // K/V tiles are loaded into registers one tile ahead.  Narrow heads
    // double-buffer the LDS tiles: tile kb+1 is written while tile kb is
    // consumed, one barrier per tile; wider heads use one buffer (two
    // barriers per tile, and no register prefetch for the widest).
    TileRegs<DHP, MHA_BN, NT, VEC> kr, vr;
    kr.load(K, base, rs, 0, S, Dh, tid);
    if (WRITE_O)
        vr.load(V, base, rs, 0, S, Dh, tid);
    if constexpr (SM::DB) {
        kr.template store<KS>(smem, tid);
        if (WRITE_O)
            vr.template store_t<VS>(smem + MHA_BN * KS, tid);
        if (nkb > 1) {
            kr.load(K, base, rs, MHA_BN, S, Dh, tid);
            if (WRITE_O)
                vr.load(V, base, rs, MHA_BN, S, Dh, tid);
        }
        __syncthreads();
        for (int kb = 0; kb < nkb; kb++) {
            const float* cur = smem + (kb & 1) * SM::TILES;
            if (kb + 1 < nkb) {
                float* nxt = smem + ((kb + 1) & 1) * SM::TILES;
                kr.template store<KS>(nxt, tid);
                if (WRITE_O)
                    vr.template store_t<VS>(nxt + MHA_BN * KS, tid);
                if (kb + 2 < nkb) {
                    kr.load(K, base, rs, (kb + 2) * MHA_BN, S, Dh, tid);
                    if (WRITE_O)
                        vr.load(V, base, rs, (kb + 2) * MHA_BN, S, Dh, tid);
                }
            }
            tile_math(cur, cur + MHA_BN * KS, kb);
            __syncthreads();
        }
    } else {
        constexpr bool PREFETCH = DHP <= 128;
        for (int kb = 0; kb < nkb; kb++) {
            const int k0 = kb * MHA_BN;
            if (!PREFETCH && kb > 0) {
                kr.load(K, base, rs, k0, S, Dh, tid);
                if (WRITE_O)
                    vr.load(V, base, rs, k0, S, Dh, tid);
            }
            __syncthreads();
            kr.template store<KS>(smem, tid);
            if (WRITE_O)
                vr.template store_t<VS>(smem + MHA_BN * KS, tid);
            __syncthreads();
            if (PREFETCH && kb + 1 < nkb) {
                kr.load(K, base, rs, k0 + MHA_BN, S, Dh, tid);
                if (WRITE_O)
                    vr.load(V, base, rs, k0 + MHA_BN, S, Dh, tid);
            }
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
    // K^T tile for the dQ product.
    {
        TileRegs<DHP, MHA_BN, NT, VEC> kt;
        kt.load(K, base, rs, k0, S, Dh, tid);
        kt.template store_t<TS>(Kt, tid);
    }

    f4 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        dk[dt] = f4zero();
        dv[dt] = f4zero();
    }

    const int nqb = (S + BM - 1) / BM;
    // Q/dO tiles and their lse/Di entries pass through registers one query
    // tile ahead of their store to LDS (DHP <= 128).
    TileRegs<DHP, BM, NT, VEC> qr, dor;
    float lse_r = 0.0f, di_r = 0.0f;
    auto load_q = [&](int q0) {
        qr.load(Q, base, rs, q0, S, Dh, tid);
        dor.load(dO, base, rs, q0, S, Dh, tid);
        if (tid < BM) {   // rows past S repeat row S-1; their P is masked to 0
            const long i = (long)bh * S + min(q0 + tid, S - 1);
            lse_r = lse[i] * kLog2e;
            di_r = Di[i];
        }
    };
    auto store_q = [&](float* st) {
        qr.template store<QS>(st, tid);
        dor.template store<QS>(st + BM * QS, tid);
        if (tid < BM) {
            st[2 * BM * QS + BM * TS + tid] = lse_r;
            st[2 * BM * QS + BM * TS + BM + tid] = di_r;
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
        f4 P[NQW], dS[NQW];
#pragma unroll
        for (int qq = 0; qq < NQW; qq++) {
            const int qt = qs * NQW + qq;
            f4 sa = f4zero(), da = f4zero();
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const f4 qa = *reinterpret_cast<const f4*>(&Qs[(16 * qt + l16) * QS + 16 * dt + 4 * g]);
                const f4 oa = *reinterpret_cast<const f4*>(&dOs[(16 * qt + l16) * QS + 16 * dt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    sa = mfma16(qa[r], kreg[dt][r], sa);
                    da = mfma16(oa[r], vreg[dt][r], da);
                }
            }
            const f4 l4 = *reinterpret_cast<const f4*>(&lse_s[16 * qt + 4 * g]);
            const f4 d4 = *reinterpret_cast<const f4*>(&di_s[16 * qt + 4 * g]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int q = q0 + 16 * qt + 4 * g + r;
                const bool ok = (!diag || mykey <= q) && q < S;
                const float p = ok ? fast_exp2(sa[r] * c2 - l4[r]) : 0.0f;
                P[qq][r] = p;
                dS[qq][r] = p * (da[r] - d4[r]);
                dSs[(16 * qt + 4 * g + r) * TS + kg * 16 + l16] = dS[qq][r];
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
    // dS (LDS) x K (LDS, transposed), added into dQ with float atomics.
    auto query_side = [&](const float* st, int q0) {
        const float* dSs = st + 2 * BM * QS;
        for (int job = wave; job < NQT * NDT; job += NW) {
            const int qt = job % NQT, dt = job / NQT;
            f4 acc = f4zero();
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const f4 a = *reinterpret_cast<const f4*>(&dSs[(16 * qt + l16) * TS + 16 * kt + 4 * g]);
                const f4 bb = *reinterpret_cast<const f4*>(&Kt[(16 * dt + l16) * TS + 16 * kt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(a[r], bb[r], acc);
            }
            const int d = 16 * dt + l16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int q = q0 + 16 * qt + 4 * g + r;
                if (q < S && d < Dh)
                    atomic_add_f32(dQ + base + (long)q * rs + d, acc[r] * scale);
            }
        }
    };

    const int qb0 = k0 / BM;
    load_q(qb0 * BM);
    if constexpr (SM::DB) {
        // Tile qb is in stage qb&1 when iteration qb starts.  Iteration qb
        // writes tile qb+1 into the other stage (last read in iteration qb-1,
        // before its barrier) and dS into its own stage, which the dQ jobs
        // read after the barrier.
        store_q(stage(qb0 & 1));
        if (qb0 + 1 < nqb)
            load_q((qb0 + 1) * BM);
        __syncthreads();
        for (int qb = qb0; qb < nqb; qb++) {
            const int q0 = qb * BM;
            float* cur = stage(qb & 1);
            if (qb + 1 < nqb) {
                store_q(stage((qb + 1) & 1));
                if (qb + 2 < nqb)
                    load_q(q0 + 2 * BM);
            }
            key_side(cur, q0);
            __syncthreads();
            query_side(cur, q0);
        }
    } else {
        constexpr bool PREFETCH = DHP <= 128;
        float* st = stage(0);
        for (int qb = qb0; qb < nqb; qb++) {
            const int q0 = qb * BM;
            if (!PREFETCH && qb > qb0)
                load_q(q0);
            __syncthreads();
            store_q(st);
            __syncthreads();
            if (PREFETCH && qb + 1 < nqb)
                load_q(q0 + BM);
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
