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
// Work decomposition (one workgroup = 4 waves = 256 threads):
//   forward : a workgroup owns 64 query rows of one (b,h); wave w owns rows
//             16w..16w+15.  Scores are computed transposed (S^T = K Q^T) so
//             lane l holds query l%16 and the softmax statistics are per lane.
//   backward: a workgroup owns 64 key rows of one (b,h); wave w owns keys
//             16w..16w+15 with K/V held in registers, accumulates dK^T/dV^T in
//             registers over all later query tiles, and adds its dQ tile into
//             the zero-initialised dQ with float atomics.
// The flat grid index is (tile * B*H + bh): heavy causal tiles dispatch first,
// and when B*H is a multiple of 8 all tiles of a head share an XCD (and its
// L2), since workgroups are dealt to the 8 XCDs round-robin.
#include "common.hpp"
#include "launch.hpp"

#include <math.h>

namespace cxg {

constexpr int MHA_BM = 64;   // query rows per tile
constexpr int MHA_BN = 64;   // key rows per tile
constexpr int MHA_THREADS = 256;

// ----------------------------------------------------------------------------
// forward (and statistics-only) kernel
// ----------------------------------------------------------------------------
template <int DHP, bool VEC, bool WRITE_O>
__global__ __launch_bounds__(MHA_THREADS) void mha_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int S, int H, int Dh, int BH, int nqb,
    float qscale)
{
    constexpr int KS = DHP + 4;       // Ks[key][d] row stride (floats)
    constexpr int VS = MHA_BN + 4;    // Vt[d][key] row stride
    constexpr int NDT = DHP / 16;
    constexpr int NU = MHA_BN * (DHP / 4);   // float4 units per tile
    __shared__ __attribute__((aligned(16))) float Ks[MHA_BN * KS];
    __shared__ __attribute__((aligned(16))) float Vt[WRITE_O ? DHP * VS : 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int qi = blockIdx.x / BH, bh = blockIdx.x - qi * BH;
    const int qb = nqb - 1 - qi;
    const int b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;

    const int myq = qb * MHA_BM + wave * 16 + l16;
    const bool qok = myq < S;
    // B operand of S^T = K Q^T: lane holds Q[myq][16*dt + 4*g + r], pre-scaled
    // by scale*log2(e) so scores land in the exp2 domain.
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
    for (int kb = 0; kb < nkb; kb++) {
        const int k0 = kb * MHA_BN;
        __syncthreads();
        for (int u = tid; u < NU; u += MHA_THREADS) {
            const int row = u / (DHP / 4), c = 4 * (u - row * (DHP / 4));
            const int key = k0 + row;
            const bool ok = key < S;
            const long off = base + (long)(ok ? key : 0) * rs;
            *reinterpret_cast<f4*>(&Ks[row * KS + c]) = load4<VEC>(K + off, c, Dh, ok);
            if (WRITE_O) {
                f4 vv = load4<VEC>(V + off, c, Dh, ok);
                Vt[(c + 0) * VS + row] = vv[0];
                Vt[(c + 1) * VS + row] = vv[1];
                Vt[(c + 2) * VS + row] = vv[2];
                Vt[(c + 3) * VS + row] = vv[3];
            }
        }
        __syncthreads();

        // S^T tile: lane holds query l16, keys k0 + 16*kt + 4*g + r.
        f4 sacc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f4 acc = f4zero();
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const f4 kv = *reinterpret_cast<const f4*>(&Ks[(16 * kt + l16) * KS + 16 * dt + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc = mfma16(kv[r], qreg[dt][r], acc);
            }
            sacc[kt] = acc;
        }
        if (kb == qb) {   // diagonal tile: causal mask key > query
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (k0 + 16 * kt + 4 * g + r > myq)
                        sacc[kt][r] = -INFINITY;
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                mloc = fmaxf(mloc, sacc[kt][r]);
        mloc = xrow_max(mloc);
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = fast_exp2(m_run - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = fast_exp2(sacc[kt][r] - m_new);
                sacc[kt][r] = p;
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
                for (int kt = 0; kt < 4; kt++) {
                    const f4 vv = *reinterpret_cast<const f4*>(&Vt[(16 * dt + l16) * VS + 16 * kt + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc = mfma16(vv[r], sacc[kt][r], acc);
                }
                oacc[dt] = acc;
            }
        }
    }
    const float l_tot = xrow_sum(l_run);
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
// backward main kernel.  BM query rows per inner tile (64, or 32 for the
// widest heads so the LDS tiles fit in 160 KB).
// ----------------------------------------------------------------------------
template <int DHP, int BM, bool VEC>
__global__ __launch_bounds__(MHA_THREADS) void mha_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int S, int H, int Dh,
    int BH, int nkb, float scale, float c2)
{
    constexpr int NDT = DHP / 16;
    constexpr int NQT = BM / 16;
    constexpr int QS = DHP + 4;        // Qs/dOs [q][d] row stride
    constexpr int TS = MHA_BN + 4;     // Kt [d][key] and dSs [q][key] row stride
    constexpr int NU = BM * (DHP / 4);
    __shared__ __attribute__((aligned(16))) float Qs[BM * QS];
    __shared__ __attribute__((aligned(16))) float dOs[BM * QS];
    __shared__ __attribute__((aligned(16))) float Kt[DHP * TS];
    __shared__ __attribute__((aligned(16))) float dSs[BM * TS];
    __shared__ __attribute__((aligned(16))) float lse_s[BM];
    __shared__ __attribute__((aligned(16))) float di_s[BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int kb = blockIdx.x / BH, bh = blockIdx.x - kb * BH;
    const int b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;
    const int k0 = kb * MHA_BN;
    const int mykey = k0 + wave * 16 + l16;
    const bool kok = mykey < S;

    // B operands for S = Q K^T and dP = dO V^T: K/V[mykey][16dt + 4g + r].
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
    for (int u = tid; u < MHA_BN * (DHP / 4); u += MHA_THREADS) {
        const int row = u / (DHP / 4), c = 4 * (u - row * (DHP / 4));
        const int key = k0 + row;
        const bool ok = key < S;
        const f4 kv = load4<VEC>(K + base + (long)(ok ? key : 0) * rs, c, Dh, ok);
        Kt[(c + 0) * TS + row] = kv[0];
        Kt[(c + 1) * TS + row] = kv[1];
        Kt[(c + 2) * TS + row] = kv[2];
        Kt[(c + 3) * TS + row] = kv[3];
    }

    f4 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        dk[dt] = f4zero();
        dv[dt] = f4zero();
    }

    const int nqb = (S + BM - 1) / BM;
    for (int qb = (k0 / BM); qb < nqb; qb++) {
        const int q0 = qb * BM;
        __syncthreads();
        for (int u = tid; u < NU; u += MHA_THREADS) {
            const int row = u / (DHP / 4), c = 4 * (u - row * (DHP / 4));
            const int q = q0 + row;
            const bool ok = q < S;
            const long off = base + (long)(ok ? q : 0) * rs;
            *reinterpret_cast<f4*>(&Qs[row * QS + c]) = load4<VEC>(Q + off, c, Dh, ok);
            *reinterpret_cast<f4*>(&dOs[row * QS + c]) = load4<VEC>(dO + off, c, Dh, ok);
        }
        if (tid < BM) {
            const int q = q0 + tid;
            const bool ok = q < S;
            lse_s[tid] = ok ? lse[(long)bh * S + q] * kLog2e : INFINITY;
            di_s[tid] = ok ? Di[(long)bh * S + q] : 0.0f;
        }
        __syncthreads();

        // S = Q K^T and dP = dO V^T: lane holds key l16, queries 16qt + 4g + r.
        const bool diag = q0 < k0 + MHA_BN;   // tile touches the causal boundary
        f4 P[NQT], dS[NQT];
#pragma unroll
        for (int qt = 0; qt < NQT; qt++) {
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
                const bool ok = !diag || (mykey <= q);
                const float p = ok ? fast_exp2(sa[r] * c2 - l4[r]) : 0.0f;
                P[qt][r] = p;
                dS[qt][r] = p * (da[r] - d4[r]);
                dSs[(16 * qt + 4 * g + r) * TS + wave * 16 + l16] = dS[qt][r];
            }
        }
        // dV^T += dO^T P and dK^T += Q^T dS (contraction over the BM queries).
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            f4 av = dv[dt], ak = dk[dt];
#pragma unroll
            for (int qt = 0; qt < NQT; qt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = (16 * qt + 4 * g + r) * QS + 16 * dt + l16;
                    av = mfma16(dOs[row], P[qt][r], av);
                    ak = mfma16(Qs[row], dS[qt][r], ak);
                }
            dv[dt] = av;
            dk[dt] = ak;
        }
        __syncthreads();
        // dQ tiles (qt, dt) of this query block, dealt round-robin to the waves:
        // dS (LDS) x K (LDS, transposed), added into dQ with float atomics.
        for (int job = wave; job < NQT * NDT; job += MHA_THREADS / 64) {
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

template <int DHP, bool VEC>
static hipError_t fwd_dispatch2(const float* Q, const float* K, const float* V, float* O,
                                float* lse, int B, int S, int H, int Dh, hipStream_t st)
{
    const int BH = B * H;
    const int nqb = (S + MHA_BM - 1) / MHA_BM;
    const float qscale = (1.0f / sqrtf((float)Dh)) * kLog2e;
    dim3 grid((unsigned)(nqb * BH)), block(MHA_THREADS);
    if (O != nullptr) {
        ProfScope ps(st, "mha_fwd");
        hipLaunchKernelGGL((mha_fwd_kernel<DHP, VEC, true>), grid, block, 0, st, Q, K, V, O, lse,
                           S, H, Dh, BH, nqb, qscale);
    } else {
        ProfScope ps(st, "mha_stats");
        hipLaunchKernelGGL((mha_fwd_kernel<DHP, VEC, false>), grid, block, 0, st, Q, K, V, O,
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

template <int DHP, int BM>
static hipError_t bwd_dispatch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st)
{
    const int BH = B * H;
    const int nkb = (S + MHA_BN - 1) / MHA_BN;
    const float scale = 1.0f / sqrtf((float)Dh);
    dim3 grid((unsigned)(nkb * BH)), block(MHA_THREADS);
    const bool vec = (Dh % 4 == 0) && aligned16(Q) && aligned16(K) && aligned16(V) &&
                     aligned16(dO) && aligned16(dK) && aligned16(dV);
    ProfScope ps(st, "mha_bwd");
    if (vec)
        hipLaunchKernelGGL((mha_bwd_kernel<DHP, BM, true>), grid, block, 0, st, Q, K, V, dO, lse, Di,
                           dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e);
    else
        hipLaunchKernelGGL((mha_bwd_kernel<DHP, BM, false>), grid, block, 0, st, Q, K, V, dO, lse,
                           Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e);
    return hipGetLastError();
}

hipError_t mha_bwd_main_launch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st)
{
    if (Dh <= 16)
        return bwd_dispatch<16, 64>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 32)
        return bwd_dispatch<32, 64>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 64)
        return bwd_dispatch<64, 64>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    if (Dh <= 128)
        return bwd_dispatch<128, 64>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
    return bwd_dispatch<256, 32>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st);
}

} // namespace cxg
