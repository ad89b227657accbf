// mhanarrow.hip -- causal softmax MHA for narrow heads on short sequences
// (gfx950, FP32 MFMA).
//
// Serves the same calls as mha.hip (two_stage_cuda::fused_mha_fwd /
// fused_mha_bwd, src/TwoStage/two_stage_cuda_kernels.cu:285-326, :830-882)
// for heads of at most 16 columns whose rows fit in LDS (S_pad * DHP <= 4096,
// DHP = 8 for Dh <= 8, else 16): TwoStageGPT's stage 1 runs H = 64 heads of
// Dh = 8 at S = 256 (two_stage_train.cpp:168-170).  At that width the 64-row
// tile kernels spend most of their time outside the products: per-tile
// staging, barriers, online-softmax bookkeeping and job start-up for 1-4
// tiles of 8-column work.  Here one workgroup of 4 waves takes a whole
// (b, h) head:
//   forward : K and V^T of the head are staged in LDS once; wave w takes the
//             16-row query blocks of pairs (nb-1-p, p), p = w, w+4, ... (each
//             pair costs nb+1 key blocks), with S^T = K Q^T on MFMA (a lane
//             holds one query, so a row's statistics need one cross-row max)
//             and O += P V.  The softmax reference is lazy: key block 0's
//             exact maximum first, then the score accumulators start at -m
//             (scores relative to m), and m moves only when a score passes it
//             by 2^8 (a wave-uniform check per chunk of 4 key blocks).
//   backward: Q (pre-scaled), dO (both transposed) and K of the head live in
//             LDS; every row's Di = dO.O is formed at the start, and for the
//             reference's signature (no lse) the statistics are recomputed by
//             the same waves first.  -lse and -Di start the S and dP
//             accumulators.  Wave w then takes key blocks of pairs
//             (p, nb-1-p): S and dP in the key-column layout (a lane holds one
//             key, four queries), dV += P^T dO and dK += dS^T Q in registers,
//             dS transposed through a per-wave LDS tile for dQ^T = K^T dS^T,
//             whose per-query-block partials stay in the wave's registers
//             until the four waves add theirs through LDS at the end.  dQ
//             leaves once: no atomics, no zeroing pass, no scratch.
// The fused RoPE calls (cxg_mha_rope_fwd/bwd, two_stage_gpt.hpp:102-106,
// :171-174) take the same kernels: Q and K rows are rotated as they are read
// or staged, dQ and dK rotated back as they are written.
// Products run on FP32 MFMA: the score contractions (S, dP) as 16x16x4 over
// DHP/4 steps, dQ, dV and dK as 16x16x4 with the head columns padded to 16
// (4x4x1 blocks for dV and dK measured no faster: their registers cost a wave
// per SIMD), O as 4x4x1 blocks over 4-column groups of the head.
#include "common.hpp"
#include "launch.hpp"

#include <math.h>

namespace cxg {

constexpr int NAR_THREADS = 256;   // 4 waves, one workgroup per head
constexpr int NAR_MAX_ELEMS = 4096;   // S_pad * DHP of one staged head tensor
constexpr int NAR_TLD = 20;          // row stride of the backward's transpose tiles

typedef float f2 __attribute__((ext_vector_type(2)));

// Workgroup b -> head.  Workgroups are dealt to the 8 XCDs round-robin
// (b % 8); when BH is a multiple of 8, XCD x takes heads x*BH/8 ... in order,
// so heads h and h+1, whose rows share cache lines, are read through one L2.
__device__ __forceinline__ int nar_head(int b, int BH)
{
    return (BH & 7) != 0 ? b : (b & 7) * (BH >> 3) + (b >> 3);
}

// KW consecutive floats d0 .. d0+KW-1 of a row (columns >= Dh and rows not
// ok read 0).  VEC: the row base is 16-byte aligned and Dh % 4 == 0.
template <int KW, bool VEC>
__device__ __forceinline__ void ld_kw(float (&o)[KW], const float* __restrict__ rowp, bool ok,
                                      int d0, int Dh)
{
    if (VEC && ok && d0 + KW <= Dh) {
        if constexpr (KW == 4) {
            const f4 v = *reinterpret_cast<const f4*>(rowp + d0);
#pragma unroll
            for (int s = 0; s < 4; s++)
                o[s] = v[s];
        } else {
            const f2 v = *reinterpret_cast<const f2*>(rowp + d0);
            o[0] = v[0];
            o[1] = v[1];
        }
    } else {
#pragma unroll
        for (int s = 0; s < KW; s++)
            o[s] = (ok && d0 + s < Dh) ? rowp[d0 + s] : 0.0f;
    }
}

// 4 columns c .. c+3 of a row, zero past Dh or when !ok.
template <bool VEC>
__device__ __forceinline__ f4 ld_c4(const float* __restrict__ rowp, bool ok, int c, int Dh)
{
    if (VEC) {
        return (ok && c < Dh) ? *reinterpret_cast<const f4*>(rowp + c) : f4zero();
    } else {
        f4 v;
#pragma unroll
        for (int i = 0; i < 4; i++)
            v[i] = (ok && c + i < Dh) ? rowp[c + i] : 0.0f;
        return v;
    }
}

template <int KW>
__device__ __forceinline__ void lds_kw(float (&o)[KW], const float* p)
{
    if constexpr (KW == 4) {
        const f4 v = *reinterpret_cast<const f4*>(p);
#pragma unroll
        for (int s = 0; s < 4; s++)
            o[s] = v[s];
    } else {
        const f2 v = *reinterpret_cast<const f2*>(p);
        o[0] = v[0];
        o[1] = v[1];
    }
}

// RoPE (the fused entry points): the head's rotary frequencies, w[i] for the
// pairs (2i, 2i+1) of at most 16 columns, copied into LDS by one lane with
// uniform indices (scalar reads of the kernel argument); the caller
// synchronises.
template <bool ROPE>
__device__ __forceinline__ void nar_rope_table(float* rw, const MhaRope& rp)
{
    if (ROPE && threadIdx.x == 0)
#pragma unroll
        for (int i = 0; i < 8; i++)
            rw[i] = rp.w[i];
}

// Rotation of the pair (a, b) at position pos by sign * pos * w.
__device__ __forceinline__ void rope2(float& a, float& b, int pos, float w, float sign)
{
    float sn, cs;
    sincos_rev(sign * (float)pos * w, &sn, &cs);
    const float x = a;
    a = x * cs - b * sn;
    b = x * sn + b * cs;
}

// The KW columns d0 .. d0+KW-1 (d0 even) of a row at position pos, rotated.
template <int KW>
__device__ __forceinline__ void rope_kw(float (&o)[KW], int pos, int d0, const float* rw)
{
#pragma unroll
    for (int s = 0; s < KW; s += 2)
        rope2(o[s], o[s + 1], pos, rw[(d0 + s) >> 1], 1.0f);
}

constexpr int NAR_CH = 4;   // forward: key blocks per score chunk
// The softmax reference moves when a score passes it by more than this (log2
// units): probabilities stay below 2^8, so no sum can overflow.
constexpr float kNarHead = 8.0f;
constexpr int NAR_CH_STATS = 8;   // the backward's statistics (its registers are shared with dQ)

// S^T block (i, j) from Ks ([SP][DHP] rows) and the query operand qo (query
// l16, columns KW g + s, pre-scaled to log2 units), added to a: lane (l16, g)
// element r is key 16j + 4g + r.  DIAG (j == i): the keys after the lane's
// query -inf.
template <int DHP, bool DIAG>
__device__ __forceinline__ f4 nar_score(const float* Ks, const float (&qo)[DHP / 4], int j,
                                        int l16, int g, f4 a)
{
    constexpr int KW = DHP / 4;
    float ka[KW];
    lds_kw<KW>(ka, &Ks[(16 * j + l16) * DHP + KW * g]);
#pragma unroll
    for (int s = 0; s < KW; s++)
        a = mfma16(ka[s], qo[s], a);   // S^T[key 4g+r][query l16]
    if (DIAG) {
#pragma unroll
        for (int r = 0; r < 4; r++)
            a[r] = (4 * g + r <= l16) ? a[r] : -INFINITY;
    }
    return a;
}

// max(a, b) of non-NaN values as one v_med3_f32 (the median of a, b and +inf).
// fmaxf also quiets signalling NaNs: a v_max_f32 x, x per operand the compiler
// cannot prove quiet, i.e. per MFMA result.
__device__ __forceinline__ float fmax_nn(float a, float b)
{
    // +inf from an opaque scalar move, so that the compiler keeps the median
    // (with a constant +inf it folds it back into fmaxf)
    float inf;
    asm("s_mov_b32 %0, 0x7f800000" : "=s"(inf));
    return __builtin_amdgcn_fmed3f(a, b, inf);
}

__device__ __forceinline__ float max4(f4 a) { return fmax_nn(fmax_nn(a[0], a[1]), fmax_nn(a[2], a[3])); }

// Maximum over the four lanes l16 + 16g that share a query.
__device__ __forceinline__ float nar_xrow_max(float v)
{
    v = fmax_nn(v, __shfl_xor(v, 16, 64));
    return fmax_nn(v, __shfl_xor(v, 32, 64));
}

// 4x4x1 FP32 MFMA, 16 independent 4x4 blocks (2 passes, the 16x16x4 form's
// rate): result lane l, register m = A[lane 4(l/4) + m] * B[lane l] summed
// over the calls.  The forward's O products use it with the head side in
// 4-column groups, so a narrow head is not padded to 16 columns; lanes of
// different g (l / 16) then hold sums over different keys, added across g
// once at the end.
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// Column group g of the sum over the four lanes l16 + 16g of a[0 .. KW-1]
// (valid in lanes g < KW): lanes g and g^1 keep the groups whose bit 0 is
// g & 1 and add the partner's copies, then lanes g and g^2 those whose bit 1
// is g >> 1 (KW = 4; with KW = 2 the second step only adds).
template <int KW>
__device__ __forceinline__ f4 nar_colsum(const f4 (&a)[KW], int g)
{
    const bool b0 = (g & 1) != 0;
    if constexpr (KW == 2) {
        f4 keep = b0 ? a[1] : a[0];
        const f4 send = b0 ? a[0] : a[1];
#pragma unroll
        for (int r = 0; r < 4; r++)
            keep[r] += __shfl_xor(send[r], 16, 64);
#pragma unroll
        for (int r = 0; r < 4; r++)
            keep[r] += __shfl_xor(keep[r], 32, 64);
        return keep;
    } else {
        f4 k0 = b0 ? a[1] : a[0], k1 = b0 ? a[3] : a[2];
        const f4 s0 = b0 ? a[0] : a[1], s1 = b0 ? a[2] : a[3];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            k0[r] += __shfl_xor(s0[r], 16, 64);
            k1[r] += __shfl_xor(s1[r], 16, 64);
        }
        const bool b1 = (g & 2) != 0;
        f4 keep = b1 ? k1 : k0;
        const f4 send = b1 ? k0 : k1;
#pragma unroll
        for (int r = 0; r < 4; r++)
            keep[r] += __shfl_xor(send[r], 32, 64);
        return keep;
    }
}

// ---------------------------------------------------------------------------
// forward: O (WRITE_O) and lse.
// ---------------------------------------------------------------------------
// Waves per SIMD the forward is compiled for (16-column heads hold four O
// accumulators a lane).
constexpr int nar_fwd_waves(int dhp) { return dhp > 8 ? 4 : 6; }

template <int DHP, bool VEC, bool WRITE_O, bool ROPE>
__global__ __launch_bounds__(NAR_THREADS) __attribute__((amdgpu_waves_per_eu(nar_fwd_waves(DHP))))
void mha_nar_fwd_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                   const float* __restrict__ V, float* __restrict__ O, float* __restrict__ lse,
                   int S, int H, int Dh, int BH, float qscale, const MhaRope rope)
{
    extern __shared__ __attribute__((aligned(16))) float nar_lds[];
    __shared__ float rw[ROPE ? 8 : 1];   // RoPE: Q and K rotated as they are read
    nar_rope_table<ROPE>(rw, rope);
    if (ROPE)
        __syncthreads();
    constexpr int KW = DHP / 4;   // score k-slots per lane (d = KW g + s); 4-column groups of d
    const int nb = (S + 15) >> 4, SP = nb * 16, VLD = SP + 4;
    float* Ks = nar_lds;             // [SP][DHP]
    float* Vt = nar_lds + SP * DHP;  // [DHP][VLD]: V^T
    const int bh = nar_head((int)blockIdx.x, BH), b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;
    const int tid = threadIdx.x;

    for (int u = tid; u < SP * KW; u += NAR_THREADS) {
        const int row = u / KW, c = 4 * (u - row * KW);
        const bool ok = row < S;
        const long ro = base + (long)min(row, S - 1) * rs;
        f4 k4 = ld_c4<VEC>(K + ro, ok, c, Dh);
        const f4 v4 = ld_c4<VEC>(V + ro, ok, c, Dh);
        if (ROPE)
            k4 = rope4(k4, row, c, rw, 1.0f);
        *reinterpret_cast<f4*>(&Ks[row * DHP + c]) = k4;
#pragma unroll
        for (int i = 0; i < 4; i++)
            Vt[(c + i) * VLD + row] = v4[i];
    }
    __syncthreads();

    const int lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
    const int npair = (nb + 1) >> 1;
    const float* vrow = &Vt[(l16 & 3) * VLD + 4 * g];   // this lane's V^T operand row, group 0
    auto qblock = [&](int i, float (&qo)[KW]) __attribute__((always_inline)) {
            const int qrow = 16 * i + l16;
            const bool qok = qrow < S;
            if (ROPE)
                rope_kw<KW>(qo, qrow, KW * g, rw);
#pragma unroll
            for (int s = 0; s < KW; s++)
                qo[s] *= qscale;
            // Online softmax with a lazy reference m (log2 units, the same in
            // the four lanes of a query): block 0's exact maximum first (key 0
            // is visible to every query, so it is finite), then every score
            // accumulator starts at -m, so scores come out relative to m; m
            // moves only when a score of the wave passes it by more than
            // kNarHead, so the probabilities stay below 2^kNarHead and most
            // blocks need no subtraction, no cross-lane maximum and no
            // rescale.  O accumulates as oacc[c]: O[query l16][4c + m] over
            // keys 4g .. 4g+3 of each block.
            f4 oacc[KW];
#pragma unroll
            for (int c = 0; c < KW; c++)
                oacc[c] = f4zero();
            float lsum = 0.0f;
            auto pv = [&](const f4& sv, int j) __attribute__((always_inline)) {
                f4 pr;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    pr[r] = fast_exp2(sv[r]);
                lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);
                if (WRITE_O) {
#pragma unroll
                    for (int c = 0; c < KW; c++) {
                        // A: V[key 16j + 4g + r][4c + (lane & 3)], B: P[query l16][that key]
                        const f4 va = *reinterpret_cast<const f4*>(vrow + 4 * c * VLD + 16 * j);
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            oacc[c] = mfma4(va[r], pr[r], oacc[c]);
                    }
                }
            };
            f4 s0 = i == 0 ? nar_score<DHP, true>(Ks, qo, 0, l16, g, f4zero())
                           : nar_score<DHP, false>(Ks, qo, 0, l16, g, f4zero());
            float m = nar_xrow_max(max4(s0));
            s0 -= m;
            f4 nm = f4zero() - m;
            pv(s0, 0);
            // raise m by d >= 0 (per query) when a relative score of the wave
            // passes kNarHead; the scores in hand move with it
            auto raise = [&](float bm, f4* sv, int n) __attribute__((always_inline)) {
                if (__builtin_amdgcn_ballot_w64(bm > kNarHead) != 0) {   // wave-uniform
                    const float d = fmax_nn(nar_xrow_max(bm), 0.0f);
                    const float f = fast_exp2(-d);
#pragma unroll
                    for (int c = 0; c < KW; c++)
                        oacc[c] *= f;
                    lsum *= f;
                    m += d;
                    nm = f4zero() - m;
                    for (int J = 0; J < n; J++)
                        sv[J] -= d;
                }
            };
            // whole chunks of NAR_CH blocks below the diagonal (straight-line:
            // every score first, one reference check), then single blocks,
            // then the diagonal block with the causal mask
            int j = 1;
            for (; j + NAR_CH <= i; j += NAR_CH) {
                f4 sc[NAR_CH];
                float cm = -INFINITY;
#pragma unroll
                for (int J = 0; J < NAR_CH; J++) {
                    sc[J] = nar_score<DHP, false>(Ks, qo, j + J, l16, g, nm);
                    cm = fmax_nn(cm, max4(sc[J]));
                }
                raise(cm, sc, NAR_CH);
#pragma unroll
                for (int J = 0; J < NAR_CH; J++)
                    pv(sc[J], j + J);
            }
            for (; j < i; j++) {
                f4 sv = nar_score<DHP, false>(Ks, qo, j, l16, g, nm);
                raise(max4(sv), &sv, 1);
                pv(sv, j);
            }
            if (i > 0) {
                f4 sv = nar_score<DHP, true>(Ks, qo, i, l16, g, nm);
                raise(max4(sv), &sv, 1);
                pv(sv, i);
            }
            const float l = xrow_sum(lsum);
            if (WRITE_O) {
                // every key's share: sum over g, as a reduce-scatter (lanes
                // g and g^1 trade half their column groups, then g and g^2),
                // so that lane (l16, g < KW) ends with column group g
                f4 o = nar_colsum<KW>(oacc, g);
                if (qok && g < KW) {
                    o *= __builtin_amdgcn_rcpf(l);   // hardware reciprocal, within 1 ulp
                    float* orow = O + base + (long)qrow * rs;
                    if (VEC && 4 * g + 3 < Dh) {
                        *reinterpret_cast<f4*>(orow + 4 * g) = o;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            if (4 * g + r < Dh)
                                orow[4 * g + r] = o[r];
                    }
                }
            }
            if (lse != nullptr && qok && g == 0)
                lse[(long)bh * S + qrow] = (m + fast_log2(l)) * kLn2;
    };
    for (int p = w; p < npair; p += 4) {
#pragma unroll 1
        for (int hf = 0; hf < 2; hf++) {
            const int i = hf == 0 ? nb - 1 - p : p;
            if (hf == 1 && i == nb - 1 - p)
                break;   // the middle block of an odd count
            float qo[KW];
            const int qrow = 16 * i + l16;
            ld_kw<KW, VEC>(qo, Q + base + (long)min(qrow, S - 1) * rs, qrow < S, KW * g, Dh);
            qblock(i, qo);
        }
    }
}

// ---------------------------------------------------------------------------
// backward: dQ, dK, dV (STATS: no lse given, the statistics are recomputed).
// NBM >= nb: the query blocks' dQ partials of a wave live in registers
// (dqp[I], NBM of them, indexed at compile time), summed over the wave's key
// blocks by the dQ products themselves; the four waves' partials are added
// through LDS once, at the end.  (LDS float atomics per block, the first
// form, made the stage-1 backward 256 us against 150 us without them.)
// ---------------------------------------------------------------------------
// Waves per SIMD the backward is compiled for: the register partials of dQ
// take 4 NBM registers, so 32 blocks (S > 256) leave room for two waves.
constexpr int nar_bwd_waves(int dhp, int nbm) { return nbm > 16 ? 2 : dhp > 8 ? 3 : 4; }

template <int DHP, bool VEC, bool STATS, int NBM, bool ROPE>
__global__ __launch_bounds__(NAR_THREADS)
__attribute__((amdgpu_waves_per_eu(nar_bwd_waves(DHP, NBM)))) void mha_nar_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ lse,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int S, int H, int Dh,
    int BH, float qscale, float scale, const MhaRope rope)
{
    extern __shared__ __attribute__((aligned(16))) float nar_lds[];
    // RoPE: Q and K rotated as they are staged, dQ and dK rotated back as
    // they are written
    __shared__ float rw[ROPE ? 8 : 1];
    nar_rope_table<ROPE>(rw, rope);
    if (ROPE)
        __syncthreads();
    constexpr int KW = DHP / 4;
    const int nb = (S + 15) >> 4, SP = nb * 16;
    // Q (pre-scaled) and dO transposed, [d][query] with row stride QLD, and a
    // zero row d = DHP that lanes past the head's columns read; both regions
    // hold a dQ partial sum ([SP][DHP]) at the end
    const int QLD = SP + 4;
    float* Qt = nar_lds;                  // [DHP + 1][QLD]
    float* dOt = Qt + (DHP + 1) * QLD;    // [DHP + 1][QLD]
    float* Ks = dOt + (DHP + 1) * QLD;    // [SP][DHP]
    // negated, so that they start the S and dP accumulators: S - lse and
    // dP - Di come out of the MFMAs
    float* L2 = Ks + SP * DHP;            // [SP] -lse * log2(e); -inf past S
    float* Dd = L2 + SP;              // [SP] -Di
    float* T = Dd + SP;               // [4][16][NAR_TLD] transpose tiles
    const int bh = nar_head((int)blockIdx.x, BH), b = bh / H, h = bh - b * H;
    const long rs = (long)H * Dh;
    const long base = (long)b * S * rs + (long)h * Dh;
    const int tid = threadIdx.x;

    for (int u = tid; u < SP * KW; u += NAR_THREADS) {
        const int row = u / KW, c = 4 * (u - row * KW);
        const bool ok = row < S;
        const long ro = base + (long)min(row, S - 1) * rs;
        f4 q4 = ld_c4<VEC>(Q + ro, ok, c, Dh);
        if (ROPE)
            q4 = rope4(q4, row, c, rw, 1.0f);
        q4 *= qscale;
        const f4 o4 = ld_c4<VEC>(dO + ro, ok, c, Dh);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            Qt[(c + i) * QLD + row] = q4[i];
            dOt[(c + i) * QLD + row] = o4[i];
        }
        f4 k4 = ld_c4<VEC>(K + ro, ok, c, Dh);
        if (ROPE)
            k4 = rope4(k4, row, c, rw, 1.0f);
        *reinterpret_cast<f4*>(&Ks[row * DHP + c]) = k4;
    }
    for (int col = tid; col < SP; col += NAR_THREADS) {
        Qt[DHP * QLD + col] = 0.0f;
        dOt[DHP * QLD + col] = 0.0f;
    }
    for (int row = tid; row < SP; row += NAR_THREADS) {
        float di = 0.0f;
        if (row < S) {
            const float* orow = O + base + (long)row * rs;
            const float* grow = dO + base + (long)row * rs;
            for (int c = 0; c < Dh; c += 4) {
                const f4 o4 = ld_c4<VEC>(orow, true, c, Dh), g4 = ld_c4<VEC>(grow, true, c, Dh);
                di += (o4[0] * g4[0] + o4[1] * g4[1]) + (o4[2] * g4[2] + o4[3] * g4[3]);
            }
        }
        Dd[row] = -di;
        if (!STATS)
            L2[row] = row < S ? -lse[(long)bh * S + row] * kLog2e : -INFINITY;
    }
    __syncthreads();

    const int lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
    const int npair = (nb + 1) >> 1;
    if (STATS) {
        // the forward's statistics (S^T layout, a lane per query) for the
        // query blocks of pairs (nb-1-p, p)
        for (int p = w; p < npair; p += 4) {
#pragma unroll 1
            for (int hf = 0; hf < 2; hf++) {
                const int i = hf == 0 ? nb - 1 - p : p;
                if (hf == 1 && i == nb - 1 - p)
                    break;
                float qo[KW];
#pragma unroll
                for (int s = 0; s < KW; s++)
                    qo[s] = Qt[(KW * g + s) * QLD + 16 * i + l16];
                // lazy reference, as in the forward
                f4 s0 = i == 0 ? nar_score<DHP, true>(Ks, qo, 0, l16, g, f4zero())
                               : nar_score<DHP, false>(Ks, qo, 0, l16, g, f4zero());
                float m = nar_xrow_max(max4(s0));
                s0 -= m;
                f4 nm = f4zero() - m;
                float lsum = (fast_exp2(s0[0]) + fast_exp2(s0[1])) +
                             (fast_exp2(s0[2]) + fast_exp2(s0[3]));
                auto take = [&](f4* sv, int n, float bm) __attribute__((always_inline)) {
                    if (__builtin_amdgcn_ballot_w64(bm > kNarHead) != 0) {   // wave-uniform
                        const float d = fmax_nn(nar_xrow_max(bm), 0.0f);
                        lsum *= fast_exp2(-d);
                        m += d;
                        nm = f4zero() - m;
                        for (int J = 0; J < n; J++)
                            sv[J] -= d;
                    }
                    for (int J = 0; J < n; J++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            lsum += fast_exp2(sv[J][r]);
                };
                int j = 1;
                for (; j + NAR_CH_STATS <= i; j += NAR_CH_STATS) {
                    f4 sc[NAR_CH_STATS];
                    float cm = -INFINITY;
#pragma unroll
                    for (int J = 0; J < NAR_CH_STATS; J++) {
                        sc[J] = nar_score<DHP, false>(Ks, qo, j + J, l16, g, nm);
                        cm = fmax_nn(cm, max4(sc[J]));
                    }
                    take(sc, NAR_CH_STATS, cm);
                }
                for (; j < i; j++) {
                    f4 sv = nar_score<DHP, false>(Ks, qo, j, l16, g, nm);
                    take(&sv, 1, max4(sv));
                }
                if (i > 0) {
                    f4 sv = nar_score<DHP, true>(Ks, qo, i, l16, g, nm);
                    take(&sv, 1, max4(sv));
                }
                const float l = xrow_sum(lsum);
                const int qrow = 16 * i + l16;
                if (g == 0)
                    L2[qrow] = qrow < S ? -(m + fast_log2(l)) : -INFINITY;
            }
        }
        __syncthreads();
    }

    float* Tw = T + w * 16 * NAR_TLD;
    const int trow = min(l16, DHP) * QLD + 4 * g;   // this lane's B operands in Qt, dOt
    f4 dqp[NBM];   // dQ^T partials: lane (query l16, g) columns 4g + r of block I
#pragma unroll
    for (int I = 0; I < NBM; I++)
        dqp[I] = f4zero();
    for (int p = w; p < npair; p += 4) {
#pragma unroll 1
        for (int hf = 0; hf < 2; hf++) {
            const int j = hf == 0 ? p : nb - 1 - p;
            if (hf == 1 && j == p)
                break;
            // key block j: K, V rows (B operands of S and dP: key l16, columns
            // KW g + s) and K^T (the A operand of dQ^T: K[4g + r][l16])
            const int krow = 16 * j + l16;
            float kb[KW], vb[KW];
            lds_kw<KW>(kb, &Ks[krow * DHP + KW * g]);
            ld_kw<KW, VEC>(vb, V + base + (long)min(krow, S - 1) * rs, krow < S, KW * g, Dh);
            float kt[4];
#pragma unroll
            for (int r = 0; r < 4; r++)
                kt[r] = l16 < DHP ? Ks[(16 * j + 4 * g + r) * DHP + min(l16, DHP - 1)] : 0.0f;
            f4 dk = f4zero(), dv = f4zero();
#pragma unroll
            for (int I = 0; I < NBM; I++) {
                if (I < j || I >= nb)
                    continue;   // wave-uniform
                float qa[KW], da[KW];
#pragma unroll
                for (int s = 0; s < KW; s++) {
                    qa[s] = Qt[(KW * g + s) * QLD + 16 * I + l16];
                    da[s] = dOt[(KW * g + s) * QLD + 16 * I + l16];
                }
                // S[query 4g+r][key l16] - lse and dP[query 4g+r][key l16] - Di
                f4 sc = *reinterpret_cast<const f4*>(&L2[16 * I + 4 * g]);
                f4 dp = *reinterpret_cast<const f4*>(&Dd[16 * I + 4 * g]);
#pragma unroll
                for (int s = 0; s < KW; s++) {
                    sc = mfma16(qa[s], kb[s], sc);
                    dp = mfma16(da[s], vb[s], dp);
                }
                f4 pr, ds;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float pv = fast_exp2(sc[r]);
                    if (I == j)
                        pv = (l16 <= 4 * g + r) ? pv : 0.0f;
                    pr[r] = pv;
                    ds[r] = pv * dp[r];
                }
                // dV[key][d] += sum_q P[q][key] dO[q][d], dK likewise with dS and
                // Q: the B operands dO[16I + 4g + r][d = l16] (zero row past DHP)
                const f4 dob = *reinterpret_cast<const f4*>(&dOt[trow + 16 * I]);
                const f4 qb = *reinterpret_cast<const f4*>(&Qt[trow + 16 * I]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    dv = mfma16(pr[r], dob[r], dv);
                    dk = mfma16(ds[r], qb[r], dk);
                }
                // dS^T through this wave's tile: Tw[q][key]
#pragma unroll
                for (int r = 0; r < 4; r++)
                    Tw[(4 * g + r) * NAR_TLD + l16] = ds[r];
                const f4 dst = *reinterpret_cast<const f4*>(&Tw[l16 * NAR_TLD + 4 * g]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    dqp[I] = mfma16(kt[r], dst[r], dqp[I]);   // dQ^T[d 4g+r][query l16]
            }
            // dK, dV rows of key block j: lane (d = l16, g) holds keys 4g + r
            // (RoPE: dK rotated back, the pair's other column from lane l16 ^ 1)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int kr = 16 * j + 4 * g + r;
                float kv = dk[r];
                if (ROPE) {
                    const float other = lane_xor16<1>(kv);
                    float sn, cs;
                    sincos_rev(-(float)kr * rw[min(l16, DHP - 1) >> 1], &sn, &cs);
                    kv = (l16 & 1) ? other * sn + kv * cs : kv * cs - other * sn;
                }
                if (kr < S && l16 < Dh) {
                    dK[base + (long)kr * rs + l16] = kv * kLn2;
                    dV[base + (long)kr * rs + l16] = dv[r];
                }
            }
        }
    }
    // the four waves' partials: waves 0, 1 store theirs over Qt, dOt (free
    // once every wave is past its products), then waves 2, 3 add theirs
    __syncthreads();
    float* part = (w & 1) ? dOt : Qt;
    if (w < 2 && g < KW) {
#pragma unroll
        for (int I = 0; I < NBM; I++)
            if (I < nb)
                *reinterpret_cast<f4*>(&part[(16 * I + l16) * DHP + 4 * g]) = dqp[I];
    }
    __syncthreads();
    if (w >= 2 && g < KW) {
#pragma unroll
        for (int I = 0; I < NBM; I++)
            if (I < nb) {
                f4* pp = reinterpret_cast<f4*>(&part[(16 * I + l16) * DHP + 4 * g]);
                *pp = *pp + dqp[I];
            }
    }
    __syncthreads();
    for (int u = tid; u < S * KW; u += NAR_THREADS) {
        const int row = u / KW, c = 4 * (u - row * KW);
        if (c >= Dh)
            continue;
        f4 v = (*reinterpret_cast<const f4*>(&Qt[row * DHP + c]) +
                *reinterpret_cast<const f4*>(&dOt[row * DHP + c])) *
               scale;
        if (ROPE)
            v = rope4(v, row, c, rw, -1.0f);
        float* qrow = dQ + base + (long)row * rs;
        if (VEC) {
            *reinterpret_cast<f4*>(qrow + c) = v;
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (c + i < Dh)
                    qrow[c + i] = v[i];
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static inline bool nar_al16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

static int nar_dhp(int Dh) { return Dh <= 8 ? 8 : 16; }

bool mha_nar_ok(int B, int S, int H, int Dh)
{
    if (B < 1 || S < 1 || H < 1 || Dh < 1 || Dh > 16)
        return false;
    const long sp = ((long)S + 15) / 16 * 16;
    return sp * nar_dhp(Dh) <= NAR_MAX_ELEMS && (long)B * H < (1L << 31) &&
           (long)S * H * Dh < (1L << 31);
}

template <int DHP, bool VEC>
static hipError_t nar_fwd_t(const float* Q, const float* K, const float* V, float* O, float* lse,
                            int B, int S, int H, int Dh, hipStream_t st, const MhaRope* rope)
{
    const int sp = (S + 15) / 16 * 16;
    const size_t lds = ((size_t)sp * DHP + (size_t)DHP * (sp + 4)) * sizeof(float);
    const float qscale = (1.0f / sqrtf((float)Dh)) * kLog2e;
    const dim3 grid((unsigned)(B * H)), block(NAR_THREADS);
    const int BH = B * H;
    const MhaRope rp = rope != nullptr ? *rope : MhaRope{};
    ProfScope ps(st, rope != nullptr ? (O != nullptr ? "mha_nar_rope_fwd" : "mha_nar_rope_stats")
                                     : (O != nullptr ? "mha_nar_fwd" : "mha_nar_stats"));
    if (rope != nullptr) {
        if (O == nullptr)
            CXG_LAUNCH((mha_nar_fwd_kernel<DHP, VEC, false, true>), grid, block, lds, st, Q, K, V,
                       O, lse, S, H, Dh, BH, qscale, rp);
        else
            CXG_LAUNCH((mha_nar_fwd_kernel<DHP, VEC, true, true>), grid, block, lds, st, Q, K, V,
                       O, lse, S, H, Dh, BH, qscale, rp);
    } else if (O == nullptr) {
        CXG_LAUNCH((mha_nar_fwd_kernel<DHP, VEC, false, false>), grid, block, lds, st, Q, K, V, O,
                   lse, S, H, Dh, BH, qscale, rp);
    } else {
        CXG_LAUNCH((mha_nar_fwd_kernel<DHP, VEC, true, false>), grid, block, lds, st, Q, K, V, O,
                   lse, S, H, Dh, BH, qscale, rp);
    }
    return hipGetLastError();
}

hipError_t mha_nar_fwd_launch(const float* Q, const float* K, const float* V, float* O,
                              float* lse, int B, int S, int H, int Dh, hipStream_t st,
                              const MhaRope* rope)
{
    if (!mha_nar_ok(B, S, H, Dh) || (rope != nullptr && Dh % 2 != 0))
        return hipErrorInvalidValue;
    const bool vec = Dh % 4 == 0 && nar_al16(Q) && nar_al16(K) && nar_al16(V) && nar_al16(O);
    if (Dh <= 8)
        return vec ? nar_fwd_t<8, true>(Q, K, V, O, lse, B, S, H, Dh, st, rope)
                   : nar_fwd_t<8, false>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    return vec ? nar_fwd_t<16, true>(Q, K, V, O, lse, B, S, H, Dh, st, rope)
               : nar_fwd_t<16, false>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
}

template <int DHP, bool VEC, int NBM, bool ROPE>
static void nar_bwd_go(const float* Q, const float* K, const float* V, const float* O,
                       const float* dO, const float* lse, float* dQ, float* dK, float* dV, int S,
                       int H, int Dh, int BH, float qscale, float scale, const MhaRope& rp,
                       size_t lds, hipStream_t st)
{
    const dim3 grid((unsigned)BH), block(NAR_THREADS);
    if (lse == nullptr)
        CXG_LAUNCH((mha_nar_bwd_kernel<DHP, VEC, true, NBM, ROPE>), grid, block, lds, st, Q, K, V,
                   O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale, scale, rp);
    else
        CXG_LAUNCH((mha_nar_bwd_kernel<DHP, VEC, false, NBM, ROPE>), grid, block, lds, st, Q, K,
                   V, O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale, scale, rp);
}

template <int DHP, bool VEC>
static hipError_t nar_bwd_t(const float* Q, const float* K, const float* V, const float* O,
                            const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                            int B, int S, int H, int Dh, hipStream_t st, const MhaRope* rope)
{
    const int sp = (S + 15) / 16 * 16;
    const size_t lds = ((size_t)2 * (DHP + 1) * (sp + 4) + (size_t)sp * DHP + 2 * (size_t)sp +
                        4 * 16 * NAR_TLD) *
                       sizeof(float);
    const float scale = 1.0f / sqrtf((float)Dh);
    const float qscale = scale * kLog2e;
    const int BH = B * H;
    const MhaRope rp = rope != nullptr ? *rope : MhaRope{};
    ProfScope ps(st, rope != nullptr ? "mha_nar_rope_bwd" : "mha_nar_bwd");
    if (sp <= 256) {
        if (rope != nullptr)
            nar_bwd_go<DHP, VEC, 16, true>(Q, K, V, O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale,
                                           scale, rp, lds, st);
        else
            nar_bwd_go<DHP, VEC, 16, false>(Q, K, V, O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale,
                                            scale, rp, lds, st);
    } else if constexpr (DHP == 8) {   // S_pad * DHP <= 4096: 32 blocks at most
        if (rope != nullptr)
            nar_bwd_go<DHP, VEC, 32, true>(Q, K, V, O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale,
                                           scale, rp, lds, st);
        else
            nar_bwd_go<DHP, VEC, 32, false>(Q, K, V, O, dO, lse, dQ, dK, dV, S, H, Dh, BH, qscale,
                                            scale, rp, lds, st);
    } else {
        return hipErrorInvalidValue;   // excluded by mha_nar_ok
    }
    return hipGetLastError();
}

hipError_t mha_nar_bwd_launch(const float* Q, const float* K, const float* V, const float* O,
                              const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                              int B, int S, int H, int Dh, hipStream_t st, const MhaRope* rope)
{
    if (!mha_nar_ok(B, S, H, Dh) || (rope != nullptr && Dh % 2 != 0))
        return hipErrorInvalidValue;
    const bool vec = Dh % 4 == 0 && nar_al16(Q) && nar_al16(K) && nar_al16(V) && nar_al16(O) &&
                     nar_al16(dO) && nar_al16(dQ) && nar_al16(dK) && nar_al16(dV);
    if (Dh <= 8)
        return vec ? nar_bwd_t<8, true>(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, st, rope)
                   : nar_bwd_t<8, false>(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, st, rope);
    return vec ? nar_bwd_t<16, true>(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, st, rope)
               : nar_bwd_t<16, false>(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, st, rope);
}

} // namespace cxg
