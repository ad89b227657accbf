// linattn_dev.hpp -- device helpers shared by the linear-attention kernels
// (linattn.hip: forward, split backward; linbwd.hip: fused backward): the
// feature map, the LDS chunk stage layout and its register views.
//
// Register layouts of a 16-row chunk (lane l, l16 = l%16, g = l/16, f4 element r):
//   R-layout:  v[ct][r] = M[t0 + l16][16ct + 4g + r]   (row per lane)
//   C-layout:  v[ct][r] = M[t0 + 4g + r][16ct + l16]   (column per lane)
#pragma once

#include "common.hpp"
#include "linattn.hpp"

namespace cxg {

constexpr int CLD = 68;             // LDS row stride of a staged 16 x 64 chunk
constexpr int CHUNK = 16 * CLD;     // floats per staged chunk matrix

template <int PHI>
struct Phi;
template <>
struct Phi<PHI_ELU1> {
    // two_stage_cuda_kernels.cu:1027-1031 / kernel_test.cpp:16-17, as the
    // median of x + 1, e^x and 1 (e^x >= 1 + x, so it is x + 1 for x > 0 and
    // e^x otherwise, up to the roundings of the two where they meet near 0):
    // one instruction fewer than the compare and select
    static __device__ __forceinline__ float f(float x)
    {
        return __builtin_amdgcn_fmed3f(x + 1.0f, __expf(x), 1.0f);
    }
    static __device__ __forceinline__ float d(float x) { return x > 0.0f ? 1.0f : __expf(x); }
    // phi'(x) from phi(x): phi(x) = x+1 > 1 for x > 0 and exp(x) <= 1 otherwise
    static __device__ __forceinline__ float d_from_f(float p) { return fminf(p, 1.0f); }
};
template <>
struct Phi<PHI_ELU1_LG> {
    // linear_cuda_kernels.cu:316-320 (phi_elu_fwd_kernel): ELU(x) + 1 with
    // ELU(x) = expf(x) - 1 for x <= 0, the two roundings kept
    static __device__ __forceinline__ float f(float x) { return x > 0.0f ? x + 1.0f : (expf(x) - 1.0f) + 1.0f; }
    // :347-364 (phi_elu_bwd_kernel)
    static __device__ __forceinline__ float d(float x) { return x > 0.0f ? 1.0f : expf(x); }
    // from phi: 1 for x > 0; for x <= 0, phi is expf(x) rounded to a multiple of
    // 2^-24 (expf(x) - 1 is rounded in [-1, -0.5)), so min(phi, 1) is within
    // 2^-25 of expf(x)
    static __device__ __forceinline__ float d_from_f(float p) { return fminf(p, 1.0f); }
};
// ELU+1 of rotated inputs: the elementwise part is two_stage's ELU+1; the
// rotation is applied to the raw row before it (rot_row below).
template <>
struct Phi<PHI_ELU1_ROPE> : Phi<PHI_ELU1> {
};
// PHI_HEXP has no elementwise form: the kernels apply it to whole rows
// (hexp_row4, hexp_colC below) and leave Phi<PHI_HEXP> undefined, so that no
// elementwise site can take it by mistake.
template <>
struct Phi<PHI_NONE> {
    static __device__ __forceinline__ float f(float x) { return x; }
    static __device__ __forceinline__ float d(float) { return 1.0f; }
    static __device__ __forceinline__ float d_from_f(float) { return 1.0f; }
};

// ---------------------------------------------------------------------------
// Hadamard+Exp feature map of a 64-column row: phi(x) = exp((H x) / 8), H the
// 64x64 Sylvester Hadamard matrix (y_i = sum_j (-1)^popcount(i & j) x_j,
// phi_hexp_* in linattn.hip).  The transform's butterflies run over the
// column bits from bit 0 up, as the one-element-per-lane transform does, so
// every layout gives the same roundings.
// ---------------------------------------------------------------------------

// One butterfly stage over lane bit M: lower lane a + b, upper lane a - b
// (a the lower lane's value, b the upper's).
template <int M>
__device__ __forceinline__ float bfly16(float v, int lane)
{
    const float u = lane_xor16<M>(v);
    return (lane & M) ? (u - v) : (v + u);
}

// Row-coalesced layout: a lane holds columns 4q .. 4q+3 (q = lane % 16) of a
// row that the 16 lanes of its group share: bits 0-1 are in-lane, bits 2-5
// exchanges within the 16-lane group.  Returns (H v) * scale.
__device__ __forceinline__ f4 fwht64_f4(f4 v, int lane, float scale)
{
    f4 t;
    t[0] = v[0] + v[1];
    t[1] = v[0] - v[1];
    t[2] = v[2] + v[3];
    t[3] = v[2] - v[3];
    v[0] = t[0] + t[2];
    v[1] = t[1] + t[3];
    v[2] = t[0] - t[2];
    v[3] = t[1] - t[3];
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = bfly16<1>(v[i], lane);
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = bfly16<2>(v[i], lane);
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = bfly16<4>(v[i], lane);
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = bfly16<8>(v[i], lane);
    return v * scale;
}

__device__ __forceinline__ f4 hexp_row4(f4 v, int lane)
{
    f4 y = fwht64_f4(v, lane, 0.125f);
#pragma unroll
    for (int i = 0; i < 4; i++)
        y[i] = __expf(y[i]);
    return y;
}

// MFMA column layout: x[k] is column 16k + l16 of the lane's row (the row is
// shared by the 16 lanes of the group): bits 0-3 are exchanges within the
// group, bits 4-5 in-lane.
__device__ __forceinline__ void hexp_colC(float (&x)[4], int lane)
{
#pragma unroll
    for (int k = 0; k < 4; k++)
        x[k] = bfly16<1>(x[k], lane);
#pragma unroll
    for (int k = 0; k < 4; k++)
        x[k] = bfly16<2>(x[k], lane);
#pragma unroll
    for (int k = 0; k < 4; k++)
        x[k] = bfly16<4>(x[k], lane);
#pragma unroll
    for (int k = 0; k < 4; k++)
        x[k] = bfly16<8>(x[k], lane);
    const float a0 = x[0] + x[1], a1 = x[0] - x[1], a2 = x[2] + x[3], a3 = x[2] - x[3];
    x[0] = __expf((a0 + a2) * 0.125f);
    x[1] = __expf((a1 + a3) * 0.125f);
    x[2] = __expf((a0 - a2) * 0.125f);
    x[3] = __expf((a1 - a3) * 0.125f);
}

// ---------------------------------------------------------------------------
// RoPE of the PHI_ELU1_ROPE maps.  The frequency table goes to LDS at kernel
// start (one lane, uniform indices, so the argument is read with scalar
// loads; the caller synchronises before the first use).  rot_row rotates an
// f4 holding columns c .. c+3 of the row at sequence position pos; other maps
// leave it unchanged.
// ---------------------------------------------------------------------------
template <int PHI, int N>
__device__ __forceinline__ void rope_tab_lds(float* __restrict__ dst, const LinRopeArg<PHI>& a)
{
    if constexpr (phi_rope(PHI)) {
        static_assert(N <= LIN_ROPE_MAX_D / 2, "rope table");
        for (int i = threadIdx.x; i < N; i += blockDim.x)
            dst[i] = a.w[i];
    }
}

template <int PHI>
__device__ __forceinline__ f4 rot_row(f4 v, int pos, int c, const float* __restrict__ rw,
                                      float sign = 1.0f)
{
    if constexpr (phi_rope(PHI))
        return rope4(v, pos, c, rw, sign);
    return v;
}

// Gradient with respect to the raw row x of a RoPE map's feature row
// phi(rot(x)): g (columns c .. c+3, gradient w.r.t. the features) times
// phi'(rot(x)), rotated back; one sin/cos per pair serves both rotations.
template <int PHI>
__device__ __forceinline__ f4 rope_phi_grad4(f4 g, f4 x, int pos, int c,
                                             const float* __restrict__ rw)
{
    f4 o;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float sn, cs;
        sincos_rev((float)pos * rw[(c >> 1) + h], &sn, &cs);
        const float x0 = x[2 * h], x1 = x[2 * h + 1];
        const float g0 = g[2 * h] * Phi<PHI>::d(x0 * cs - x1 * sn);
        const float g1 = g[2 * h + 1] * Phi<PHI>::d(x0 * sn + x1 * cs);
        o[2 * h] = g0 * cs + g1 * sn;
        o[2 * h + 1] = -g0 * sn + g1 * cs;
    }
    return o;
}

// ---------------------------------------------------------------------------
// chunk staging helpers
// ---------------------------------------------------------------------------
// Template flags of the fast-path kernels: VEC = widths multiple of 4 and
// 16-byte aligned rows (16-byte loads / stores), FW = D == E == 64 (no column
// masks at all).  Row addresses are a wave-uniform chunk base plus a 32-bit
// per-lane offset.

// Raw R-layout registers of a chunk: lane (l16, g) holds chunk row `ro` (the
// caller clamps it into the segment), columns 16ct + 4g .. +3 (clamped to ncol).
template <bool VEC>
__device__ __forceinline__ void ldR(f4 (&v)[4], const float* __restrict__ base, int ld, int ro,
                                    int ncol, int g)
{
    const float* p = base + ro * ld;
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
        v[ct] = load4c<VEC>(p, 16 * ct + 4 * g, ncol);
}

// Apply phi, then zero the entries outside the valid columns (unless the
// width is full) and rows (only in a partial chunk; `full` is wave-uniform).
template <int PHI, bool APPLY, bool FW>
__device__ __forceinline__ void finR(f4 (&v)[4], bool full, bool rok, int ncol, int g)
{
    if constexpr (APPLY && PHI != PHI_NONE)
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[ct][i] = Phi<PHI>::f(v[ct][i]);
    if (!FW)
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[ct][i] = (16 * ct + 4 * g + i < ncol) ? v[ct][i] : 0.0f;
    if (!full)
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
            v[ct] = rok ? v[ct] : f4zero();
}

// Store an R-layout f4 of one row: no guard for a full width.
template <bool VEC, bool FW>
__device__ __forceinline__ void stR(float* __restrict__ row, int c, int n, f4 v)
{
    if (FW)
        *reinterpret_cast<f4*>(row + c) = v;
    else
        store4<VEC>(row, c, n, v);
}

__device__ __forceinline__ void putR(float* __restrict__ buf, const f4 (&v)[4], int l16, int g)
{
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
        *reinterpret_cast<f4*>(&buf[l16 * CLD + 16 * ct + 4 * g]) = v[ct];
}

// The same for a part of a chunk: column tiles ct0 .. ct0+NCT-1.  The waves
// of a segment stage the chunk's inputs by column tiles, so each wave loads
// and transforms (phi) an equal share.
template <bool VEC, int NCT>
__device__ __forceinline__ void ldRp(f4 (&v)[NCT], const float* __restrict__ base, int ld, int ro,
                                     int ncol, int g, int ct0)
{
    const float* p = base + ro * ld;
#pragma unroll
    for (int i = 0; i < NCT; i++)
        v[i] = load4c<VEC>(p, 16 * (ct0 + i) + 4 * g, ncol);
}

template <int PHI, bool APPLY, bool FW, int NCT>
__device__ __forceinline__ void finRp(f4 (&v)[NCT], bool full, bool rok, int ncol, int g, int ct0)
{
    if constexpr (APPLY && PHI != PHI_NONE)
#pragma unroll
        for (int i = 0; i < NCT; i++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[i][e] = Phi<PHI>::f(v[i][e]);
    if (!FW)
#pragma unroll
        for (int i = 0; i < NCT; i++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[i][e] = (16 * (ct0 + i) + 4 * g + e < ncol) ? v[i][e] : 0.0f;
    if (!full)
#pragma unroll
        for (int i = 0; i < NCT; i++)
            v[i] = rok ? v[i] : f4zero();
}

template <int NCT>
__device__ __forceinline__ void putRp(float* __restrict__ buf, const f4 (&v)[NCT], int l16, int g,
                                      int ct0)
{
#pragma unroll
    for (int i = 0; i < NCT; i++)
        *reinterpret_cast<f4*>(&buf[l16 * CLD + 16 * (ct0 + i) + 4 * g]) = v[i];
}

__device__ __forceinline__ void getR(const float* __restrict__ buf, f4 (&v)[4], int l16, int g)
{
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
        v[ct] = *reinterpret_cast<const f4*>(&buf[l16 * CLD + 16 * ct + 4 * g]);
}

__device__ __forceinline__ void getC(const float* __restrict__ buf, f4 (&c)[4], int l16, int g)
{
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            c[ct][r] = buf[(4 * g + r) * CLD + 16 * ct + l16];
}

// Per-row scalars of chunk rows 4g+r (row offsets clamped to rmax), column layout.
__device__ __forceinline__ f4 ldRowsC(const float* __restrict__ w, int rmax, int g)
{
    f4 v;
#pragma unroll
    for (int r = 0; r < 4; r++)
        v[r] = w[min(4 * g + r, rmax)];
    return v;
}

// Inclusive prefix sum over the 16 chunk rows of a column-layout value
// (rows 4g+r of column l16); returns the prefixes and the column total.
__device__ __forceinline__ f4 col_prefix16(f4 c, float& total, int lane)
{
    const int g = lane >> 4;
    f4 p;
    p[0] = c[0];
    p[1] = p[0] + c[1];
    p[2] = p[1] + c[2];
    p[3] = p[2] + c[3];
    float x = p[3];
    float y = __shfl_up(x, 16, 64);
    x = g >= 1 ? x + y : x;
    y = __shfl_up(x, 32, 64);
    x = g >= 2 ? x + y : x;   // inclusive prefix of the 4-row totals over g
    const float excl = x - p[3];
    total = __shfl(x, 48 + (lane & 15), 64);
    return p + excl;
}

__device__ __forceinline__ f4 colC(const float* __restrict__ buf, int ct, int l16, int g)
{
    f4 c;
#pragma unroll
    for (int r = 0; r < 4; r++)
        c[r] = buf[(4 * g + r) * CLD + 16 * ct + l16];
    return c;
}

} // namespace cxg
