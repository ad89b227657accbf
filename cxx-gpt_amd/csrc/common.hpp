// common.hpp -- device helpers shared by the gfx950 attention kernels.
//
// MFMA fragment convention used throughout (v_mfma_f32_16x16x4_f32, wave64):
//   lane l, l16 = l % 16, g = l / 16
//   A operand (16 x 4):  lane l holds A[i = l16][k = g]
//   B operand (4 x 16):  lane l holds B[k = g][j = l16]
//   C/D (16 x 16, f4):   lane l, element r holds D[i = 4*g + r][j = l16]
// A contraction over a long axis is split into 4-wide steps; which physical
// index feeds (instruction, k-slot) is free as long as A and B agree, and the
// kernels pick the mapping that lets an accumulator feed the next MFMA
// directly: instruction r, k-slot g <-> index 4*g + r of a 16-block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace cxg {

typedef float f4 __attribute__((ext_vector_type(4)));

// Compile-time integer argument for generic lambdas (a lambda body
// instantiated once per value).
template <int N>
using ic = std::integral_constant<int, N>;

__device__ __forceinline__ f4 mfma16(float a, float b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 f4zero()
{
    f4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return z;
}

__device__ __forceinline__ f4 f4splat(float v)
{
    f4 z = {v, v, v, v};
    return z;
}

// 2^x on the hardware transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Sum / max over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float xrow_sum(float v)
{
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}
__device__ __forceinline__ float xrow_max(float v)
{
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Lane exchange within a 16-lane row through DPP (no LDS round trip).  The
// patterns used here (quad_perm, row_ror, row_mirror, row_half_mirror) have a
// source lane for every lane, so bound_ctrl is set: no old value to keep,
// which lets the compiler fold the move into the instruction that uses it.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// The value of lane l ^ M (M = 1, 2, 4, 8: within the lane's 16-lane row)
// through DPP lane moves, which stay in the VALU (a shuffle through
// ds_bpermute takes a round trip through the LDS unit).  Lane l ^ 4 is two
// moves: row_half_mirror (lane i of each 8 reads lane 7 - i, i.e. i ^ 7),
// then quad_perm [3,2,1,0] (i ^ 3): i ^ 7 ^ 3 = i ^ 4.
template <int M>
__device__ __forceinline__ float lane_xor16(float v)
{
    if constexpr (M == 1)
        return dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    else if constexpr (M == 2)
        return dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    else if constexpr (M == 8)
        return dpp_f<0x128>(v);   // row_ror:8
    else {
        static_assert(M == 4, "lane_xor16: M in {1, 2, 4, 8}");
        return dpp_f<0x1B>(dpp_f<0x141>(v));   // row_half_mirror, quad_perm [3,2,1,0]
    }
}

// Sum over the 16 lanes of one row (lanes sharing l / 16): rotations by 8
// and 4 within the row, then the quad swaps 2 and 1.  Each lane adds the same
// pairs as an xor-8/4/2/1 butterfly, so the result is that butterfly's.
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f<0x128>(v);   // row_ror:8
    v += dpp_f<0x124>(v);   // row_ror:4
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    return v;
}

// Guarded 4-wide load of row[c..c+3] (columns >= n read as 0).  VEC requires
// the row base to be 16-byte aligned and n % 4 == 0.
template <bool VEC>
__device__ __forceinline__ f4 load4(const float* __restrict__ row, int c, int n, bool ok)
{
    f4 v = f4zero();
    if (!ok)
        return v;
    if (VEC) {
        if (c < n)
            v = *reinterpret_cast<const f4*>(row + c);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (c + i < n)
                v[i] = row[c + i];
    }
    return v;
}

template <bool VEC>
__device__ __forceinline__ void store4(float* __restrict__ row, int c, int n, f4 v)
{
    if (VEC) {
        if (c < n)
            *reinterpret_cast<f4*>(row + c) = v;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (c + i < n)
                row[c + i] = v[i];
    }
}

// Clamped 4-wide load for streamed tiles: the row and column are clamped into
// the valid data, so the load always issues and never needs a guard.  Padded
// positions (rows >= S, columns >= Dh) therefore hold copies of real, finite
// inputs; the kernels neutralise them elsewhere: the operand they meet in a
// product is zero (Q/K/V registers zeroed beyond Dh) or the probability they
// carry is masked to exactly 0.  Keeping loads unconditional lets a thread put
// all of a tile's loads in flight at once.  VEC: n % 4 == 0 and the row base
// is 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ f4 load4c(const float* __restrict__ row, int c, int n)
{
    f4 v;
    if (VEC) {
        v = *reinterpret_cast<const f4*>(row + (c < n ? c : n - 4));
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
            v[i] = row[c + i < n ? c + i : n - 1];
    }
    return v;
}

// Zero the lanes of a loaded f4 whose row is invalid (!ok) or whose columns
// lie past n.  Applied apart from the (clamped, unconditional) load, once the
// data is needed anyway, so that the load itself stays asynchronous.
__device__ __forceinline__ f4 mask4(f4 v, int c, int n, bool ok)
{
#pragma unroll
    for (int i = 0; i < 4; i++)
        v[i] = (ok && c + i < n) ? v[i] : 0.0f;
    return v;
}

__device__ __forceinline__ void atomic_add_f32(float* p, float v)
{
    unsafeAtomicAdd(p, v);
}

// Stores and float atomic adds through a raw buffer descriptor over
// [base, base + 2 GiB): a lane whose byte offset is kDropOffset (past the
// descriptor's range) is dropped by the hardware bounds check, as is every
// lane of a descriptor built with no records.  Masked lanes therefore need no
// branch, and every path issues the same number of memory instructions, which
// keeps the compiler's waits on earlier loads exact (a branch around a store
// or atomic makes it wait for all of them).
constexpr unsigned kDropOffset = 0x7ffffff0u;

typedef unsigned u4 __attribute__((ext_vector_type(4)));

// Raw (stride 0) buffer; 0x00020000: 32-bit data format, the gfx9 raw layout.
// base == nullptr gives a descriptor that drops every access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const float* base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                             base != nullptr ? (int)kDropOffset : 0, 0x00020000);
}

__device__ __forceinline__ void buffer_atomic_add_f32(__amdgpu_buffer_rsrc_t r, unsigned off,
                                                      float v)
{
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r, (int)off, 0, 0);
}

// 4-byte load at voff + soff, soff wave-uniform
__device__ __forceinline__ float buffer_load_f32s(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

// atomic add at voff + soff, soff wave-uniform
__device__ __forceinline__ void buffer_atomic_add_f32s(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                       unsigned soff, float v)
{
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r, (int)voff, (int)soff, 0);
}

__device__ __forceinline__ void buffer_store_f4(__amdgpu_buffer_rsrc_t r, unsigned off, f4 v)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, (int)off, 0, 0);
}

__device__ __forceinline__ void buffer_store_f32(__amdgpu_buffer_rsrc_t r, unsigned off, float v)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)off, 0, 0);
}

// Load through a buffer descriptor: out-of-range lanes read 0.
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, unsigned off)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

__device__ __forceinline__ f4 buffer_load_f4(__amdgpu_buffer_rsrc_t r, unsigned off)
{
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Device-coherent accesses (cache policy sc1 on gfx950): a store is written
// through to where every compute unit of the device reads it, and a load does
// not take a copy that another XCD's L2 may have made stale.  Data shared
// between workgroups inside one launch moves this way, so that no
// device-scope fence (an L2-wide write-back or invalidate) is needed.
constexpr int kCPolDevice = 16;

__device__ __forceinline__ void buffer_store_f4_dev(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                    unsigned soff, f4 v)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, (int)voff, (int)soff,
                                           kCPolDevice);
}

__device__ __forceinline__ void buffer_store_f32_dev(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                     unsigned soff, float v)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)voff,
                                          (int)soff, kCPolDevice);
}

__device__ __forceinline__ float buffer_load_f32s_dev(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                      unsigned soff)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff,
                                                                          kCPolDevice));
}

// Wait until this wave's vector memory operations (loads and stores) are done.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Raw buffer over [base, base + bytes): reads at or past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_n(const float* base, unsigned bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)bytes, 0x00020000);
}

// 16-byte load at voff + soff, soff wave-uniform (a scalar operand, so a
// tile's row offset costs no vector instruction).
__device__ __forceinline__ f4 buffer_load_f4s(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff)
{
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Rotary embedding of one f4 of a row at position pos, columns c .. c+3 of a
// head (c a multiple of 4): pairs (c, c+1) and (c+2, c+3) rotate by
// sign * pos * w[pair] (sign -1: the inverse, for gradients).
// sin and cos of a float angle a (radians, |a| < 2^20): reduced to [-pi, pi]
// in double precision (k = rint(a / 2pi), r = a - 2pi k: error below 1e-10 at
// these magnitudes), then evaluated on r / 2pi revolutions by the hardware
// v_sin_f32 / v_cos_f32 (max abs error 1.3e-7 over [-0.5, 0.5] revolutions,
// measured on MI355X against double).  About ten instructions, against the
// general-argument library routine's hundred.
__device__ __forceinline__ void sincos_rev(float a, float* s, float* c)
{
    constexpr double kInv2Pi = 0.15915494309189535;
    constexpr double k2Pi = 6.283185307179586;
    const double ad = (double)a;
    const double k = rint(ad * kInv2Pi);
    const float x = (float)(fma(-k, k2Pi, ad) * kInv2Pi);
    *s = __builtin_amdgcn_sinf(x);
    *c = __builtin_amdgcn_cosf(x);
}

// w: the frequency table (an LDS copy: w[i] = 10000^(-2i/head_dim)).
__device__ __forceinline__ f4 rope4(f4 v, int pos, int c, const float* w, float sign)
{
    float s0, c0, s1, c1;
    sincos_rev(sign * (float)pos * w[c >> 1], &s0, &c0);
    sincos_rev(sign * (float)pos * w[(c >> 1) + 1], &s1, &c1);
    f4 o;
    o[0] = v[0] * c0 - v[1] * s0;
    o[1] = v[0] * s0 + v[1] * c0;
    o[2] = v[2] * c1 - v[3] * s1;
    o[3] = v[2] * s1 + v[3] * c1;
    return o;
}

} // namespace cxg
