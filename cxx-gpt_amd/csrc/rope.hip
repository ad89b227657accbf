// rope.hip -- rotary position embedding on (B*S, D) activations, in place.
//
// Replaces two_stage_cuda::rope_fwd / rope_bwd
// (src/TwoStage/two_stage_cuda_kernels.cu:1810-1878), which rotate the
// stage-1 q/k heads and the stage-2 q/k feature rows of two_stage_gpt.hpp
// (:102, :113, :160, :174).  Pair i of a head of width head_dim in a row at
// position p (row % S) rotates by sign * p * w_i, w_i = 10000^(-2i/head_dim):
//   x'_2i = x_2i cos - x_2i+1 sin,   x'_2i+1 = x_2i sin + x_2i+1 cos;
// sign -1 (the backward) is the inverse rotation.
//
// Design.  HBM-bound: 16 bytes read and written per pair of Q and K.  A
// thread owns one pair column and ROWS consecutive rows, so the pair's
// frequency is fetched once and a wave covers 64 consecutive pairs (512 B of
// one row) per access; pairs move as 8-byte loads and stores.  The
// frequencies w_i come from the host (powf of the same float exponent the
// reference's CPU check uses, kernel_test.cpp:453), so the angle sign*p*w_i
// is the same float product on both sides.  When Q and K are one buffer the
// reference rotates it twice (once as Q, once as K); the ALIAS variant does
// the same in registers.
#include "common.hpp"
#include "launch.hpp"

#include <math.h>

namespace cxg {

constexpr int ROPE_THREADS = 256;
constexpr int ROPE_ROWS = 2;

// VEC: rows of Q and K 8-byte aligned (pairs move as float2).  Q and K may be
// one buffer (ALIAS), so they are not declared restrict.
template <bool ALIAS, bool VEC>
__global__ __launch_bounds__(ROPE_THREADS) void rope_kernel(float* Q, float* K, long rows, int S,
                                                            int D, int head_dim, float sign,
                                                            RopeFreqs fr)
{
    const int np = D / 2;
    const long idx = (long)blockIdx.x * ROPE_THREADS + threadIdx.x;
    const long rblk = idx / np;
    const int pair = (int)(idx - rblk * np);
    const long r0 = rblk * ROPE_ROWS;
    if (r0 >= rows)
        return;
    const int pih = pair % (head_dim / 2);
    const float w = fr.w[pih];
    const long off0 = r0 * D + (long)(pair / (head_dim / 2)) * head_dim + 2 * pih;
    int p = (int)(r0 % S);
    auto rot = [&](float2 v, float c, float s) {
        float2 o;
        o.x = v.x * c - v.y * s;
        o.y = v.x * s + v.y * c;
        return o;
    };
    auto ld = [&](const float* a) {
        if (VEC)
            return *reinterpret_cast<const float2*>(a);
        return make_float2(a[0], a[1]);
    };
    auto st = [&](float* a, float2 v) {
        if (VEC) {
            *reinterpret_cast<float2*>(a) = v;
        } else {
            a[0] = v.x;
            a[1] = v.y;
        }
    };
#pragma unroll
    for (int k = 0; k < ROPE_ROWS; k++) {
        if (r0 + k < rows) {
            const float ang = sign * (float)p * w;
            float s, c;
            sincosf(ang, &s, &c);
            const long off = off0 + (long)k * D;
            if (ALIAS) {
                st(Q + off, rot(rot(ld(Q + off), c, s), c, s));
            } else {
                if (Q != nullptr)
                    st(Q + off, rot(ld(Q + off), c, s));
                if (K != nullptr)
                    st(K + off, rot(ld(K + off), c, s));
            }
        }
        p = (p + 1 == S) ? 0 : p + 1;
    }
}

void rope_freqs(int head_dim, RopeFreqs* fr)
{
    // kernel_test.cpp:453: w = pow(10000.0f, -2.0f * (float)i / (float)head_dim)
    for (int i = 0; i < head_dim / 2; i++)
        fr->w[i] = powf(10000.0f, -2.0f * (float)i / (float)head_dim);
}

hipError_t rope_launch(float* Q, float* K, long B, int S, int D, int head_dim, float sign,
                       hipStream_t st)
{
    RopeFreqs fr;
    rope_freqs(head_dim, &fr);
    const long rows = B * S;
    const long nthreads = (rows + ROPE_ROWS - 1) / ROPE_ROWS * (D / 2);
    dim3 grid((unsigned)((nthreads + ROPE_THREADS - 1) / ROPE_THREADS)), block(ROPE_THREADS);
    ProfScope ps(st, sign > 0 ? "rope_fwd" : "rope_bwd");
    const bool vec = ((uintptr_t)Q & 7u) == 0 && ((uintptr_t)K & 7u) == 0;
    const bool alias = Q != nullptr && Q == K;
    if (alias && vec)
        CXG_LAUNCH((rope_kernel<true, true>), grid, block, 0, st, Q, K, rows, S, D,
                           head_dim, sign, fr);
    else if (alias)
        CXG_LAUNCH((rope_kernel<true, false>), grid, block, 0, st, Q, K, rows, S, D,
                           head_dim, sign, fr);
    else if (vec)
        CXG_LAUNCH((rope_kernel<false, true>), grid, block, 0, st, Q, K, rows, S, D,
                           head_dim, sign, fr);
    else
        CXG_LAUNCH((rope_kernel<false, false>), grid, block, 0, st, Q, K, rows, S, D,
                           head_dim, sign, fr);
    return hipGetLastError();
}

} // namespace cxg
