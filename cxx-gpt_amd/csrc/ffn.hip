// ffn.hip -- the two-stage block's expander FFNs: two bias-free Linear
// layers with the exact GELU between them, forward and backward, as FP32
// MFMA GEMMs with the elementwise work in their epilogues.
//
// Replaces the call sequence (per expander, two_stage_gpt.hpp:86-99 and
// :177-195; Linear::forward/backward at gpt_gpt.hpp:86-112):
//   forward   pre = X W1^T; act = gelu(pre); Y = act W2^T
//   backward  dP = dY W2; dact = dP * gelu'(G); dW2 += dY^T act;
//             dX = dact W1; dW1 += dact^T X
// X [M][E], W1 [F][E], W2 [E][F], row-major.  G is the tensor the caller
// evaluates gelu' at: the expanders pass their GELU output, the final FFN its
// pre-activation (:141, :179).
//
// One GEMM kernel C[M][N] = sum_k A(i,k) B(k,j) covers all six products:
//   AK: A(i,k) at A[i*lda + k] (k contiguous), else at A[k*lda + i];
//   BK: B(k,j) at B[j*ldb + k], else at B[k*ldb + j].
// A workgroup of 4 waves computes a 128 x 128 tile of C, each wave 64 x 64
// (4 x 4 blocks of v_mfma_f32_16x16x4_f32), over k-tiles of 32: the next
// tile's global loads are issued before the current tile's MFMAs, land in
// registers and are written to the other half of a double-buffered LDS stage
// after them (one barrier per k-tile).  In LDS a k-contiguous operand keeps
// its rows ([row][k], stride 36: a lane's four k-slots are one 16-byte read)
// and a row-contiguous one its k-rows ([k][row], stride 132).  The MFMA takes
// the B fragment as its first operand, so a lane's accumulator holds four
// consecutive columns of one row of C and every epilogue access is 16 bytes.
// Shapes whose tile count leaves most compute units idle (N = E = 768 at
// M = 2048) split K over workgroups: partial tiles go to a workspace and a
// reduction applies the epilogue.
//
// Requires E, F multiples of 4 and 16-byte aligned tensors (checked at the C
// ABI); any M.
#include "common.hpp"
#include "gelu_dev.hpp"
#include "launch.hpp"

#include <algorithm>

namespace cxg {

constexpr int GT = 128;                 // tile rows and columns
constexpr int GKT = 32;                 // k-tile
constexpr int KLD = GKT + 4;            // [row][k] stride
constexpr int RLD = GT + 4;             // [k][row] stride
constexpr int OPF = GT * KLD > GKT * RLD ? GT * KLD : GKT * RLD;   // floats per operand stage

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    const float* G;
    float* pre;
    long lda, ldb, ldc;
    int M, N, K;
    int tn;            // tiles along N
    int tiles;         // tiles per split
    int ktp;           // k-tiles per split
    long sstride;      // floats between split partials (0: no split)
};

// Epilogue for four consecutive columns of one row of C at element offset off.
template <int EPI>
__device__ __forceinline__ void epi_apply(f4 v, long off, float* C, const float* G, float* pre)
{
    if (EPI == FFN_EPI_STORE) {
        *reinterpret_cast<f4*>(C + off) = v;
    } else if (EPI == FFN_EPI_GELU) {
        if (pre != nullptr)
            *reinterpret_cast<f4*>(pre + off) = v;
#pragma unroll
        for (int e = 0; e < 4; e++)
            v[e] = gelu_f(v[e]);
        *reinterpret_cast<f4*>(C + off) = v;
    } else if (EPI == FFN_EPI_DGELU) {
        const f4 g = *reinterpret_cast<const f4*>(G + off);
#pragma unroll
        for (int e = 0; e < 4; e++)
            v[e] *= gelu_d(g[e]);
        *reinterpret_cast<f4*>(C + off) = v;
    } else {   // FFN_EPI_ACCUM
        const f4 c = *reinterpret_cast<const f4*>(C + off);
        *reinterpret_cast<f4*>(C + off) = c + v;
    }
}

// One operand's 128 x 32 k-tile, 4 float4 per thread.  KC: element (row, k)
// at P[row*ld + k].  Rows past the end are clamped onto the last row (their
// products land in C rows/columns that are never stored); k past K reads 0.
template <bool KC>
__device__ __forceinline__ void tile_fetch(const float* __restrict__ P, long ld, int r0, int rows,
                                           int k0, int K, f4 (&v)[4])
{
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int idx = t + 256 * q;
        if (KC) {
            const int r = min(r0 + (idx >> 3), rows - 1);
            const int k = k0 + (idx & 7) * 4;
            const f4 x = *reinterpret_cast<const f4*>(P + (long)r * ld + min(k, K - 4));
            v[q] = k < K ? x : f4zero();
        } else {
            const int k = k0 + (idx >> 5);
            const int r = min(r0 + (idx & 31) * 4, rows - 4);
            const f4 x = *reinterpret_cast<const f4*>(P + (long)min(k, K - 1) * ld + r);
            v[q] = k < K ? x : f4zero();
        }
    }
}

template <bool KC>
__device__ __forceinline__ void tile_put(float* L, const f4 (&v)[4])
{
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int idx = t + 256 * q;
        if (KC)
            *reinterpret_cast<f4*>(L + (idx >> 3) * KLD + (idx & 7) * 4) = v[q];
        else
            *reinterpret_cast<f4*>(L + (idx >> 5) * RLD + (idx & 31) * 4) = v[q];
    }
}

// Fragment of rows rb..rb+15 for the 16-wide k-block h: lane (l16, g) gets
// the operand at row rb + l16, k = 16h + 4g + r in element r.
template <bool KC>
__device__ __forceinline__ f4 frag(const float* L, int rb, int h, int l16, int g)
{
    if (KC)
        return *reinterpret_cast<const f4*>(L + (rb + l16) * KLD + 16 * h + 4 * g);
    f4 v;
#pragma unroll
    for (int r = 0; r < 4; r++)
        v[r] = L[(16 * h + 4 * g + r) * RLD + rb + l16];
    return v;
}

template <bool AK, bool BK, int EPI>
__global__ __launch_bounds__(256, 2) void ffn_gemm_kernel(GemmArgs a)
{
    __shared__ __attribute__((aligned(16))) float lds[2][2][OPF];   // [stage][A, B]

    const int split = blockIdx.x / a.tiles;
    const int tile = blockIdx.x - split * a.tiles;
    const int m0 = (tile / a.tn) * GT;
    const int n0 = (tile % a.tn) * GT;
    const int kt0 = split * a.ktp;
    const int nkt = min(a.ktp, (a.K + GKT - 1) / GKT - kt0);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][j] = f4zero();

    f4 ra[4], rb[4];
    tile_fetch<AK>(a.A, a.lda, m0, a.M, kt0 * GKT, a.K, ra);
    tile_fetch<BK>(a.B, a.ldb, n0, a.N, kt0 * GKT, a.K, rb);
    tile_put<AK>(lds[0][0], ra);
    tile_put<BK>(lds[0][1], rb);
    __syncthreads();

    for (int kt = 0; kt < nkt; kt++) {
        const int st = kt & 1;
        // Next k-tile in flight during this one's MFMAs (past the split's end
        // it reads valid memory that is never used).
        tile_fetch<AK>(a.A, a.lda, m0, a.M, (kt0 + kt + 1) * GKT, a.K, ra);
        tile_fetch<BK>(a.B, a.ldb, n0, a.N, (kt0 + kt + 1) * GKT, a.K, rb);
        const float* LA = lds[st][0];
        const float* LB = lds[st][1];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            f4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                fa[i] = frag<AK>(LA, wm + 16 * i, h, l16, g);
#pragma unroll
            for (int j = 0; j < 4; j++)
                fb[j] = frag<BK>(LB, wn + 16 * j, h, l16, g);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[i][j] = mfma16(fb[j][r], fa[i][r], acc[i][j]);
        }
        tile_put<AK>(lds[st ^ 1][0], ra);
        tile_put<BK>(lds[st ^ 1][1], rb);
        __syncthreads();
    }

    // lane (l16, g), accumulator (i, j): row m0 + wm + 16i + l16, columns
    // n0 + wn + 16j + 4g .. +3.
    float* C = a.C + (long)split * a.sstride;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = m0 + wm + 16 * i + l16;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = n0 + wn + 16 * j + 4 * g;
            if (row < a.M && col < a.N)
                epi_apply<EPI>(acc[i][j], (long)row * a.ldc + col, C, a.G, a.pre);
        }
    }
}

// C = epilogue(sum over splits of P[s]), rows of N floats with stride ldc.
template <int EPI>
__global__ __launch_bounds__(256) void ffn_reduce_kernel(const float* __restrict__ P, int splits,
                                                         long sstride, int M, int N, float* C,
                                                         long ldc, const float* G, float* pre)
{
    const long n4 = (long)M * (N / 4);
    const long stride = (long)gridDim.x * 256;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const long row = i / (N / 4);
        const long col = (i - row * (N / 4)) * 4;
        const long off = row * N + col;
        f4 v = *reinterpret_cast<const f4*>(P + off);
        for (int s = 1; s < splits; s++)
            v += *reinterpret_cast<const f4*>(P + s * sstride + off);
        epi_apply<EPI>(v, row * ldc + col, C, G, pre);
    }
}

static int dev_cus()
{
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return cus;
}

int ffn_gemm_splits(int M, int N, int K)
{
    const long tiles = (long)((M + GT - 1) / GT) * ((N + GT - 1) / GT);
    const long slots = 2L * dev_cus();   // two workgroups per compute unit
    const int ktiles = (K + GKT - 1) / GKT;
    if (tiles >= slots / 2)
        return 1;
    int s = (int)std::min<long>(8, slots / tiles);
    s = std::min(s, std::max(1, ktiles / 4));   // at least 4 k-tiles per split
    return std::max(1, s);
}

size_t ffn_gemm_ws_floats(int M, int N, int K)
{
    const int s = ffn_gemm_splits(M, N, K);
    return s > 1 ? (size_t)s * M * N : 0;
}

template <bool AK, bool BK>
static void launch_main(int epi, dim3 grid, hipStream_t st, const GemmArgs& a)
{
    switch (epi) {
    case FFN_EPI_GELU:
        hipLaunchKernelGGL((ffn_gemm_kernel<AK, BK, FFN_EPI_GELU>), grid, dim3(256), 0, st, a);
        break;
    case FFN_EPI_DGELU:
        hipLaunchKernelGGL((ffn_gemm_kernel<AK, BK, FFN_EPI_DGELU>), grid, dim3(256), 0, st, a);
        break;
    case FFN_EPI_ACCUM:
        hipLaunchKernelGGL((ffn_gemm_kernel<AK, BK, FFN_EPI_ACCUM>), grid, dim3(256), 0, st, a);
        break;
    default:
        hipLaunchKernelGGL((ffn_gemm_kernel<AK, BK, FFN_EPI_STORE>), grid, dim3(256), 0, st, a);
    }
}

hipError_t ffn_gemm_launch(const FfnGemm& op, float* ws, hipStream_t st)
{
    if (op.M <= 0 || op.N <= 0 || op.K <= 0)
        return hipSuccess;
    if (!op.ak && op.bk)
        return hipErrorInvalidValue;   // no caller needs A row-contiguous with B k-contiguous
    const int s = ffn_gemm_splits(op.M, op.N, op.K);
    if (s > 1 && ws == nullptr)
        return hipErrorInvalidValue;
    const int ktiles = (op.K + GKT - 1) / GKT;
    GemmArgs a;
    a.A = op.A;
    a.B = op.B;
    a.lda = op.lda;
    a.ldb = op.ldb;
    a.M = op.M;
    a.N = op.N;
    a.K = op.K;
    a.tn = (op.N + GT - 1) / GT;
    a.tiles = ((op.M + GT - 1) / GT) * a.tn;
    a.ktp = (ktiles + s - 1) / s;
    const int used = (ktiles + a.ktp - 1) / a.ktp;   // splits that get k-tiles
    a.G = op.G;
    a.pre = op.pre;
    int epi = op.epi;
    if (used > 1) {
        a.C = ws;
        a.ldc = op.N;
        a.sstride = (long)op.M * op.N;
        epi = FFN_EPI_STORE;
    } else {
        a.C = op.C;
        a.ldc = op.ldc;
        a.sstride = 0;
    }
    const dim3 grid((unsigned)(a.tiles * used));
    {
        ProfScope ps(st, "ffn_gemm");
        if (op.ak && op.bk)
            launch_main<true, true>(epi, grid, st, a);
        else if (op.ak)
            launch_main<true, false>(epi, grid, st, a);
        else
            launch_main<false, false>(epi, grid, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || used == 1)
        return e;
    const long want = ((long)op.M * (op.N / 4) + 255) / 256;
    const unsigned blocks = (unsigned)std::max(1L, std::min(want, 8L * dev_cus()));
    ProfScope ps(st, "ffn_reduce");
    switch (op.epi) {
    case FFN_EPI_GELU:
        hipLaunchKernelGGL((ffn_reduce_kernel<FFN_EPI_GELU>), dim3(blocks), dim3(256), 0, st, ws,
                           used, a.sstride, op.M, op.N, op.C, op.ldc, op.G, op.pre);
        break;
    case FFN_EPI_DGELU:
        hipLaunchKernelGGL((ffn_reduce_kernel<FFN_EPI_DGELU>), dim3(blocks), dim3(256), 0, st, ws,
                           used, a.sstride, op.M, op.N, op.C, op.ldc, op.G, op.pre);
        break;
    case FFN_EPI_ACCUM:
        hipLaunchKernelGGL((ffn_reduce_kernel<FFN_EPI_ACCUM>), dim3(blocks), dim3(256), 0, st, ws,
                           used, a.sstride, op.M, op.N, op.C, op.ldc, op.G, op.pre);
        break;
    default:
        hipLaunchKernelGGL((ffn_reduce_kernel<FFN_EPI_STORE>), dim3(blocks), dim3(256), 0, st, ws,
                           used, a.sstride, op.M, op.N, op.C, op.ldc, op.G, op.pre);
    }
    return hipGetLastError();
}

} // namespace cxg
