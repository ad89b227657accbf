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
// Work is spread stream-K: two workgroups per compute unit, each taking an
// equal run of (tile, k-tile) units in tile-major order, so every shape keeps
// every unit equally busy (a tile count just above the unit count would
// otherwise leave most units idle for a second round).  A run computes whole
// tiles straight into C with the epilogue; a tile cut by a run boundary is
// left as partial tiles in the workspace (at most two per run, no waiting on
// other workgroups) and a fix-up kernel sums them in run order and applies
// the epilogue.
//
// A batch of same-shape products with element strides between them shares
// one launch: its tiles are numbered product-major and the runs cut across
// products like any other tiles.
//
// Requires E, F multiples of 4 and 16-byte aligned tensors (checked at the C
// ABI); any M.  Callers with other shapes (GPT's score matrices, whose
// sequence length S need not be a multiple of 4) store into padded rows and
// bound the operand reads separately (FfnGemm::Mc, Nc, Kc).
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
    float* part;       // 2 * P partial tiles of GT * GT floats (slot 0, 1 per workgroup)
    long lda, ldb, ldc;
    int M, N, K;
    int Mc, Nc, Kc;    // read extents (FfnGemm)
    int tn;            // tiles along N
    int Tb;            // tiles per product of the batch
    long sA, sB, sC;   // batch strides (elements)
    int T;             // tiles (all products)
    int KT;            // k-tiles per tile
    int P;             // workgroups
    long U;            // T * KT units
};

// Stream-K partition: the U (tile, k-tile) units, tile-major, are cut into P
// contiguous runs of equal length; run w is [sk_begin(w), sk_begin(w + 1)).
__host__ __device__ inline long sk_begin(long U, int P, int w) { return U * w / P; }

// The workgroup whose run holds unit u.
__device__ inline int sk_owner(long U, int P, long u)
{
    int w = (int)(u * P / U);
    while (w + 1 < P && sk_begin(U, P, w + 1) <= u)
        w++;
    while (w > 0 && sk_begin(U, P, w) > u)
        w--;
    return w;
}

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
// at P[row*ld + k].  Rows past `rows` are clamped onto the last row (KC) or
// the last 4-row group (their products land in C rows/columns that are never
// stored, or are multiplied by zeros of the other operand); k past K reads 0,
// and a row-contiguous operand's k-rows are clamped below Kc.
template <bool KC>
__device__ __forceinline__ void tile_fetch(const float* __restrict__ P, long ld, int r0, int rows,
                                           int k0, int K, int Kc, f4 (&v)[4])
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
            const f4 x = *reinterpret_cast<const f4*>(P + (long)min(k, Kc - 1) * ld + r);
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

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    const long ub = sk_begin(a.U, a.P, blockIdx.x);
    const long ue = sk_begin(a.U, a.P, blockIdx.x + 1);
    for (long u = ub; u < ue;) {
        // segment: k-tiles [ka, kb) of tile t
        const int t = (int)(u / a.KT);
        const int ka = (int)(u - (long)t * a.KT);
        const int kb = (int)min((long)a.KT, (long)ka + (ue - u));
        const int bt = t / a.Tb, tl = t - bt * a.Tb;   // product of the batch, its tile
        const int m0 = (tl / a.tn) * GT;
        const int n0 = (tl % a.tn) * GT;
        const int nkt = kb - ka;
        const float* Ab = a.A + bt * a.sA;
        const float* Bb = a.B + bt * a.sB;
        const long cb = bt * a.sC;

        f4 acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = f4zero();

        // (LDS is free here: the previous segment's last reads precede its
        // final barrier.)
        f4 ra[4], rb[4];
        tile_fetch<AK>(Ab, a.lda, m0, a.Mc, ka * GKT, a.K, a.Kc, ra);
        tile_fetch<BK>(Bb, a.ldb, n0, a.Nc, ka * GKT, a.K, a.Kc, rb);
        tile_put<AK>(lds[0][0], ra);
        tile_put<BK>(lds[0][1], rb);
        __syncthreads();

        for (int kt = 0; kt < nkt; kt++) {
            const int st = kt & 1;
            // Next k-tile in flight during this one's MFMAs (past the
            // segment's end it reads valid memory that is never used).
            tile_fetch<AK>(Ab, a.lda, m0, a.Mc, (ka + kt + 1) * GKT, a.K, a.Kc, ra);
            tile_fetch<BK>(Bb, a.ldb, n0, a.Nc, (ka + kt + 1) * GKT, a.K, a.Kc, rb);
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

        // lane (l16, g), accumulator (i, j): tile row wm + 16i + l16, columns
        // wn + 16j + 4g .. +3.
        if (ka == 0 && kb == a.KT) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = m0 + wm + 16 * i + l16;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int col = n0 + wn + 16 * j + 4 * g;
                    if (row < a.M && col < a.N)
                        epi_apply<EPI>(acc[i][j], cb + (long)row * a.ldc + col, a.C, a.G,
                                       a.pre);
                }
            }
        } else {
            // A piece of a tile shared with neighbouring runs: slot 0 if it
            // opens this run, else slot 1 (then it closes the run).
            float* P = a.part + ((long)2 * blockIdx.x + (u == ub ? 0 : 1)) * (GT * GT);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    *reinterpret_cast<f4*>(P + (wm + 16 * i + l16) * GT + wn + 16 * j + 4 * g) =
                        acc[i][j];
        }
        u += nkt;
    }
}

// Tiles whose units span more than one run: sum the pieces in run order and
// apply the epilogue.  Four workgroups per tile (32 rows each, four float4
// per thread, so the pieces' loads of many tiles are in flight at once);
// whole tiles return at once.
template <int EPI>
__global__ __launch_bounds__(256) void ffn_fixup_kernel(GemmArgs a)
{
    const int t = (int)(blockIdx.x >> 2), quarter = (int)(blockIdx.x & 3);
    const long u0 = (long)t * a.KT;
    const int wa = sk_owner(a.U, a.P, u0);
    const int wb = sk_owner(a.U, a.P, u0 + a.KT - 1);
    if (wa == wb)
        return;
    // thread's float4s: q = quarter * 1024 + threadIdx.x + 256 e: tile row q / 32,
    // column 4 (q % 32)
    constexpr int NE = GT * GT / 4 / 4 / 256;
    f4 v[NE];
#pragma unroll
    for (int e = 0; e < NE; e++)
        v[e] = f4zero();
    for (int w = wa; w <= wb; w++) {
        const long b = sk_begin(a.U, a.P, w);
        if (sk_begin(a.U, a.P, w + 1) == b)
            continue;   // empty run
        const float* src = a.part + ((long)2 * w + (b >= u0 ? 0 : 1)) * (GT * GT) +
                           (long)quarter * (GT * GT / 4);
        f4 x[NE];
#pragma unroll
        for (int e = 0; e < NE; e++)
            x[e] = *reinterpret_cast<const f4*>(src + (threadIdx.x + 256 * e) * 4);
#pragma unroll
        for (int e = 0; e < NE; e++)
            v[e] += x[e];
    }
    const int bt = t / a.Tb, tl = t - bt * a.Tb;
    const int m0 = (tl / a.tn) * GT;
    const int n0 = (tl % a.tn) * GT;
    const long cb = bt * a.sC;
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const int q = quarter * (GT * GT / 16) + threadIdx.x + 256 * e;
        const int row = m0 + (q >> 5), col = n0 + (q & 31) * 4;
        if (row < a.M && col < a.N)
            epi_apply<EPI>(v[e], cb + (long)row * a.ldc + col, a.C, a.G, a.pre);
    }
}

static int dev_cus()
{
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return cus;
}

// Two workgroups per compute unit (LDS and registers allow two; one alone
// leaves the MFMA pipe idle half the time), or one per unit of work.
static int sk_wgs(long U) { return (int)std::min<long>(2L * dev_cus(), U); }

size_t ffn_gemm_ws_floats(int M, int N, int K, int batch)
{
    const long U = (long)std::max(batch, 1) * ((M + GT - 1) / GT) * ((N + GT - 1) / GT) *
                   ((K + GKT - 1) / GKT);
    return (size_t)2 * sk_wgs(U) * GT * GT;
}

template <bool AK, bool BK>
static void launch_main(int epi, dim3 grid, hipStream_t st, const GemmArgs& a)
{
    switch (epi) {
    case FFN_EPI_GELU:
        CXG_LAUNCH((ffn_gemm_kernel<AK, BK, FFN_EPI_GELU>), grid, dim3(256), 0, st, a);
        break;
    case FFN_EPI_DGELU:
        CXG_LAUNCH((ffn_gemm_kernel<AK, BK, FFN_EPI_DGELU>), grid, dim3(256), 0, st, a);
        break;
    case FFN_EPI_ACCUM:
        CXG_LAUNCH((ffn_gemm_kernel<AK, BK, FFN_EPI_ACCUM>), grid, dim3(256), 0, st, a);
        break;
    default:
        CXG_LAUNCH((ffn_gemm_kernel<AK, BK, FFN_EPI_STORE>), grid, dim3(256), 0, st, a);
    }
}

template <int EPI>
static void launch_fixup(dim3 grid, hipStream_t st, const GemmArgs& a)
{
    CXG_LAUNCH((ffn_fixup_kernel<EPI>), grid, dim3(256), 0, st, a);
}

hipError_t ffn_gemm_launch(const FfnGemm& op, float* ws, hipStream_t st)
{
    if (op.M <= 0 || op.N <= 0 || op.K <= 0)
        return hipSuccess;
    if ((!op.ak && op.bk) || ws == nullptr)
        return hipErrorInvalidValue;   // no caller needs A row-contiguous with B k-contiguous
    GemmArgs a;
    a.A = op.A;
    a.B = op.B;
    a.C = op.C;
    a.G = op.G;
    a.pre = op.pre;
    a.part = ws;
    a.lda = op.lda;
    a.ldb = op.ldb;
    a.ldc = op.ldc;
    a.M = op.M;
    a.N = op.N;
    a.K = op.K;
    a.Mc = op.Mc > 0 ? op.Mc : op.M;
    a.Nc = op.Nc > 0 ? op.Nc : op.N;
    a.Kc = op.Kc > 0 ? op.Kc : op.K;
    a.tn = (op.N + GT - 1) / GT;
    a.Tb = ((op.M + GT - 1) / GT) * a.tn;
    a.sA = op.sA;
    a.sB = op.sB;
    a.sC = op.sC;
    a.T = std::max(op.batch, 1) * a.Tb;
    a.KT = (op.K + GKT - 1) / GKT;
    a.U = (long)a.T * a.KT;
    a.P = sk_wgs(a.U);
    {
        ProfScope ps(st, "ffn_gemm");
        const dim3 grid((unsigned)a.P);
        if (op.ak && op.bk)
            launch_main<true, true>(op.epi, grid, st, a);
        else if (op.ak)
            launch_main<true, false>(op.epi, grid, st, a);
        else
            launch_main<false, false>(op.epi, grid, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    bool split = false;   // does any run boundary fall inside a tile?
    for (int w = 1; w < a.P && !split; w++)
        split = sk_begin(a.U, a.P, w) % a.KT != 0;
    if (!split)
        return hipSuccess;
    ProfScope ps(st, "ffn_fixup");
    const dim3 grid((unsigned)a.T * 4);
    switch (op.epi) {
    case FFN_EPI_GELU: launch_fixup<FFN_EPI_GELU>(grid, st, a); break;
    case FFN_EPI_DGELU: launch_fixup<FFN_EPI_DGELU>(grid, st, a); break;
    case FFN_EPI_ACCUM: launch_fixup<FFN_EPI_ACCUM>(grid, st, a); break;
    default: launch_fixup<FFN_EPI_STORE>(grid, st, a);
    }
    return hipGetLastError();
}

} // namespace cxg
