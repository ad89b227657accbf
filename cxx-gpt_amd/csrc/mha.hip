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
// In both, the second split numbers its 16-row groups in reverse (waves w and
// w+4 share a SIMD), and 16x16 blocks that lie wholly above the causal
// diagonal are skipped, so a diagonal tile costs each SIMD at most 3 of the 4
// block-columns of work a full tile does.
// Jobs are numbered (tile * B*H + bh): heavy causal tiles first, and when B*H
// is a multiple of 8 all tiles of a head share an XCD (and its L2), since
// workgroups are dealt to the 8 XCDs round-robin.
#include "common.hpp"

#include <type_traits>
#include "launch.hpp"

#include <math.h>

namespace cxg {

constexpr int MHA_BM = 64;   // query rows per tile
// Forward online softmax: the reference max moves when a score exceeds it by
// more than this (log2 units), so unnormalised probabilities stay <= 2^8.
constexpr float kLazyRescale = 8.0f;
constexpr int MHA_BN = 64;   // key rows per tile

// Copy the rotary frequencies into LDS (by one lane, with uniform indices so
// the kernel argument is read with scalar loads); the caller synchronises.
__device__ __forceinline__ void rope_table(float* __restrict__ w, const MhaRope& rp)
{
    if (threadIdx.x == 0)
#pragma unroll
        for (int i = 0; i < 128; i++)
            w[i] = rp.w[i];
}

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
    // Whole-width heads (Dh == DHP, 16-byte aligned rows): the same units
    // through a buffer descriptor whose range ends with row S-1 of the head,
    // so rows past S read 0.  voff[i]: byte offset of unit i within a tile
    // (tile-invariant, formed once); soff: the tile's first row, in bytes.
    struct Offs {
        unsigned v[UPT];
    };
    __device__ __forceinline__ static Offs offsets(long rs, int tid)
    {
        Offs o;
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = min(tid + i * NT, NU - 1);
            const int row = u / CPR, c = 4 * (u - row * CPR);
            o.v[i] = (unsigned)((row * rs + c) * 4);
        }
        return o;
    }
    __device__ __forceinline__ void loadb(__amdgpu_buffer_rsrc_t rsrc, const Offs& o, unsigned soff)
    {
#pragma unroll
        for (int i = 0; i < UPT; i++)
            r[i] = buffer_load_f4s(rsrc, o.v[i], soff);
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
    // row-major like store(), each row rotated (positions row0 + row, clamped
    // to S-1 as the load was; columns past Dh hold zeros or repeats that the
    // consumers mask)
    template <int LD>
    __device__ __forceinline__ void store_rope(float* __restrict__ T, int tid, int row0, int S,
                                               const float* rw) const
    {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + i * NT;
            if (NU % NT == 0 || u < NU) {
                const int row = u / CPR, c = 4 * (u - row * CPR);
                *reinterpret_cast<f4*>(&T[row * LD + c]) =
                    rope4(r[i], min(row0 + row, S - 1), c, rw, 1.0f);
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

// Persistent grids: workgroup w of G takes job r*G + w in even rounds r and
// r*G + G-1-w in odd rounds.  Jobs are numbered heaviest first, so the
// serpentine order pairs a workgroup's heavy early jobs with light late ones.
__device__ __forceinline__ int snake_job(int r)
{
    const int G = gridDim.x, w = blockIdx.x;
    return r * G + ((r & 1) ? G - 1 - w : w);
}

// Job of workgroup w in a grid of one job per workgroup, N jobs on C compute
// units holding two workgroups each (C < N <= 2C).  Workgroup w + C is
// placed on the compute unit of workgroup w (the dispatcher fills every
// compute unit once before it doubles up), so the P = N - C compute units
// that receive two workgroups take a heavy and a light job each (indices
// summing to a constant) and the other C - P take the C - P heaviest jobs
// alone.  Two resident jobs overlap one another's load and merge phases.
__device__ __forceinline__ int paired_job(int w, int N, int C)
{
    const int P = N - C;
    if (w >= C)
        return N - 1 - (w - C);
    return w >= P ? w - P : (C - P) + w;
}

// Row (or key) group of wave `wave` in a workgroup of 4 or 8 waves.  The
// waves of a workgroup are dealt to the compute unit's four SIMDs
// round-robin, so waves w and w+4 share a SIMD; the second four take the
// 16-row groups in reverse order, so that in a tile on the causal diagonal,
// where a group's share of unmasked blocks grows with its index, the SIMDs
// get nearly equal work (3, 3, 2, 2 of the 10 unmasked 16x16 blocks).
__device__ __forceinline__ int pair_group(int wave)
{
    return (wave & 4) ? 3 - (wave & 3) : (wave & 3);
}

// Wave index as a scalar (wave-uniform) value, so that branches on it are
// uniform branches.
__device__ __forceinline__ int wave_id(int tid)
{
    return __builtin_amdgcn_readfirstlane(tid >> 6);
}

// threadIdx.x, re-read per job behind an empty asm so that the compiler does
// not hoist the job body's thread-dependent address arithmetic out of the job
// loop (holding it across jobs costs registers).
__device__ __forceinline__ int job_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Persistent forward kernel.  Job qi*BH + bh is query tile qb = nqb-1-qi of
// head bh (longest first); a workgroup takes jobs in serpentine order and,
// once the last key tile of a job has been through its math, requests the
// next job's Q rows and first two K/V tiles, so that they arrive while the
// current job merges its key splits and writes O.
//
// PREP (statistics pass, DHP <= 64 only): the backward's pre-pass rides along,
// Di = rowsum(dO * O) of the job's rows into Di and their dQ rows zeroed, so
// the reference-signature backward needs no separate pre-pass launch.
template <int DHP, int NSPLIT, bool VEC, bool WRITE_O, bool ROPE, bool PREP = false,
          bool BUF = false>
__global__ __launch_bounds__(256 * NSPLIT, DHP <= 64 ? 4 : 1) void mha_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int S, int H, int Dh, int BH, int nqb,
    float qscale, int pair_cus, const MhaRope rope, const float* __restrict__ pO,
    const float* __restrict__ pdO, float* __restrict__ pDi, float* __restrict__ pdQ)
{
    static_assert(!PREP || (!WRITE_O && DHP <= 64 && NSPLIT == 2), "pre-pass rides on 512-thread statistics passes");
    static_assert(!BUF || VEC, "buffer loads need aligned whole-width rows");
    using SM = FwdSmem<DHP, NSPLIT>;
    constexpr int NT = 256 * NSPLIT;
    constexpr int KS = SM::KS, MS = SM::MS;
    constexpr int NDT = DHP / 16;
    constexpr int NKT = 4 / NSPLIT;   // 16-key blocks per wave per tile
    __shared__ __attribute__((aligned(16))) float smem[SM::FLOATS];
    __shared__ float rope_w[ROPE ? 128 : 1];
    if constexpr (ROPE) {
        rope_table(rope_w, rope);
        __syncthreads();
    }

    const int njobs = nqb * BH;
    const long rs = (long)H * Dh;
    struct Job {
        int bh, qb;
        long base;
    };
    // BUF: descriptors over a head's rows 0..S-1 (built where used, in scalar
    // registers: kept in the job record they would go to scratch memory)
    const unsigned head_bytes = (unsigned)(((long)(S - 1) * rs + Dh) * 4);
    auto job_of = [&](int job) {
        Job j;
        const int qi = job / BH;
        j.bh = job - qi * BH;
        j.qb = nqb - 1 - qi;
        const int b = j.bh / H, h = j.bh - b * H;
        j.base = (long)b * S * rs + (long)h * Dh;
        return j;
    };

    // B operand of S^T = K Q^T: lane holds Q[myq][16*dt + 4*g + r], pre-scaled
    // by scale*log2(e) so scores land in the exp2 domain; zero past Dh.  The
    // rows are loaded raw (clamped) and masked and scaled at the start of the
    // job, so that the loads stay in flight with the K/V loads.
    f4 qreg[NDT];
    // Narrow heads (DB) run a four-deep pipeline: two register stages, loaded
    // from global memory three tiles ahead of use, feed two LDS buffers; tile
    // kb+1 is written to LDS while tile kb is consumed, one barrier per tile.
    // Wider heads use one LDS buffer (two barriers per tile) and one register
    // stage (none for the widest).
    TileRegs<DHP, MHA_BN, NT, VEC> kr, vr, kr1, vr1;
    using Offs = typename TileRegs<DHP, MHA_BN, NT, VEC>::Offs;
    Offs koffs;
    if constexpr (BUF)
        koffs = TileRegs<DHP, MHA_BN, NT, VEC>::offsets(rs, threadIdx.x);
    auto load_kv = [&](TileRegs<DHP, MHA_BN, NT, VEC>& kx, TileRegs<DHP, MHA_BN, NT, VEC>& vx,
                       const Job& j, int kb) {
        if constexpr (BUF) {
            const unsigned so = (unsigned)((long)kb * MHA_BN * rs * 4);
            kx.loadb(buf_rsrc_n(K + j.base, head_bytes), koffs, so);
            if (WRITE_O)
                vx.loadb(buf_rsrc_n(V + j.base, head_bytes), koffs, so);
        } else {
            const int tid = job_tid();
            kx.load(K, j.base, rs, kb * MHA_BN, S, Dh, tid);
            if (WRITE_O)
                vx.load(V, j.base, rs, kb * MHA_BN, S, Dh, tid);
        }
    };
    // A job's first loads: Q rows and key tile 0 (and, for the single-stage
    // pipeline, nothing more; the double-buffered one requests tiles 1 and 2
    // once tile 0 is in LDS, so that every workgroup's first tile arrives
    // ahead of the later ones).
    // PREP: O and dO of the job's rows, 8 threads a row (row tid/8, f4 units
    // tid%8 + 8i), loaded with the job's first loads; their dot products are
    // formed once key tile 0 is in LDS, before the next job's loads reuse them.
    constexpr int PUPR = DHP / 4;                  // f4 units per row
    constexpr int PPU = PUPR >= 8 ? PUPR / 8 : 1;  // units per thread
    f4 po[PREP ? PPU : 1], pd[PREP ? PPU : 1];
    float pdot = 0.0f;
    auto load_first = [&](const Job& j) {
        const int tid = job_tid(), lane = tid & 63, wave = wave_id(tid);
        const int l16 = lane & 15, g = lane >> 4, qg = pair_group(wave);
        if constexpr (BUF) {
            // rows past S read 0 (masked at the job start all the same)
            const unsigned vo = (unsigned)(((qg * 16 + l16) * rs + 4 * g) * 4);
            const unsigned so = (unsigned)((long)j.qb * MHA_BM * rs * 4);
            const __amdgpu_buffer_rsrc_t rq = buf_rsrc_n(Q + j.base, head_bytes);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                qreg[dt] = buffer_load_f4s(rq, vo + 64 * dt, so);
        } else {
            const int q = min(j.qb * MHA_BM + qg * 16 + l16, S - 1);
            const float* qrow = Q + j.base + (long)q * rs;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                qreg[dt] = load4c<VEC>(qrow, 16 * dt + 4 * g, Dh);
        }
        load_kv(kr, vr, j, 0);
        if constexpr (PREP) {
            const int prow = min(j.qb * MHA_BM + (tid >> 3), S - 1);
            const long off = j.base + (long)prow * rs;
#pragma unroll
            for (int i = 0; i < PPU; i++) {
                po[i] = load4c<VEC>(pO + off, 4 * ((tid & 7) + 8 * i), Dh);
                pd[i] = load4c<VEC>(pdO + off, 4 * ((tid & 7) + 8 * i), Dh);
            }
        }
    };

    // The grid never exceeds the job count.  pair_cus > 0: one job per
    // workgroup, two workgroups per compute unit (paired_job).
    Job jc = job_of(pair_cus > 0 ? paired_job(blockIdx.x, njobs, pair_cus) : snake_job(0));
    load_first(jc);
#pragma nounroll
    for (int r = 0;; r++) {
        const int jn = snake_job(r + 1);
        const bool more = jn < njobs;
        const Job jnext = job_of(more ? jn : 0);

        const int tid = job_tid(), lane = tid & 63, wave = wave_id(tid);
        const int l16 = lane & 15, g = lane >> 4;
        const int qg = pair_group(wave), ks = wave >> 2;
        const int qb = jc.qb, bh = jc.bh;
        const long base = jc.base;
        const int myq = qb * MHA_BM + qg * 16 + l16;
        const bool qok = myq < S;
        const int nkb = qb + 1;   // causal: key tiles 0..qb (MHA_BM == MHA_BN)

        f4 oacc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            oacc[dt] = f4zero();
        // m_run: the lane's reference maximum (its query row's running max at
        // the last rescale); l_run and oacc are relative to it.  A split that
        // never sees a key keeps -1e30 and drops out of the merge.
        float m_run = -1e30f, l_run = 0.0f;
        // kb: the key tile held in (kx, vx); K is rotated on its way to LDS
        // under ROPE.
        auto store_kv = [&](const TileRegs<DHP, MHA_BN, NT, VEC>& kx,
                            const TileRegs<DHP, MHA_BN, NT, VEC>& vx, float* buf, int kb) {
            if constexpr (ROPE)
                kx.template store_rope<KS>(buf, tid, kb * MHA_BN, S, rope_w);
            else
                kx.template store<KS>(buf, tid);
            if (WRITE_O)
                vx.template store<KS>(buf + MHA_BN * KS, tid);
        };
        // One key tile of math on the tiles in LDS (Ks, Vs: [key][d], row stride
        // KS), over the first NA of the wave's NKT key blocks (the others lie
        // wholly above the causal diagonal).
        auto tile_math = [&](const float* __restrict__ Ks, const float* __restrict__ Vs, int kb,
                             auto na) __attribute__((always_inline)) {
            constexpr int NA = decltype(na)::value;
            const int k0 = kb * MHA_BN;
            // S^T block kt of this wave: lane holds query l16, keys k0 + 16*kt + 4*g + r.
            // The NA key blocks run as interleaved accumulation chains.  The
            // accumulators start at -m_run, so scores come out relative to
            // the lane's reference (raw on the first tile, which sets it).
            const bool first = kb == 0;   // wave-uniform
            const f4 init = f4splat(first ? 0.0f : -m_run);
            f4 sacc[NA];
#pragma unroll
            for (int kk = 0; kk < NA; kk++)
                sacc[kk] = init;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                for (int kk = 0; kk < NA; kk++) {
                    const int kt = ks * NKT + kk;
                    const f4 kv = *reinterpret_cast<const f4*>(&Ks[(16 * kt + l16) * KS + 16 * dt + 4 * g]);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        sacc[kk] = mfma16(kv[r], qreg[dt][r], sacc[kk]);
                }
            }
            if (kb == qb) {   // diagonal tile: causal mask key > query
#pragma unroll
                for (int kk = 0; kk < NA; kk++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (k0 + 16 * (ks * NKT + kk) + 4 * g + r > myq)
                            sacc[kk][r] = -INFINITY;
            }
            float mloc = -INFINITY;
#pragma unroll
            for (int kk = 0; kk < NA; kk++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    mloc = fmaxf(mloc, sacc[kk][r]);
            // Lazy rescaling: the reference moves only on the first tile or
            // when a score of the wave exceeds its row's reference by more
            // than 2^kLazyRescale (so p <= 2^8 and no sum can overflow).  The
            // common case then needs no row max, no subtraction and no
            // rescale of the accumulators; each VALU instruction here costs
            // matrix-pipe time, since VALU and MFMA do not overlap on a SIMD.
            float psum = 0.0f;
            if (first || __builtin_amdgcn_ballot_w64(mloc > kLazyRescale) != 0) {
                mloc = xrow_max(mloc);   // every row has an unmasked key in a live block
                const float d = first ? mloc : fmaxf(mloc, 0.0f);
                const float alpha = first ? 0.0f : fast_exp2(-d);
                m_run = (first ? 0.0f : m_run) + d;
#pragma unroll
                for (int kk = 0; kk < NA; kk++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float p = fast_exp2(sacc[kk][r] - d);
                        sacc[kk][r] = p;
                        psum += p;
                    }
                l_run = l_run * alpha + psum;
                if (WRITE_O && !first)   // the first tile's accumulators are still zero
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++)
                        oacc[dt] = oacc[dt] * alpha;
            } else {
#pragma unroll
                for (int kk = 0; kk < NA; kk++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float p = fast_exp2(sacc[kk][r]);
                        sacc[kk][r] = p;
                        psum += p;
                    }
                l_run += psum;
            }
            if (WRITE_O) {
                // O^T += V^T P^T: A = V^T[d = 16dt + l16][key = 16kt + 4g + r], read
                // as single floats from the row-major V tile; B = P^T from sacc.
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
                    f4 acc = oacc[dt];
#pragma unroll
                    for (int kk = 0; kk < NA; kk++) {
                        const int kt = ks * NKT + kk;
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc = mfma16(Vs[(16 * kt + 4 * g + r) * KS + 16 * dt + l16], sacc[kk][r], acc);
                    }
                    oacc[dt] = acc;
                }
            }
        };
        // A key tile: off the diagonal every block is live; on it (two key
        // splits) key block kt = ks*NKT + kk is live for kt <= qg, a prefix of
        // the wave's blocks, and the rest are skipped (a block of scores that
        // are all masked leaves the online-softmax state unchanged), down to
        // the whole tile.
        auto tile = [&](const float* __restrict__ Ks, const float* __restrict__ Vs, int kb)
                        __attribute__((always_inline)) {
            if (NSPLIT == 1 || kb != qb) {
                tile_math(Ks, Vs, kb, ic<NKT>{});
            } else {
                const int na = qg - ks * NKT + 1;
                if (na >= NKT)
                    tile_math(Ks, Vs, kb, ic<NKT>{});
                else if (na == 1)
                    tile_math(Ks, Vs, kb, ic<1>{});
            }
        };
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            // BUF: rows past S were read as 0 and there are no columns past Dh
            f4 q = BUF ? qreg[dt] : mask4(qreg[dt], 16 * dt + 4 * g, Dh, qok);
            if constexpr (ROPE)
                q = rope4(q, min(myq, S - 1), 16 * dt + 4 * g, rope_w, 1.0f);
            qreg[dt] = q * qscale;
        }
        if constexpr (SM::DB) {
            store_kv(kr, vr, smem, 0);
            __builtin_amdgcn_sched_barrier(0);
            // Tiles past the last one repeat it (clamped index), so these
            // loads are the same on every path and the waits stay tight.
            load_kv(kr1, vr1, jc, min(1, nkb - 1));
            load_kv(kr, vr, jc, min(2, nkb - 1));
            __syncthreads();
            if constexpr (PREP) {
                // this thread's part of Di (columns past Dh masked)
                pdot = 0.0f;
#pragma unroll
                for (int i = 0; i < PPU; i++) {
                    const int c = 4 * ((tid & 7) + 8 * i);
                    const f4 o = mask4(po[i], c, Dh, true), d = mask4(pd[i], c, Dh, true);
                    pdot += o[0] * d[0] + o[1] * d[1] + o[2] * d[2] + o[3] * d[3];
                }
            }
            // Iteration kb < nkb-1: the math of tile kb (LDS buffer kb&1),
            // then registers (kx, vx), holding tile kb+1, go to buffer
            // (kb+1)&1 (last read in iteration kb-1) and are refilled with
            // tile kb+3.
            auto step = [&](TileRegs<DHP, MHA_BN, NT, VEC>& kx,
                            TileRegs<DHP, MHA_BN, NT, VEC>& vx, int kb) __attribute__((always_inline)) {
                const float* cur = smem + (kb & 1) * SM::TILES;
                __builtin_amdgcn_s_setprio(1);
                tile(cur, cur + MHA_BN * KS, kb);
                __builtin_amdgcn_s_setprio(0);
                store_kv(kx, vx, smem + ((kb + 1) & 1) * SM::TILES, kb + 1);
                // Keep the refill below the LDS writes: issued earlier, the
                // wait for the old data would include the new loads.
                __builtin_amdgcn_sched_barrier(0);
                if (kb + 3 < nkb)
                    load_kv(kx, vx, jc, kb + 3);
                __syncthreads();
            };
            int kb = 0;
            for (; kb + 2 < nkb; kb += 2) {
                step(kr1, vr1, kb);
                step(kr, vr, kb + 1);
            }
            if (kb + 1 < nkb)
                step(kr1, vr1, kb++);
            // The last key tile; then the next job's first loads (all register
            // stages are free by then).
            const float* cur = smem + (kb & 1) * SM::TILES;
            __builtin_amdgcn_s_setprio(1);
            tile(cur, cur + MHA_BN * KS, kb);
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);   // not above the math: it reads qreg
            if (more)
                load_first(jnext);
            __syncthreads();
        } else {
            constexpr bool PREFETCH = DHP <= 128;
            for (int kb = 0; kb < nkb; kb++) {
                if (!PREFETCH && kb > 0)
                    load_kv(kr, vr, jc, kb);
                __syncthreads();
                store_kv(kr, vr, smem, kb);
                __syncthreads();
                if (PREFETCH && kb + 1 < nkb)
                    load_kv(kr, vr, jc, kb + 1);
                tile(smem, smem + MHA_BN * KS, kb);
                if (kb + 1 == nkb && more) {   // next job's first loads, as above
                    __builtin_amdgcn_sched_barrier(0);
                    load_first(jnext);
                }
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
            if (ks == 0) {
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
        }
        if (ks == 0 && qok) {
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
        if constexpr (PREP) {
            float dsum = pdot;
            dsum += lane_xor16<1>(dsum);
            dsum += lane_xor16<2>(dsum);
            dsum += lane_xor16<4>(dsum);
            const int prow = qb * MHA_BM + (tid >> 3);
            if (prow < S) {
                if ((tid & 7) == 0)
                    pDi[(long)bh * S + prow] = dsum;
                float* drow = pdQ + base + (long)prow * rs;
#pragma unroll
                for (int i = 0; i < PPU; i++)
                    store4<VEC>(drow, 4 * ((tid & 7) + 8 * i), Dh, f4zero());
            }
        }
        if (!more)
            break;
        jc = jnext;
        __syncthreads();   // the merge records are consumed
    }
}

// ----------------------------------------------------------------------------
// backward pre-pass: Di = rowsum(dO * O) (the reference's gs, kernel_test.cpp:76-78)
// and dQ = 0.  16 lanes per (row, head) segment.
// ----------------------------------------------------------------------------
template <bool VEC, bool ZERO, int TPR>
__global__ __launch_bounds__(256) void mha_bwd_prep_kernel(
    const float* __restrict__ O, const float* __restrict__ dO, float* __restrict__ Di,
    float* __restrict__ dQ, int S, int H, int Dh, long nseg)
{
    // TPR threads per (row, head) segment: 16, or a whole wave for wide heads
    const long seg = ((long)blockIdx.x * 256 + threadIdx.x) / TPR;
    const int sub = threadIdx.x & (TPR - 1);
    const bool ok = seg < nseg;
    float acc = 0.0f;
    if (ok) {
        const long off = seg * Dh;   // segment (b*S + s)*H + h starts at seg*Dh
        for (int c = 4 * sub; c < Dh; c += 4 * TPR) {
            const f4 o = load4<VEC>(O + off, c, Dh, true);
            const f4 d = load4<VEC>(dO + off, c, Dh, true);
            acc += o[0] * d[0] + o[1] * d[1] + o[2] * d[2] + o[3] * d[3];
            if (ZERO)
                store4<VEC>(dQ + off, c, Dh, f4zero());
        }
    }
    acc = row16_sum(acc);
    if (TPR == 64)
        acc = xrow_sum(acc);
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

// Persistent backward kernel.  Job kb*BH + bh is key tile kb of head bh; a
// workgroup takes jobs in serpentine order and, once the last query tile of a
// job has been through its key-side work, requests the next job's K/V rows
// and first query tiles, so that they arrive while the current job finishes
// its dQ jobs and dK/dV reduction.
//
// The softmax scale is folded into V (so dP and dS come out scaled) and Di
// once per job, which removes a multiply per dQ atomic and per dK element;
// scale * log2(e) is folded into the K operand of S, and the S and dP
// accumulators start at -lse * log2(e) and -Di, so that P = exp2(S) and
// dS = P * dP need no further arithmetic.
// BUF (whole-width heads, double-buffered path): Q/dO/K/V rows through buffer
// descriptors over the head's rows 0..S-1 with scalar row offsets, and dQ
// atomics through one whose range drops rows past S, so neither loads nor
// atomics spend vector instructions on addresses or masks.
template <int DHP, int BM, int NSPLIT, bool VEC, bool ROPE, bool BUF = false, bool IPREP = false>
__global__ __launch_bounds__(256 * NSPLIT) void mha_bwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ Di,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int S, int H, int Dh,
    int BH, int nkb, float scale, float c2, const MhaRope rope, const MhaIPrep ip)
{
    using SM = BwdSmem<DHP, BM>;
    static_assert(!BUF || (VEC && SM::DB), "buffer loads need the double-buffered aligned path");
    // The pre-pass inside the kernel: query tiles and key tiles coincide (a
    // job's first query tile is its own key tile) and the grid is persistent.
    static_assert(!IPREP || (BUF && BM == MHA_BN && NSPLIT == 2 && DHP == 64 && !ROPE),
                  "in-kernel pre-pass: whole-width Dh = 64 heads, 64-row tiles");
    constexpr int NT = 256 * NSPLIT;
    constexpr int NW = NT / 64;
    constexpr int NDT = DHP / 16;
    constexpr int NQT = BM / 16;        // 16-row query blocks per tile
    constexpr int NQW = NQT / NSPLIT;   // ... per wave
    constexpr int QS = SM::QS, TS = SM::TS;
    static_assert(NQW >= 1, "query split too fine for BM");
    // Eight waves over four query blocks (two per wave): query/key blocks on
    // the far side of the causal diagonal are skipped in the key-side and dQ
    // products, and the dQ blocks are paired across SIMDs.
    constexpr bool SKIP = NW == 8 && NQT == 4;
    __shared__ __attribute__((aligned(16))) float smem[SM::FLOATS];
    __shared__ float rope_w[ROPE ? 128 : 1];
    if constexpr (ROPE) {
        rope_table(rope_w, rope);
        __syncthreads();
    }
    float* Kt = smem;
    // Stage i: Qs [BM][QS], dOs [BM][QS], dSs [BM][TS], lse_s [BM], di_s [BM].
    auto stage = [&](int i) { return smem + DHP * TS + i * SM::STAGE; };

    const int njobs = nkb * BH;
    const int nqb = (S + BM - 1) / BM;
    const long rs = (long)H * Dh;

    // Job geometry.
    struct Job {
        int bh, k0, qb0;
        long base;
    };
    auto job_of = [&](int job) {
        Job j;
        const int kb = job / BH;
        j.bh = job - kb * BH;
        const int b = j.bh / H, h = j.bh - b * H;
        j.base = (long)b * S * rs + (long)h * Dh;
        j.k0 = kb * MHA_BN;
        j.qb0 = j.k0 / BM;
        return j;
    };

    // A query tile in registers on its way to LDS: Q and dO rows, and the
    // tile's lse and Di entries (negated on their way to LDS, lse in log2
    // units, Di scaled).
    struct QTile {
        TileRegs<DHP, BM, NT, VEC> q, d;
        TileRegs<DHP, BM, NT, VEC> o;   // in-kernel pre-pass: O rows, for the tile's Di
        float lse, di;
    };
    // BUF: bytes from a head's first element to the end of its row S-1
    const unsigned head_bytes = (unsigned)(((long)(S - 1) * rs + Dh) * 4);
    using Offs = typename TileRegs<DHP, BM, NT, VEC>::Offs;
    Offs qoffs;
    if constexpr (BUF)
        qoffs = TileRegs<DHP, BM, NT, VEC>::offsets(rs, threadIdx.x);
    auto load_q = [&](QTile& t, const Job& j, int q0) {
        const int tid = job_tid();
        if constexpr (BUF) {
            const unsigned so = (unsigned)((long)q0 * rs * 4);
            t.q.loadb(buf_rsrc_n(Q + j.base, head_bytes), qoffs, so);
            t.d.loadb(buf_rsrc_n(dO + j.base, head_bytes), qoffs, so);
        } else {
            t.q.load(Q, j.base, rs, q0, S, Dh, tid);
            t.d.load(dO, j.base, rs, q0, S, Dh, tid);
        }
        // Every thread loads (rows past S repeat row S-1, their P is masked to
        // 0); threads tid < BM store.  No use of the loaded data here (lse is
        // scaled at the LDS store), so the loads stay in flight.
        if constexpr (BUF) {
            // [BH][S] arrays: rows past S read the next head's (or 0 past the
            // end); their probabilities are masked
            const unsigned n = (unsigned)((long)BH * S * 4);
            const unsigned vo = (unsigned)((tid & (BM - 1)) * 4);
            const unsigned so = (unsigned)(((long)j.bh * S + q0) * 4);
            t.lse = buffer_load_f32s(buf_rsrc_n(lse, n), vo, so);
            if constexpr (!IPREP)   // in-kernel pre-pass: Di from the O and dO rows
                t.di = buffer_load_f32s(buf_rsrc_n(Di, n), vo, so);
        } else {
            const long i = (long)j.bh * S + min(q0 + (tid & (BM - 1)), S - 1);
            t.lse = lse[i];
            t.di = Di[i];
        }
    };
    // Loads past the last query tile repeat it (clamped tile index), so the
    // job prologue issues the same memory operations on every path and the
    // compiler's waits for its register stages stay tight.
    auto tile_q0 = [&](int qb) { return min(qb, nqb - 1) * BM; };
    // In-kernel pre-pass: a tile's O rows, for its Di.  Requested one pipeline
    // step after its Q and dO rows (once the other stage's O rows have been
    // consumed), so that only one register stage holds O rows at a time.
    auto load_o = [&](QTile& t, const Job& j, int q0) {
        if constexpr (IPREP)
            t.o.loadb(buf_rsrc_n(ip.O + j.base, head_bytes), qoffs, (unsigned)((long)q0 * rs * 4));
    };

    // B operands for S = Q K^T and dP = dO V^T: K/V[key][16dt + 4g + r] for the
    // lane's key (zeroed past S and Dh at the start of the job); and the
    // first two query tiles.
    f4 kreg[NDT], vreg[NDT];
    QTile t0, t1;
    auto load_kv = [&](const Job& j) {
        const int tid = job_tid(), lane = tid & 63, wave = wave_id(tid);
        const int l16 = lane & 15, g = lane >> 4, kg = pair_group(wave);
        if constexpr (BUF) {   // keys past S read 0
            const unsigned vo = (unsigned)(((kg * 16 + l16) * rs + 4 * g) * 4);
            const unsigned so = (unsigned)((long)j.k0 * rs * 4);
            const __amdgpu_buffer_rsrc_t rk = buf_rsrc_n(K + j.base, head_bytes);
            const __amdgpu_buffer_rsrc_t rv = buf_rsrc_n(V + j.base, head_bytes);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                kreg[dt] = buffer_load_f4s(rk, vo + 64 * dt, so);
                vreg[dt] = buffer_load_f4s(rv, vo + 64 * dt, so);
            }
        } else {
            const int key = min(j.k0 + kg * 16 + l16, S - 1);   // masked at job start
            const long off = j.base + (long)key * rs;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                kreg[dt] = load4c<VEC>(K + off, 16 * dt + 4 * g, Dh);
                vreg[dt] = load4c<VEC>(V + off, 16 * dt + 4 * g, Dh);
            }
        }
    };
    auto load_first_q = [&](const Job& j) {
        load_q(t0, j, j.qb0 * BM);
        load_o(t0, j, j.qb0 * BM);
        if (SM::DB)
            load_q(t1, j, tile_q0(j.qb0 + 1));
    };

    Job jc = job_of(snake_job(0));   // the grid never exceeds the job count
    load_kv(jc);
    load_first_q(jc);
    // In-kernel pre-pass.  Every job forms the Di of each query tile it
    // visits from the tile's O and dO rows (loaded with its Q rows).  The dQ
    // rows are zeroed before any atomic reaches them: query tile t = qb*BH + bh
    // (numbered like the jobs, so a workgroup's first job w starts on its own
    // tile w) belongs to workgroup t mod G, which zeroes it before its first
    // job, with device-coherent stores, and then posts its arrival; before its
    // first atomic into a tile of another workgroup (after its first tile's
    // key-side work), a workgroup waits until all have arrived.
    if constexpr (IPREP) {
        const int tid = threadIdx.x, u = tid & 15, rr = tid >> 4;
        const int G = gridDim.x, ntiles = nqb * BH;
        for (int t = blockIdx.x; t < ntiles; t += G) {
            const int qb = t / BH, bh = t - qb * BH;
            const int b = bh / H, h = bh - b * H;
            const __amdgpu_buffer_rsrc_t rq =
                buf_rsrc_n(dQ + (long)b * S * rs + (long)h * Dh, head_bytes);
#pragma unroll
            for (int k = 0; k < 2; k++) {   // thread: rows rr, rr + 32, columns 4u .. 4u+3
                const long s0 = (long)qb * BM + rr + 32 * k;
                // rows past S fall outside the descriptor and are dropped
                buffer_store_f4_dev(rq, (unsigned)(min(s0, (long)S) * rs + 4 * u) * 4u, 0u,
                                    f4zero());
            }
        }
        // Arrival: every wave's device-coherent stores are complete before the
        // count moves (no fence: a device-scope one writes back the whole L2;
        // the dQ atomics are performed past the L2).
        wait_vmem();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(ip.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Wait until every workgroup has arrived (thread 0, bounded: a workgroup
    // that never arrives is counted in sync[2] and the wait gives up).  A
    // workgroup's first query tile is its own (zeroed by itself), so the wait
    // comes before its second tile's dQ atomics; the count is requested after
    // its first tile's key-side work (arrivals come within the first
    // microseconds of the launch) and checked a tile later, so that the check
    // rarely waits for a round trip.  phase: 0 before the first key side, 1
    // count requested, 2 first query side done, 3 waited.
    int phase = IPREP ? 0 : 3;
    unsigned arrived = 0;
    auto first_wait = [&]() {
        if constexpr (IPREP) {
            if (threadIdx.x == 0) {
                const unsigned G = gridDim.x;
                unsigned n = arrived;
                for (int spin = 0; n < G && spin < (1 << 20); spin++) {
                    __builtin_amdgcn_s_sleep(2);
                    n = __hip_atomic_load(ip.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (n < G)
                    __hip_atomic_fetch_add(ip.sync + 2, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
        }
    };
    auto after_key_side = [&]() {
        if constexpr (IPREP) {
            if (phase == 0) {
                if (threadIdx.x == 0)
                    arrived =
                        __hip_atomic_load(ip.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                phase = 1;
            }
        }
    };
    auto before_query_side = [&]() {
        if constexpr (IPREP) {
            if (phase == 2) {
                first_wait();
                phase = 3;
            }
        }
    };
    auto after_query_side = [&]() {
        if constexpr (IPREP) {
            if (phase == 1)
                phase = 2;
        }
    };
#pragma nounroll
    for (int r = 0;; r++) {
        const int jn = snake_job(r + 1);
        const bool more = jn < njobs;
        const Job jnext = job_of(more ? jn : 0);

        const int tid = job_tid(), lane = tid & 63, wave = wave_id(tid);
        const int l16 = lane & 15, g = lane >> 4;
        const int kg = pair_group(wave), qs = wave >> 2;
        const long base = jc.base;
        const int k0 = jc.k0, qb0 = jc.qb0;
        const int mykey = k0 + kg * 16 + l16;
        const bool kok = mykey < S;

        f4 dk[NDT], dv[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            dk[dt] = f4zero();
            dv[dt] = f4zero();
        }
        // q0: the tile's first row (its Q rows are rotated on the way under ROPE)
        auto store_q = [&](const QTile& t, float* st, int q0) __attribute__((always_inline)) {
            if constexpr (ROPE)
                t.q.template store_rope<QS>(st, tid, q0, S, rope_w);
            else
                t.q.template store<QS>(st, tid);
            t.d.template store<QS>(st + BM * QS, tid);
            if (tid < BM) {
                // negated: they start the S and dP accumulators
                st[2 * BM * QS + BM * TS + tid] = -t.lse * kLog2e;
                if constexpr (!IPREP)
                    st[2 * BM * QS + BM * TS + BM + tid] = -t.di * scale;   // scaled as dP is
            }
            if constexpr (IPREP) {
                // Di of rows tid/16 + 32i: a row's 16 units are the 16 lanes of a
                // row group, summed in the separate pre-pass's order
                // (mha_bwd_prep_vec_kernel), so both paths give the same Di
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const f4 o = t.o.r[i], d = t.d.r[i];
                    float di = o[0] * d[0] + o[1] * d[1] + o[2] * d[2] + o[3] * d[3];
                    di += lane_xor16<1>(di);
                    di += lane_xor16<2>(di);
                    di += lane_xor16<4>(di);
                    di += lane_xor16<8>(di);
                    if ((tid & 15) == 0)
                        st[2 * BM * QS + BM * TS + BM + (tid >> 4) + 32 * i] = -di * scale;
                }
            }
        };
        // S = Q K^T and dP = dO V^T for this wave's query blocks (lane holds key
        // l16, queries 16qt + 4g + r); dS goes to LDS for the dQ product, then
        // dV^T += dO^T P and dK^T += Q^T dS accumulate in registers.  The
        // first F of the wave's NQW query blocks lie wholly before its key
        // block (all masked: P = dS = 0) and are skipped; the dQ product never
        // reads their dS.
        // INTERIOR: the tile lies wholly below the causal boundary with every
        // query row before S, so no score needs a mask.
        auto key_side_f = [&](float* st, int q0, auto first, auto interior) __attribute__((always_inline)) {
            constexpr int F = decltype(first)::value;
            constexpr bool INTERIOR = decltype(interior)::value;
            // Raised issue priority for this MFMA-dense section: the other
            // wave of the SIMD fills its stalls instead of interleaving.
            __builtin_amdgcn_s_setprio(1);
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
                // S (K pre-scaled to log2 units) starts at -lse and dP at -Di,
                // so the probabilities are exp2 of the accumulators and dS the
                // product of two of them
                f4 sa[QI], da[QI];
#pragma unroll
                for (int j = 0; j < QI; j++) {
                    const int qt = qs * NQW + q1 + j;
                    sa[j] = *reinterpret_cast<const f4*>(&lse_s[16 * qt + 4 * g]);
                    da[j] = *reinterpret_cast<const f4*>(&di_s[16 * qt + 4 * g]);
                }
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                    for (int j = 0; j < QI; j++) {
                        if (q1 + j < F)
                            continue;
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
                    if (qq < F)
                        continue;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int q = q0 + 16 * qt + 4 * g + r;
                        const bool ok = INTERIOR || ((!diag || mykey <= q) && q < S);
                        const float p = ok ? fast_exp2(sa[j][r]) : 0.0f;
                        P[qq][r] = p;
                        dS[qq][r] = p * da[j][r];
                        dSs[(16 * qt + 4 * g + r) * TS + kg * 16 + l16] = dS[qq][r];
                    }
                }
            }
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                f4 av = dv[dt], ak = dk[dt];
#pragma unroll
                for (int qq = F; qq < NQW; qq++) {
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
            __builtin_amdgcn_s_setprio(0);
        };
        auto key_side = [&](float* st, int q0) __attribute__((always_inline)) {
            // Leading query blocks of the wave that end before its first key.
            int f = 0;
#pragma unroll
            for (int qq = 0; qq < NQW; qq++)
                if (q0 + 16 * (qs * NQW + qq) + 15 < k0 + 16 * kg)
                    f = qq + 1;
            // (only where a third copy of this section fits the registers:
            // the whole-width buffer path without the in-kernel pre-pass or
            // RoPE, at most 64 columns; elsewhere it spills)
            constexpr bool kInterior = BUF && !IPREP && !ROPE && DHP <= 64;
            if (kInterior && q0 >= k0 + MHA_BN && q0 + BM <= S)   // wave-uniform
                key_side_f(st, q0, ic<0>{}, std::true_type{});
            else if (!SKIP || f == 0)
                key_side_f(st, q0, ic<0>{}, std::false_type{});
            else if (f == 1)
                key_side_f(st, q0, ic<1>{}, std::false_type{});
        };
        // dQ tiles (qt, dt) of the query block, dealt round-robin to the waves:
        // dS (LDS) x K (LDS, transposed), added into dQ with float atomics.  A
        // wave's jobs share qt (NW is a multiple of NQT), so pairs of jobs run as
        // two interleaved MFMA chains over one read of the dS operand.  With
        // eight waves and four query blocks, waves w and w+4 (one SIMD) take
        // blocks qt and 3-qt; a block's key blocks past its last query are
        // masked out and skipped.
        constexpr int NJOB = NQT * NDT;
        constexpr int NJ = (NJOB + NW - 1) / NW;   // jobs per wave (the last may be empty)
        static_assert(NW % NQT == 0, "dQ jobs of a wave must share their query block");
        // dQ adds through a buffer descriptor based at the tile's first row;
        // rows past S and columns past Dh are dropped by the descriptor's
        // bounds check rather than by a branch (byte offsets of a 64-row tile
        // stay below 2 GiB for H*Dh < 8M).
        auto dq_store = [&](f4 acc, int q0, int qt, int dt) __attribute__((always_inline)) {
            const int d = 16 * dt + l16;
            if constexpr (ROPE) {
                // Gradient w.r.t. the unrotated Q: rotate this contribution by
                // -pos*w (linear, so the sum of rotated contributions is the
                // rotated sum).  Columns d and d^1 form a pair; they sit in
                // lanes l16 and l16^1.
                const float wv = rope_w[d >> 1];
                const bool odd = (l16 & 1) != 0;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int q = min(q0 + 16 * qt + 4 * g + r, S - 1);
                    float sn, cs;
                    sincos_rev(-(float)q * wv, &sn, &cs);
                    const float other = lane_xor16<1>(acc[r]);
                    acc[r] = odd ? other * sn + acc[r] * cs : acc[r] * cs - other * sn;
                }
            }
            if constexpr (BUF) {
                // rows past S fall outside the descriptor and are dropped
                const __amdgpu_buffer_rsrc_t rq = buf_rsrc_n(dQ + base, head_bytes);
                const unsigned vo = (unsigned)(((16 * qt + 4 * g) * rs + l16) * 4);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    buffer_atomic_add_f32s(rq, vo, (unsigned)(((long)(q0 + r) * rs + 16 * dt) * 4),
                                           acc[r]);
            } else {
                const __amdgpu_buffer_rsrc_t rq = buf_rsrc(dQ + base + (long)q0 * rs);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int qi = 16 * qt + 4 * g + r;
                    const unsigned off = (q0 + qi < S && d < Dh) ? (unsigned)(qi * rs + d) * 4u
                                                                 : kDropOffset;
                    buffer_atomic_add_f32(rq, off, acc[r]);
                }
            }
        };
        const int dq_qt = SKIP ? pair_group(wave) : wave % NQT;
        // FULL: all four key blocks are live; otherwise those before kend.
        auto query_side_f = [&](const float* st, int q0, int kend, auto full) __attribute__((always_inline)) {
            constexpr bool FULL = decltype(full)::value;
            const float* dSs = st + 2 * BM * QS;
            const int qt = dq_qt;
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
                        if (!FULL && kt >= kend)
                            break;
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
                for (int jq = wave; jq < NJOB; jq += NW) {
                    const int dt = jq / NQT;
                    const float* b0 = Kt + (16 * dt + l16) * TS + 4 * g;
                    f4 acc = f4zero();
#pragma unroll
                    for (int kt = 0; kt < 4; kt++) {
                        if (!FULL && kt >= kend)
                            break;
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
        auto query_side = [&](const float* st, int q0) __attribute__((always_inline)) {
            // Key blocks kt with a key at or before the block's last query.
            const int kend = (q0 + 16 * dq_qt + 15 - k0) / 16 + 1;
            if (!SKIP || kend >= 4)
                query_side_f(st, q0, 4, std::true_type{});
            else
                query_side_f(st, q0, kend, std::false_type{});
        };

        // Zero the K/V operands past S and Dh (their loads were clamped; BUF
        // loads read 0 there already), and fold the softmax scale into V.
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if constexpr (!BUF)
                kreg[dt] = mask4(kreg[dt], 16 * dt + 4 * g, Dh, kok);
            if constexpr (ROPE)
                kreg[dt] = rope4(kreg[dt], min(mykey, S - 1), 16 * dt + 4 * g, rope_w, 1.0f);
            vreg[dt] = (BUF ? vreg[dt] : mask4(vreg[dt], 16 * dt + 4 * g, Dh, kok)) * scale;
        }
        // K^T tile for the dQ product, written from the K operand registers by
        // the waves of query split 0 (their key blocks kg cover the tile);
        // then the K operand of S takes the softmax scale in log2 units.
        if (qs == 0) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int r4 = 0; r4 < 4; r4++)
                    Kt[(16 * dt + 4 * g + r4) * TS + kg * 16 + l16] = kreg[dt][r4];
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            kreg[dt] *= c2;
        if constexpr (SM::DB) {
            // Four-deep pipeline: two register stages loaded three query tiles
            // ahead of use, two LDS stages.  Tile qb is in stage qb&1 when
            // iteration qb starts.  The iteration writes dS into its own stage
            // (the dQ jobs read it after the barrier) and, once its own
            // S/dP/dV/dK work is issued, tile qb+1 into the Q/dO/lse/Di part of
            // the other stage: that part was last read before the previous
            // barrier, and the dQ jobs of iteration qb-1 still running on other
            // waves read only the other stage's dS part.  Writing the next tile
            // after the key-side work, rather than at the top, leaves the dQ
            // atomics and loads of the previous iteration time to drain before
            // the wait for its registers.
            store_q(t0, stage(qb0 & 1), qb0 * BM);
            load_q(t0, jc, tile_q0(qb0 + 2));
            load_o(t1, jc, tile_q0(qb0 + 1));
            __syncthreads();
            // Iteration qb < nqb-1: registers tx hold tile qb+1 and are
            // refilled with qb+3; ty hold tile qb+2 (its O rows requested here).
            auto step = [&](QTile& tx, QTile& ty, int qb) {
                const int q0 = qb * BM;
                float* cur = stage(qb & 1);
                key_side(cur, q0);
                after_key_side();
                store_q(tx, stage((qb + 1) & 1), (qb + 1) * BM);
                // Keep the refill below the LDS writes: issued earlier, the
                // wait for the old data would include the new loads.
                __builtin_amdgcn_sched_barrier(0);
                if (qb + 3 < nqb)
                    load_q(tx, jc, q0 + 3 * BM);
                load_o(ty, jc, tile_q0(qb + 2));
                __syncthreads();
                before_query_side();
                query_side(cur, q0);
                after_query_side();
            };
            int qb = qb0;
            for (; qb + 2 < nqb; qb += 2) {
                step(t1, t0, qb);
                step(t0, t1, qb + 1);
            }
            if (qb + 1 < nqb)
                step(t1, t0, qb++);
            // The last query tile: once its key-side work is issued the next
            // job's K/V rows and first query tiles are requested (all register
            // stages are free by then), ahead of this tile's dQ atomics.
            {
                const int q0 = qb * BM;
                float* cur = stage(qb & 1);
                key_side(cur, q0);
                after_key_side();
                // Not above the key-side work: the loads overwrite its operands.
                __builtin_amdgcn_sched_barrier(0);
                if (more) {
                    load_kv(jnext);
                    load_first_q(jnext);
                }
                __syncthreads();
                before_query_side();
                query_side(cur, q0);
                after_query_side();
            }
        } else {
            constexpr bool PREFETCH = DHP <= 128;
            float* st = stage(0);
            for (int qb = qb0; qb < nqb; qb++) {
                const int q0 = qb * BM;
                if (!PREFETCH && qb > qb0)
                    load_q(t0, jc, q0);
                __syncthreads();
                store_q(t0, st, q0);
                __syncthreads();
                if (PREFETCH && qb + 1 < nqb)
                    load_q(t0, jc, q0 + BM);
                key_side(st, q0);
                __builtin_amdgcn_sched_barrier(0);
                if (qb + 1 == nqb && more) {   // next job's loads, as above
                    load_kv(jnext);
                    load_first_q(jnext);
                }
                __syncthreads();
                query_side(st, q0);
            }
        }

        if (NSPLIT > 1) {
            // Sum the per-split partial dK^T/dV^T: splits qs > 0 publish
            // through LDS (reusing the Q/dO tiles), split 0 adds and stores.
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
            if (qs == 0) {
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
        }
        if (qs == 0 && kok) {
            const long off = base + (long)mykey * rs;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                if constexpr (ROPE)   // gradient w.r.t. the unrotated K: the inverse rotation
                    dk[dt] = rope4(dk[dt], mykey, 16 * dt + 4 * g, rope_w, -1.0f);
                store4<VEC>(dK + off, 16 * dt + 4 * g, Dh, dk[dt]);   // dS carries the scale
                store4<VEC>(dV + off, 16 * dt + 4 * g, Dh, dv[dt]);
            }
        }
        if (!more)
            break;
        jc = jnext;
        __syncthreads();   // the reduction records and K^T tile are consumed
    }
    // In-kernel pre-pass: the last workgroup to finish resets the counters
    // for the next launch (every workgroup has passed its wait by now).
    if constexpr (IPREP) {
        if (threadIdx.x == 0 &&
            __hip_atomic_fetch_add(ip.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                gridDim.x - 1) {
            __hip_atomic_store(ip.sync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ip.sync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (cached per device).
static int device_cus()
{
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 256;
    if (cached[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Grid size for the job-loop kernels: a persistent grid (`per_cu` resident
// workgroups per compute unit) with serpentine job order, or one workgroup
// per job under the hardware's dynamic dispatch.  The serpentine order
// balances heavy-first triangular job lists over pairs of rounds (two rounds
// sum to nearly the same work on every workgroup), so it is used for up to
// two rounds, and, where `even_rounds` allows, for any even number of rounds.
// Persistent workgroups also prefetch their next job.
static unsigned job_grid(long njobs, int per_cu, bool even_rounds)
{
    const long g = (long)device_cus() * per_cu;
    const long rounds = (njobs + g - 1) / g;
    if (rounds <= 2 || (even_rounds && rounds % 2 == 0))
        return (unsigned)(njobs < g ? njobs : g);
    return (unsigned)njobs;
}

// Wave groups per workgroup: two per SIMD wherever registers allow.
template <int DHP>
struct MhaSplits {
    static constexpr int FWD = DHP <= 128 ? 2 : 1;
    static constexpr int BWD = DHP <= 64 ? 2 : 1;
    static constexpr int BWD_BM = DHP <= 128 ? 64 : 32;
    // Resident workgroups per CU assumed for the persistent grids (the
    // backward's is read from the kernel's occupancy; this is its fallback).
    static constexpr int FWD_PER_CU = 1;
    static constexpr int BWD_PER_CU = 1;
    // Two forward workgroups fit one compute unit (at most 128 VGPRs under
    // the kernel's launch bound, 2 x 68 KB of LDS): job counts between one
    // and two per compute unit run as one paired round (paired_job).
    static constexpr bool FWD_PAIR = DHP <= 64;
};

// The backward pre-pass riding on a statistics pass (mha_stats_prep_launch).
struct MhaPrep {
    const float* O;
    const float* dO;
    float* Di;
    float* dQ;
};

template <int DHP, bool VEC, bool ROPE, bool BUF = false>
static hipError_t fwd_dispatch2(const float* Q, const float* K, const float* V, float* O,
                                float* lse, int B, int S, int H, int Dh, hipStream_t st,
                                const MhaRope& rope, const MhaPrep* prep = nullptr)
{
    constexpr int NS = MhaSplits<DHP>::FWD;
    const int BH = B * H;
    const int nqb = (S + MHA_BM - 1) / MHA_BM;
    const float qscale = (1.0f / sqrtf((float)Dh)) * kLog2e;
    const long njobs = (long)nqb * BH;
    const int cus = device_cus();
    int pair = 0;
    dim3 grid(job_grid(njobs, MhaSplits<DHP>::FWD_PER_CU, false)), block(256 * NS);
    if (MhaSplits<DHP>::FWD_PAIR && njobs > cus && njobs <= 2L * cus) {
        pair = cus;
        grid.x = (unsigned)njobs;
    }
    if (O != nullptr) {
        ProfScope ps(st, ROPE ? "mha_rope_fwd" : "mha_fwd");
        CXG_LAUNCH((mha_fwd_kernel<DHP, NS, VEC, true, ROPE, false, BUF>), grid, block, 0, st, Q,
                   K, V, O, lse, S, H, Dh, BH, nqb, qscale, pair, rope, nullptr, nullptr, nullptr,
                   nullptr);
    } else if (prep != nullptr) {
        if constexpr (DHP <= 64) {
            ProfScope ps(st, "mha_stats");
            CXG_LAUNCH((mha_fwd_kernel<DHP, NS, VEC, false, ROPE, true, BUF>), grid, block, 0,
                       st, Q, K, V, O, lse, S, H, Dh, BH, nqb, qscale, pair, rope, prep->O,
                       prep->dO, prep->Di, prep->dQ);
        } else {
            return hipErrorInvalidValue;   // the caller runs the separate pre-pass
        }
    } else {
        ProfScope ps(st, "mha_stats");
        CXG_LAUNCH((mha_fwd_kernel<DHP, NS, VEC, false, ROPE, false, BUF>), grid, block, 0, st,
                   Q, K, V, O, lse, S, H, Dh, BH, nqb, qscale, pair, rope, nullptr, nullptr,
                   nullptr, nullptr);
    }
    return hipGetLastError();
}

template <int DHP>
static hipError_t fwd_dispatch(const float* Q, const float* K, const float* V, float* O,
                               float* lse, int B, int S, int H, int Dh, hipStream_t st,
                               const MhaRope* rope, const MhaPrep* prep = nullptr)
{
    const bool vec = (Dh % 4 == 0) && aligned16(Q) && aligned16(K) && aligned16(V) &&
                     (O == nullptr || aligned16(O)) &&
                     (prep == nullptr ||
                      (aligned16(prep->O) && aligned16(prep->dO) && aligned16(prep->dQ)));
    // Whole-width heads take scalar-offset buffer loads (byte offsets within
    // a head's S rows must fit 31 bits).
    const bool buf = vec && Dh == DHP && (long)S * H * Dh * 4 < (1L << 31);
    if (rope != nullptr) {
        if (buf)
            return fwd_dispatch2<DHP, true, true, true>(Q, K, V, O, lse, B, S, H, Dh, st, *rope,
                                                        prep);
        if (vec)
            return fwd_dispatch2<DHP, true, true>(Q, K, V, O, lse, B, S, H, Dh, st, *rope, prep);
        return fwd_dispatch2<DHP, false, true>(Q, K, V, O, lse, B, S, H, Dh, st, *rope, prep);
    }
    const MhaRope none{};
    if (buf)
        return fwd_dispatch2<DHP, true, false, true>(Q, K, V, O, lse, B, S, H, Dh, st, none,
                                                     prep);
    if (vec)
        return fwd_dispatch2<DHP, true, false>(Q, K, V, O, lse, B, S, H, Dh, st, none, prep);
    return fwd_dispatch2<DHP, false, false>(Q, K, V, O, lse, B, S, H, Dh, st, none, prep);
}

void mha_rope_freqs(int Dh, MhaRope* r)
{
    // kernel_test.cpp:453 (the reference's CPU RoPE): powf of the same float exponent
    for (int i = 0; i < 128; i++)
        r->w[i] = i < Dh / 2 ? powf(10000.0f, -2.0f * (float)i / (float)Dh) : 0.0f;
}

hipError_t mha_fwd_launch(const float* Q, const float* K, const float* V, float* O, float* lse,
                          int B, int S, int H, int Dh, hipStream_t st, const MhaRope* rope)
{
    if (mha_nar_ok(B, S, H, Dh))
        return mha_nar_fwd_launch(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    if (Dh <= 16)
        return fwd_dispatch<16>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    if (Dh <= 32)
        return fwd_dispatch<32>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    if (Dh <= 64)
        return fwd_dispatch<64>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    if (Dh <= 128)
        return fwd_dispatch<128>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
    return fwd_dispatch<256>(Q, K, V, O, lse, B, S, H, Dh, st, rope);
}

// The pre-pass rides on the statistics pass for heads up to 64 wide when the
// pass's jobs fit one round of two workgroups per compute unit: the saved
// launch (C2 legacy step 63.1 -> 58.8 us) outweighs each job's extra loads and
// stores there, not over many rounds (B32 H64 S256 Dh8: statistics pass 56 ->
// 66 us against an 11 us pre-pass).
bool mha_stats_prep_ok(int B, int S, int H, int Dh)
{
    const long njobs = (long)B * H * ((S + MHA_BM - 1) / MHA_BM);
    return Dh <= 64 && njobs <= 2L * device_cus();
}

// Statistics pass (lse) with the backward's pre-pass (Di, dQ = 0) in the same
// launch (mha_stats_prep_ok shapes; others return hipErrorInvalidValue and
// take mha_fwd_launch + mha_bwd_prep_launch).
hipError_t mha_stats_prep_launch(const float* Q, const float* K, const float* V, const float* O,
                                 const float* dO, float* lse, float* Di, float* dQ, int B, int S,
                                 int H, int Dh, hipStream_t st, const MhaRope* rope)
{
    if (!mha_stats_prep_ok(B, S, H, Dh))
        return hipErrorInvalidValue;
    const MhaPrep prep{O, dO, Di, dQ};
    if (Dh <= 16)
        return fwd_dispatch<16>(Q, K, V, nullptr, lse, B, S, H, Dh, st, rope, &prep);
    if (Dh <= 32)
        return fwd_dispatch<32>(Q, K, V, nullptr, lse, B, S, H, Dh, st, rope, &prep);
    if (Dh <= 64)
        return fwd_dispatch<64>(Q, K, V, nullptr, lse, B, S, H, Dh, st, rope, &prep);
    return hipErrorInvalidValue;
}

// The same for Dh = 4U (U = 1, 2, 4, 8, 16 lanes per (row, head) segment) with
// aligned rows: O and dO are read as one flat array of 16-byte units, thread
// t taking units t + j*T (T threads in the grid, j < PREP_UNITS) with every
// load issued before any arithmetic (C2, 19.6 MB: 5.2 us at one or four units
// per thread, 4.7 us at two, 6.4 us at eight).  A segment's U units sit in U
// consecutive lanes of one 16-lane row; their partial dot products are summed
// by an xor butterfly of DPP lane moves.
constexpr int PREP_UNITS = 2;

template <int U, bool ZERO>
__global__ __launch_bounds__(256) void mha_bwd_prep_vec_kernel(
    const float* __restrict__ O, const float* __restrict__ dO, float* __restrict__ Di,
    float* __restrict__ dQ, int S, int H, long nunits)
{
    const long t0 = (long)blockIdx.x * 256 + threadIdx.x;
    const long T = (long)gridDim.x * 256;
    const int sub = threadIdx.x & (U - 1);
    f4 o[PREP_UNITS], d[PREP_UNITS];
#pragma unroll
    for (int j = 0; j < PREP_UNITS; j++) {
        const long u = min(t0 + j * T, nunits - 1);   // past the end: a repeated unit
        o[j] = *reinterpret_cast<const f4*>(O + 4 * u);
        d[j] = *reinterpret_cast<const f4*>(dO + 4 * u);
    }
#pragma unroll
    for (int j = 0; j < PREP_UNITS; j++) {
        const long u = t0 + j * T;
        float acc = o[j][0] * d[j][0] + o[j][1] * d[j][1] + o[j][2] * d[j][2] + o[j][3] * d[j][3];
        if constexpr (U > 1)
            acc += lane_xor16<1>(acc);
        if constexpr (U > 2)
            acc += lane_xor16<2>(acc);
        if constexpr (U > 4)
            acc += lane_xor16<4>(acc);
        if constexpr (U > 8)
            acc += lane_xor16<8>(acc);
        if (u < nunits) {
            if (ZERO)
                *reinterpret_cast<f4*>(dQ + 4 * u) = f4zero();
            if (sub == 0) {
                const long seg = u / U;
                const long row = seg / H;
                const int h = (int)(seg - row * H);
                const long b = row / S;
                Di[(b * H + h) * (long)S + (row - b * S)] = acc;
            }
        }
    }
}

template <int U, bool ZERO>
static void prep_vec_go(long nseg, const float* O, const float* dO, float* Di, float* dQ, int S,
                        int H, hipStream_t st)
{
    const long nunits = nseg * U;
    const long threads = (nunits + PREP_UNITS - 1) / PREP_UNITS;
    CXG_LAUNCH((mha_bwd_prep_vec_kernel<U, ZERO>), dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, st, O, dO, Di, dQ, S, H, nunits);
}

template <bool VEC, bool ZERO>
static void prep_go(bool wide, long nseg, const float* O, const float* dO, float* Di, float* dQ,
                    int S, int H, int Dh, hipStream_t st)
{
    if (VEC) {
        switch (Dh) {
        case 4: prep_vec_go<1, ZERO>(nseg, O, dO, Di, dQ, S, H, st); return;
        case 8: prep_vec_go<2, ZERO>(nseg, O, dO, Di, dQ, S, H, st); return;
        case 16: prep_vec_go<4, ZERO>(nseg, O, dO, Di, dQ, S, H, st); return;
        case 32: prep_vec_go<8, ZERO>(nseg, O, dO, Di, dQ, S, H, st); return;
        case 64: prep_vec_go<16, ZERO>(nseg, O, dO, Di, dQ, S, H, st); return;
        default: break;
        }
    }
    const int tpr = wide ? 64 : 16;
    dim3 grid((unsigned)((nseg * tpr + 255) / 256)), block(256);
    if (wide)
        CXG_LAUNCH((mha_bwd_prep_kernel<VEC, ZERO, 64>), grid, block, 0, st, O, dO, Di,
                           dQ, S, H, Dh, nseg);
    else
        CXG_LAUNCH((mha_bwd_prep_kernel<VEC, ZERO, 16>), grid, block, 0, st, O, dO, Di,
                           dQ, S, H, Dh, nseg);
}

// Di = rowsum(O * dO) per (row, head); dQ zeroed for the atomic backward
// (dQ == nullptr: not touched, for kernels that store dQ outright).
hipError_t mha_bwd_prep_launch(const float* O, const float* dO, float* Di, float* dQ, int B,
                               int S, int H, int Dh, hipStream_t st)
{
    const long nseg = (long)B * S * H;
    const bool wide = Dh > 256;
    ProfScope ps(st, "mha_bwd_prep");
    const bool vec = (Dh % 4 == 0) && aligned16(O) && aligned16(dO) && aligned16(dQ);
    if (vec) {
        if (dQ)
            prep_go<true, true>(wide, nseg, O, dO, Di, dQ, S, H, Dh, st);
        else
            prep_go<true, false>(wide, nseg, O, dO, Di, dQ, S, H, Dh, st);
    } else {
        if (dQ)
            prep_go<false, true>(wide, nseg, O, dO, Di, dQ, S, H, Dh, st);
        else
            prep_go<false, false>(wide, nseg, O, dO, Di, dQ, S, H, Dh, st);
    }
    return hipGetLastError();
}

// Resident backward workgroups per compute unit for the persistent grid: what
// the kernel's registers and LDS allow (two for Dh <= 16, one above), found
// once; jobs are claimed by index, so any grid size is correct.
template <int DHP, bool ROPE>
static int bwd_per_cu()
{
    constexpr int NS = MhaSplits<DHP>::BWD, BM = MhaSplits<DHP>::BWD_BM;
    static int per_cu = 0;
    if (per_cu <= 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, (const void*)mha_bwd_kernel<DHP, BM, NS, true, ROPE>, 256 * NS, 0) !=
                hipSuccess ||
            n <= 0)
            n = MhaSplits<DHP>::BWD_PER_CU;
        per_cu = n;
    }
    return per_cu;
}

// Byte offsets within a head's S rows fit 31 bits (the buffer-descriptor path).
static bool bwd_buf_ok(int S, int H, int Dh) { return (long)S * H * Dh * 4 < (1L << 31); }

template <int DHP, bool ROPE>
static hipError_t bwd_dispatch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st,
                               const MhaRope& rope, const MhaIPrep* ip)
{
    constexpr int NS = MhaSplits<DHP>::BWD, BM = MhaSplits<DHP>::BWD_BM;
    const int BH = B * H;
    const int nkb = (S + MHA_BN - 1) / MHA_BN;
    const float scale = 1.0f / sqrtf((float)Dh);
    const int per_cu = bwd_per_cu<DHP, ROPE>();
    dim3 grid(job_grid((long)nkb * BH, per_cu, true)), block(256 * NS);
    const bool vec = (Dh % 4 == 0) && aligned16(Q) && aligned16(K) && aligned16(V) &&
                     aligned16(dO) && aligned16(dK) && aligned16(dV);
    const MhaIPrep noip{};
    ProfScope ps(st, ROPE ? "mha_rope_bwd" : "mha_bwd");
    // Whole-width heads on the double-buffered path take buffer loads and
    // atomics (byte offsets within a head's S rows must fit 31 bits).
    if constexpr (BwdSmem<DHP, BM>::DB) {
        if (vec && Dh == DHP && aligned16(dQ) && bwd_buf_ok(S, H, Dh)) {
            if constexpr (DHP == 64 && !ROPE) {
                if (ip != nullptr) {   // the caller checked mha_bwd_iprep_ok
                    CXG_LAUNCH((mha_bwd_kernel<DHP, BM, NS, true, ROPE, true, true>), grid, block,
                               0, st, Q, K, V, dO, lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale,
                               scale * kLog2e, rope, *ip);
                    return hipGetLastError();
                }
            }
            CXG_LAUNCH((mha_bwd_kernel<DHP, BM, NS, true, ROPE, true>), grid, block, 0, st, Q, K,
                       V, dO, lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e, rope,
                       noip);
            return hipGetLastError();
        }
    }
    if (ip != nullptr)
        return hipErrorInvalidValue;
    if (vec)
        CXG_LAUNCH((mha_bwd_kernel<DHP, BM, NS, true, ROPE>), grid, block, 0, st, Q, K, V, dO,
                           lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e, rope,
                           noip);
    else
        CXG_LAUNCH((mha_bwd_kernel<DHP, BM, NS, false, ROPE>), grid, block, 0, st, Q, K, V, dO,
                           lse, Di, dQ, dK, dV, S, H, Dh, BH, nkb, scale, scale * kLog2e, rope,
                           noip);
    return hipGetLastError();
}

// The in-kernel pre-pass (MhaIPrep) applies to whole-width Dh = 64 heads on
// the buffer-descriptor path whose grid is persistent (every workgroup
// resident at once, so the wait for all arrivals ends), for sequences of up
// to 8 query tiles: each job forms the Di of every tile it visits, which pays
// where a tile has few visitors and the separate pre-pass's launch is a large
// share of the step (C2: 49.7 -> 48.5 us a step), and costs more than that
// pass at long sequences (C5, 64 tiles: 1.48 -> 1.52 ms).
bool mha_bwd_iprep_ok(int B, int S, int H, int Dh, const float* Q, const float* K,
                      const float* V, const float* dO, const float* O, const float* dQ,
                      const float* dK, const float* dV)
{
    if (Dh != 64 || S > 8 * MHA_BN || !bwd_buf_ok(S, H, Dh))
        return false;
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(dO) || !aligned16(O) ||
        !aligned16(dQ) || !aligned16(dK) || !aligned16(dV))
        return false;
    const long njobs = (long)((S + MHA_BN - 1) / MHA_BN) * B * H;
    const long slots = (long)device_cus() * bwd_per_cu<64, false>();
    return (long)job_grid(njobs, bwd_per_cu<64, false>(), true) <= slots;
}

hipError_t mha_bwd_main_launch(const float* Q, const float* K, const float* V, const float* dO,
                               const float* lse, const float* Di, float* dQ, float* dK,
                               float* dV, int B, int S, int H, int Dh, hipStream_t st,
                               const MhaRope* rope, const MhaIPrep* ip)
{
    const MhaRope none{};
    const MhaRope& rp = rope != nullptr ? *rope : none;
    if (ip != nullptr && (rope != nullptr || Dh != 64))
        return hipErrorInvalidValue;
#define CXG_BWD(D)                                                                            \
    return rope != nullptr                                                                    \
               ? bwd_dispatch<D, true>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st, rp,  \
                                       nullptr)                                               \
               : bwd_dispatch<D, false>(Q, K, V, dO, lse, Di, dQ, dK, dV, B, S, H, Dh, st, rp, \
                                        ip)
    if (Dh <= 16)
        CXG_BWD(16);
    if (Dh <= 32)
        CXG_BWD(32);
    if (Dh <= 64)
        CXG_BWD(64);
    if (Dh <= 128)
        CXG_BWD(128);
    CXG_BWD(256);
#undef CXG_BWD
}

} // namespace cxg
