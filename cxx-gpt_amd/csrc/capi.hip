// capi.hip -- extern "C" entry points declared in include/cxxgpt_attn.h:
// argument checks, workspace handling and dispatch to the kernel launchers.
#include "../../include/cxxgpt_attn.h"
#include "launch.hpp"
#include "linattn.hpp"

#include <hip/hip_runtime.h>

#include <limits.h>
#include <stdint.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace cxg {

// ---------------------------------------------------------------------------
// timing hook
// ---------------------------------------------------------------------------
namespace {
struct ProfRec {
    hipEvent_t a, b;
    std::string name;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRec> g_prof_recs;
std::vector<hipEvent_t> g_prof_free;

hipEvent_t prof_event()
{
    hipEvent_t e = nullptr;
    if (!g_prof_free.empty()) {
        e = g_prof_free.back();
        g_prof_free.pop_back();
        return e;
    }
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}
} // namespace

bool prof_enabled() { return g_prof_on; }

int prof_begin(hipEvent_t* a, hipEvent_t* b)
{
    std::lock_guard<std::mutex> lk(g_prof_mu);
    ProfRec r;
    r.a = prof_event();
    r.b = prof_event();
    if (!r.a || !r.b)
        return -1;
    *a = r.a;
    *b = r.b;
    g_prof_recs.push_back(r);
    return (int)g_prof_recs.size() - 1;
}

void prof_end(int token, const char* name)
{
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (token < 0 || token >= (int)g_prof_recs.size())
        return;
    g_prof_recs[token].name = name;
}

namespace {
thread_local ProfScope* t_prof_scope = nullptr;
}

ProfScope::ProfScope(hipStream_t, const char* n)
    : tok(-1), name(n), a(nullptr), b(nullptr), started(false), outer(t_prof_scope)
{
    if (prof_enabled())
        tok = prof_begin(&a, &b);
    if (tok >= 0)
        t_prof_scope = this;
}

ProfScope::~ProfScope()
{
    if (tok >= 0) {
        t_prof_scope = outer;
        // a scope that launched nothing has unrecorded events: its record is
        // left unnamed and never matches a query
        if (started)
            prof_end(tok, name);
    }
}

ProfScope* prof_scope() { return t_prof_scope; }

// ---------------------------------------------------------------------------
// status helpers
// ---------------------------------------------------------------------------
static thread_local int t_last_hip = 0;

static int hip_status(hipError_t e)
{
    if (e == hipSuccess)
        return CXG_OK;
    t_last_hip = (int)e;
    return CXG_ERR_HIP;
}

static bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

// Scratch for calls without a caller workspace, cached per (device, stream):
// a buffer that grows to the largest request seen on that stream and is kept
// until the process ends.  Calls on one stream are ordered on the device, so
// reuse needs no synchronisation; the entry's mutex is held for the whole
// call, so host threads sharing a stream do not swap the buffer under one
// another.  Growth frees the old buffer with hipFree (which waits for the
// device), so it happens only while a caller's sizes are still rising.
namespace {
struct StreamScratch {
    std::mutex mu;
    void* p = nullptr;
    size_t n = 0;
};
std::mutex g_scratch_map_mu;
std::map<std::pair<int, hipStream_t>, std::unique_ptr<StreamScratch>> g_scratch_map;
} // namespace

// Three device words per (device, stream) for the backward's in-kernel
// pre-pass (MhaIPrep::sync): allocated and zeroed at the first eligible call
// on the stream, left zero by every launch, held until the process ends (a
// graph captured on the stream keeps pointing at them).  Under stream capture
// no new words are allocated (the call takes the separate pre-pass instead).
namespace {
std::mutex g_sync_mu;
std::map<std::pair<int, hipStream_t>, unsigned*> g_sync_map;

unsigned* stream_sync(hipStream_t s, bool create)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess)
        return nullptr;
    std::lock_guard<std::mutex> lk(g_sync_mu);
    auto it = g_sync_map.find(std::make_pair(dev, s));
    if (it != g_sync_map.end())
        return it->second;
    if (!create)
        return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, 256) != hipSuccess)
        return nullptr;
    if (hipMemset(p, 0, 256) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    g_sync_map[std::make_pair(dev, s)] = (unsigned*)p;
    return (unsigned*)p;
}
} // namespace

// Scratch for one call: caller memory if provided; else the stream's cached
// buffer; under stream capture, stream-ordered memory for the duration of the
// call (hipMallocAsync, which capture records as graph memory nodes).
struct Scratch {
    void* p = nullptr;
    bool owned = false;
    hipStream_t st = nullptr;
    std::unique_lock<std::mutex> held;
    int acquire(void* ws, size_t ws_bytes, size_t need, hipStream_t s)
    {
        st = s;
        if (need == 0)
            return CXG_OK;
        if (ws != nullptr) {
            if (ws_bytes < need)
                return CXG_ERR_WORKSPACE;
            p = ws;
            return CXG_OK;
        }
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        int dev = -1;
        if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone &&
            hipGetDevice(&dev) == hipSuccess) {
            StreamScratch* e;
            {
                std::lock_guard<std::mutex> lk(g_scratch_map_mu);
                auto& slot = g_scratch_map[std::make_pair(dev, s)];
                if (!slot)
                    slot.reset(new StreamScratch);
                e = slot.get();
            }
            held = std::unique_lock<std::mutex>(e->mu);
            if (e->n < need) {
                if (e->p != nullptr)
                    (void)hipFree(e->p);
                e->p = nullptr;
                e->n = 0;
                const size_t want = need + need / 4;   // room for slightly larger calls
                hipError_t err = hipMalloc(&e->p, want);
                if (err != hipSuccess) {
                    t_last_hip = (int)err;
                    e->p = nullptr;
                    return CXG_ERR_WORKSPACE;
                }
                e->n = want;
            }
            p = e->p;
            return CXG_OK;
        }
        hipError_t e = hipMallocAsync(&p, need, s);
        if (e != hipSuccess) {
            t_last_hip = (int)e;
            p = nullptr;
            return CXG_ERR_WORKSPACE;
        }
        owned = true;
        return CXG_OK;
    }
    ~Scratch()
    {
        if (owned && p)
            (void)hipFreeAsync(p, st);
    }
};

static size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static bool al16c(const void* p) { return ((uintptr_t)p & 15u) == 0; }

} // namespace cxg

using namespace cxg;

extern "C" {

const char* cxg_status_str(int status)
{
    switch (status) {
    case CXG_OK: return "ok";
    case CXG_ERR_NULL: return "null pointer argument";
    case CXG_ERR_DIMS: return "invalid dimensions";
    case CXG_ERR_HEAD_DIM: return "head_dim > 256 not supported";
    case CXG_ERR_HIP: return "HIP runtime error";
    case CXG_ERR_WORKSPACE: return "workspace too small or allocation failed";
    case CXG_ERR_ALIGN: return "tensor not 16-byte aligned or width not a multiple of 4";
    default: return "unknown status";
    }
}

int cxg_last_hip_error(void) { return t_last_hip; }

const char* cxg_version(void) { return "cxxgpt-attn-gfx950 0.1"; }

int cxg_release_scratch(cxg_stream_t stream)
{
    const hipStream_t s = (hipStream_t)stream;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return hip_status(e);
    std::unique_ptr<StreamScratch> victim;
    {
        std::lock_guard<std::mutex> lk(g_scratch_map_mu);
        auto it = g_scratch_map.find(std::make_pair(dev, s));
        if (it == g_scratch_map.end())
            return CXG_OK;
        victim = std::move(it->second);
        g_scratch_map.erase(it);
    }
    std::lock_guard<std::mutex> held(victim->mu);   // a call holding it finishes first
    e = hipStreamSynchronize(s);
    if (e == hipSuccess && victim->p != nullptr)
        e = hipFree(victim->p);
    victim->p = nullptr;
    victim->n = 0;
    return hip_status(e);
}

// ---------------------------------------------------------------------------
// softmax MHA
// ---------------------------------------------------------------------------
static int mha_check(size_t B, size_t S, size_t H, size_t Dh, bool* empty)
{
    *empty = (B == 0 || S == 0 || H == 0);
    if (Dh == 0)
        return CXG_ERR_DIMS;
    if (Dh > 256)
        return CXG_ERR_HEAD_DIM;
    if (*empty)
        return CXG_OK;
    if (!fits_int(B) || !fits_int(S) || !fits_int(H) || !fits_int(B * H))
        return CXG_ERR_DIMS;
    const size_t ntile = (S + 63) / 64;
    // grid x = tiles * B * H workgroups of 256 threads must stay below 2^32 threads
    if (ntile * B * H > ((size_t)1 << 23))
        return CXG_ERR_DIMS;
    return CXG_OK;
}

int cxg_mha_fwd(const float* Q, const float* K, const float* V, float* O, float* lse,
                size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream)
{
    bool empty;
    int st = mha_check(B, S, H, Dh, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O)
        return CXG_ERR_NULL;
    return hip_status(mha_fwd_launch(Q, K, V, O, lse, (int)B, (int)S, (int)H, (int)Dh,
                                     (hipStream_t)stream));
}

int cxg_mha_rope_fwd(const float* Q, const float* K, const float* V, float* O, float* lse,
                     size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream)
{
    bool empty;
    int st = mha_check(B, S, H, Dh, &empty);
    if (st == CXG_OK && Dh % 2 != 0)
        st = CXG_ERR_DIMS;
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O)
        return CXG_ERR_NULL;
    MhaRope rope;
    mha_rope_freqs((int)Dh, &rope);
    return hip_status(mha_fwd_launch(Q, K, V, O, lse, (int)B, (int)S, (int)H, (int)Dh,
                                     (hipStream_t)stream, &rope));
}

size_t cxg_mha_bwd_workspace_size(size_t B, size_t S, size_t H, size_t Dh)
{
    (void)Dh;
    const size_t rows = B * H * S;
    return 2 * round_up(rows * sizeof(float), 256);
}

static int mha_bwd_common(const float* Q, const float* K, const float* V, const float* O,
                          const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                          size_t B, size_t S, size_t H, size_t Dh, void* workspace,
                          size_t workspace_bytes, cxg_stream_t stream, bool with_rope)
{
    bool empty;
    int st = mha_check(B, S, H, Dh, &empty);
    if (st == CXG_OK && with_rope && Dh % 2 != 0)
        st = CXG_ERR_DIMS;
    if (st != CXG_OK || empty)
        return st;
    MhaRope rope_freq;
    const MhaRope* rope = nullptr;
    if (with_rope) {
        mha_rope_freqs((int)Dh, &rope_freq);
        rope = &rope_freq;
    }
    if (!Q || !K || !V || !O || !dO || !dQ || !dK || !dV)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const int iB = (int)B, iS = (int)S, iH = (int)H, iD = (int)Dh;
    if (mha_nar_ok(iB, iS, iH, iD)) {
        // one launch that uses no scratch; a caller's workspace is still
        // checked against the documented size, whichever kernels run
        if (workspace != nullptr && workspace_bytes < cxg_mha_bwd_workspace_size(B, S, H, Dh))
            return CXG_ERR_WORKSPACE;
        return hip_status(
            mha_nar_bwd_launch(Q, K, V, O, dO, lse, dQ, dK, dV, iB, iS, iH, iD, s, rope));
    }
    const size_t half = round_up(B * H * S * sizeof(float), 256);
    Scratch ws;
    st = ws.acquire(workspace, workspace_bytes, cxg_mha_bwd_workspace_size(B, S, H, Dh), s);
    if (st != CXG_OK)
        return st;
    float* Di = (float*)ws.p;
    float* lse_ws = (float*)((char*)ws.p + half);
    hipError_t e;
    if (lse == nullptr && mha_stats_prep_ok(iB, iS, iH, iD)) {
        // statistics-only forward pass (the reference recomputes them too),
        // with the pre-pass in the same launch
        e = mha_stats_prep_launch(Q, K, V, O, dO, lse_ws, Di, dQ, iB, iS, iH, iD, s, rope);
        if (e != hipSuccess)
            return hip_status(e);
        lse = lse_ws;
    } else {
        if (lse == nullptr) {
            e = mha_fwd_launch(Q, K, V, nullptr, lse_ws, iB, iS, iH, iD, s, rope);
            if (e != hipSuccess)
                return hip_status(e);
            lse = lse_ws;
        }
        // Di and dQ = 0 inside the backward kernel where it can take them
        unsigned* sync = rope == nullptr &&
                                 mha_bwd_iprep_ok(iB, iS, iH, iD, Q, K, V, dO, O, dQ, dK, dV)
                             ? stream_sync(s, true)
                             : nullptr;
        if (sync != nullptr) {
            const MhaIPrep ip{O, sync};
            return hip_status(mha_bwd_main_launch(Q, K, V, dO, lse, Di, dQ, dK, dV, iB, iS, iH,
                                                  iD, s, nullptr, &ip));
        }
        e = mha_bwd_prep_launch(O, dO, Di, dQ, iB, iS, iH, iD, s);
        if (e != hipSuccess)
            return hip_status(e);
    }
    e = mha_bwd_main_launch(Q, K, V, dO, lse, Di, dQ, dK, dV, iB, iS, iH, iD, s, rope);
    return hip_status(e);
}

int cxg_wait_timeouts(cxg_stream_t stream, unsigned* count)
{
    if (count == nullptr)
        return CXG_ERR_NULL;
    *count = 0;
    hipStream_t s = (hipStream_t)stream;
    unsigned* p = stream_sync(s, false);
    if (p == nullptr)
        return CXG_OK;
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess)
        e = hipMemcpy(count, p + 2, sizeof(unsigned), hipMemcpyDeviceToHost);
    return hip_status(e);
}

int cxg_mha_bwd(const float* Q, const float* K, const float* V, const float* O,
                const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                size_t B, size_t S, size_t H, size_t Dh, void* workspace,
                size_t workspace_bytes, cxg_stream_t stream)
{
    return mha_bwd_common(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, workspace,
                          workspace_bytes, stream, false);
}

// ---------------------------------------------------------------------------
// allocation-free backward: the scratch (Di and the statistics pass's lse) lives
// in a file-scope device array instead of a workspace
// ---------------------------------------------------------------------------
} // extern "C"

namespace cxg {
// One copy per GPU the library runs on, held until the process ends.  In host
// code `scratch` is only a handle: its device address (per device) comes from
// hipGetSymbolAddress, and only that address reaches kernels.
constexpr size_t kNoAllocScratchFloats = 2 * (size_t)CXG_MHA_BWD_NOALLOC_MAX_ROWS;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices];

// Device address of this device's scratch array (resolved once per device, with
// that device current); nullptr and *err set on failure.
float* scratch_ptr(hipError_t* err)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices))
        e = hipErrorInvalidDevice;
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
            return nullptr;
        }
        g_scratch_ptr[dev] = (float*)p;
    }
    return g_scratch_ptr[dev];
}
} // namespace
} // namespace cxg

extern "C" {

int cxg_mha_bwd_noalloc(const float* Q, const float* K, const float* V, const float* O,
                        const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                        size_t B, size_t S, size_t H, size_t Dh, cxg_stream_t stream)
{
    bool empty;
    int st = mha_check(B, S, H, Dh, &empty);
    if (st != CXG_OK || empty)
        return st;
    // the capacity check comes first: a problem beyond the array is refused
    // whatever else is wrong with the call
    const size_t rows = B * H * S;
    if (rows > (size_t)CXG_MHA_BWD_NOALLOC_MAX_ROWS)
        return CXG_ERR_WORKSPACE;
    if (!Q || !K || !V || !O || !dO || !dQ || !dK || !dV)
        return CXG_ERR_NULL;
    if (mha_nar_ok((int)B, (int)S, (int)H, (int)Dh))   // its kernel uses no scratch
        return hip_status(mha_nar_bwd_launch(Q, K, V, O, dO, lse, dQ, dK, dV, (int)B, (int)S,
                                             (int)H, (int)Dh, (hipStream_t)stream));
    hipError_t e = hipSuccess;
    float* sp = scratch_ptr(&e);
    if (sp == nullptr)
        return hip_status(e);
    // Di in the first half, the statistics pass's lse in the second; both are
    // written in full before they are read, so nothing needs clearing
    float* Di = sp;
    float* lse_ws = sp + CXG_MHA_BWD_NOALLOC_MAX_ROWS;
    hipStream_t s = (hipStream_t)stream;
    const int iB = (int)B, iS = (int)S, iH = (int)H, iD = (int)Dh;
    if (lse == nullptr && mha_stats_prep_ok(iB, iS, iH, iD)) {
        e = mha_stats_prep_launch(Q, K, V, O, dO, lse_ws, Di, dQ, iB, iS, iH, iD, s);
        if (e != hipSuccess)
            return hip_status(e);
        lse = lse_ws;
    } else {
        if (lse == nullptr) {
            e = mha_fwd_launch(Q, K, V, nullptr, lse_ws, iB, iS, iH, iD, s);
            if (e != hipSuccess)
                return hip_status(e);
            lse = lse_ws;
        }
        e = mha_bwd_prep_launch(O, dO, Di, dQ, iB, iS, iH, iD, s);
        if (e != hipSuccess)
            return hip_status(e);
    }
    return hip_status(mha_bwd_main_launch(Q, K, V, dO, lse, Di, dQ, dK, dV, iB, iS, iH, iD, s));
}

int cxg_mha_rope_bwd(const float* Q, const float* K, const float* V, const float* O,
                     const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                     size_t B, size_t S, size_t H, size_t Dh, void* workspace,
                     size_t workspace_bytes, cxg_stream_t stream)
{
    return mha_bwd_common(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, H, Dh, workspace,
                          workspace_bytes, stream, true);
}

// ---------------------------------------------------------------------------
// GPT's attention: one head over the embedding (H = 1, Dh = E)
// ---------------------------------------------------------------------------
static int gpt_check(size_t B, size_t S, size_t E, bool* empty)
{
    *empty = (B == 0 || S == 0);
    if (E == 0)
        return CXG_ERR_DIMS;
    if (*empty)
        return CXG_OK;
    if (E > (size_t)MHA_WIDE_MAX_DH) {
        // scores in memory: causal score blocks (E a multiple of 16, within the
        // block-score scratch budget), else S x S floats per sequence (S <=
        // 16384: 1 GiB) with GEMM shapes in int; any S, E a multiple of 4
        if (!fits_int(B) || !fits_int(E) || S > 16384 || B * S * E > ((size_t)1 << 40))
            return CXG_ERR_DIMS;
        return gpt_mat_ok((int)S, (int)E) ? CXG_OK : CXG_ERR_ALIGN;
    }
    if (!fits_int(B) || !fits_int(S) || B * ((S + 15) / 16) > ((size_t)1 << 23))
        return CXG_ERR_DIMS;
    // the wide kernels address one sequence with 32-bit byte offsets
    if (E > 256 && S * E > ((size_t)1 << 28))
        return CXG_ERR_DIMS;
    return CXG_OK;
}

// Widths above 256 that are multiples of 16 take the causal score blocks
// (faster than the wide-head kernels at E = 512: 58 against 81 us a B8 S256
// step) whenever their scratch fits; others the wide-head kernels (up to 512)
// or the S x S scores and GEMMs.
static bool gpt_blocks(size_t B, size_t S, size_t E)
{
    return E > 256 && E % 16 == 0 && gpt_qs_ok((int)B, (int)S, (int)E);
}

int cxg_gpt_attn_fwd(const float* Q, const float* K, const float* V, float* O, float* lse,
                     size_t B, size_t S, size_t E, cxg_stream_t stream)
{
    if (E > 0 && E <= 256)
        return cxg_mha_fwd(Q, K, V, O, lse, B, S, 1, E, stream);
    bool empty;
    int st = gpt_check(B, S, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    if (E > (size_t)MHA_WIDE_MAX_DH || gpt_blocks(B, S, E)) {
        if (!al16c(Q) || !al16c(K) || !al16c(V) || !al16c(O))
            return CXG_ERR_ALIGN;
        if (gpt_blocks(B, S, E)) {
            Scratch ws;
            st = ws.acquire(nullptr, 0, gpt_qs_ws_bytes((int)B, (int)S, (int)E, false), s);
            if (st != CXG_OK)
                return st;
            return hip_status(
                gpt_qs_fwd_launch(Q, K, V, O, lse, (int)B, (int)S, (int)E, ws.p, s));
        }
        Scratch ws;
        st = ws.acquire(nullptr, 0, gpt_mat_fwd_ws_floats((int)B, (int)S, (int)E) * sizeof(float),
                        s);
        if (st != CXG_OK)
            return st;
        return hip_status(gpt_mat_fwd_launch(Q, K, V, O, lse, (int)B, (int)S, (int)E,
                                             (float*)ws.p, s));
    }
    Scratch ws;   // split-KV partial states (few-job shapes)
    st = ws.acquire(nullptr, 0, mha_wide_fwd_ws_floats((int)B, (int)S) * sizeof(float), s);
    if (st != CXG_OK)
        return st;
    return hip_status(
        mha_wide_fwd_launch(Q, K, V, O, lse, (int)B, (int)S, 1, (int)E, (float*)ws.p, s));
}

size_t cxg_gpt_attn_bwd_workspace_size(size_t B, size_t S, size_t E)
{
    if (E <= 256)
        return cxg_mha_bwd_workspace_size(B, S, 1, E);
    bool empty;
    if (gpt_check(B, S, E, &empty) != CXG_OK || empty)
        return 0;
    if (gpt_blocks(B, S, E))   // P and dS blocks, Di and lse
        return gpt_qs_ws_bytes((int)B, (int)S, (int)E, true);
    if (E > (size_t)MHA_WIDE_MAX_DH)   // the scores of a group of sequences, GEMM partials
        return gpt_mat_ws_floats((int)B, (int)S, (int)E) * sizeof(float);
    // Di, lse, and the partial records of the statistics pass and of the
    // backward (used one after the other)
    const size_t part = std::max(mha_wide_fwd_ws_floats((int)B, (int)S),
                                 mha_wide_bwd_ws_floats((int)B, (int)S));
    return 2 * round_up(B * S * sizeof(float), 256) + round_up(part * sizeof(float), 256);
}

int cxg_gpt_attn_bwd(const float* Q, const float* K, const float* V, const float* O,
                     const float* dO, const float* lse, float* dQ, float* dK, float* dV,
                     size_t B, size_t S, size_t E, void* workspace, size_t workspace_bytes,
                     cxg_stream_t stream)
{
    if (E > 0 && E <= 256)
        return cxg_mha_bwd(Q, K, V, O, dO, lse, dQ, dK, dV, B, S, 1, E, workspace,
                           workspace_bytes, stream);
    bool empty;
    int st = gpt_check(B, S, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O || !dO || !dQ || !dK || !dV)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const size_t half = round_up(B * S * sizeof(float), 256);
    Scratch ws;
    st = ws.acquire(workspace, workspace_bytes, cxg_gpt_attn_bwd_workspace_size(B, S, E), s);
    if (st != CXG_OK)
        return st;
    if (E > (size_t)MHA_WIDE_MAX_DH || gpt_blocks(B, S, E)) {
        if (!al16c(Q) || !al16c(K) || !al16c(V) || !al16c(dO) || !al16c(dQ) || !al16c(dK) ||
            !al16c(dV) || !al16c(ws.p))
            return CXG_ERR_ALIGN;
        if (gpt_blocks(B, S, E))
            return hip_status(gpt_qs_bwd_launch(Q, K, V, O, dO, lse, dQ, dK, dV, (int)B, (int)S,
                                                (int)E, ws.p, s));
        return hip_status(gpt_mat_bwd_launch(Q, K, V, dO, lse, dQ, dK, dV, (int)B, (int)S,
                                             (int)E, (float*)ws.p, s));
    }
    float* Di = (float*)ws.p;
    float* lse_ws = (float*)((char*)ws.p + half);
    float* part = (float*)((char*)ws.p + 2 * half);
    const int iB = (int)B, iS = (int)S, iE = (int)E;
    hipError_t e;
    if (lse == nullptr) {
        e = mha_wide_fwd_launch(Q, K, V, nullptr, lse_ws, iB, iS, 1, iE, part, s);
        if (e != hipSuccess)
            return hip_status(e);
        lse = lse_ws;
    }
    e = mha_bwd_prep_launch(O, dO, Di, nullptr, iB, iS, 1, iE, s);   // dQ is stored outright
    if (e != hipSuccess)
        return hip_status(e);
    return hip_status(
        mha_wide_bwd_launch(Q, K, V, dO, lse, Di, dQ, dK, dV, iB, iS, 1, iE, part, s));
}

// ---------------------------------------------------------------------------
// linear attention
// ---------------------------------------------------------------------------
// Dimensions of a (B sequences x S rows) problem with Q/K width D and V width E.
static int lin_check(size_t B, size_t S, size_t D, size_t E, bool* empty)
{
    *empty = (B == 0 || S == 0);
    if (D == 0 || E == 0)
        return CXG_ERR_DIMS;
    if (*empty)
        return CXG_OK;
    if (!fits_int(B) || !fits_int(S) || !fits_int(D) || !fits_int(E) || !fits_int(B * S))
        return CXG_ERR_DIMS;
    // element offsets stay within 63 bits and the generic state fits memory indexing
    if (B * S > ((size_t)1 << 40) / (D > E ? D : E) || B * D * E > ((size_t)1 << 40))
        return CXG_ERR_DIMS;
    return CXG_OK;
}

// Contexts the forwards have written: device, shape, feature map and byte
// span per context pointer, so that the fused backward refuses a context
// written for another problem (whose records it would read at the wrong
// offsets) or by another API's forward (whose sums use another feature map).
// The check is on shape and feature map only: it cannot tell that a context's
// memory was freed and reused for another context of the same shape.  A
// forward that writes a context drops every tag on the same device whose span
// overlaps it (that memory now holds the new context), and the table keeps at
// most kCtxTagsMax tags, so it stays bounded by the contexts that are live.
namespace {
struct CtxTag {
    int dev, phi;
    size_t B, S, D, E, bytes;
};
constexpr size_t kCtxTagsMax = 4096;
std::mutex g_ctx_mu;
std::unordered_map<const void*, CtxTag> g_ctx_tags;

void ctx_record(const void* ctx, size_t bytes, int phi, size_t B, size_t S, size_t D, size_t E)
{
    int dev = -1;
    (void)hipGetDevice(&dev);
    const uintptr_t lo = (uintptr_t)ctx, hi = lo + bytes;
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    for (auto it = g_ctx_tags.begin(); it != g_ctx_tags.end();) {
        const uintptr_t a = (uintptr_t)it->first, b = a + it->second.bytes;
        if (it->second.dev == dev && a < hi && lo < b)
            it = g_ctx_tags.erase(it);
        else
            ++it;
    }
    if (g_ctx_tags.size() >= kCtxTagsMax)
        g_ctx_tags.erase(g_ctx_tags.begin());
    g_ctx_tags[ctx] = CtxTag{dev, phi, B, S, D, E, bytes};
}

bool ctx_matches(const void* ctx, int phi, size_t B, size_t S, size_t D, size_t E)
{
    int dev = -1;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    auto it = g_ctx_tags.find(ctx);
    if (it == g_ctx_tags.end())
        return false;
    const CtxTag& t = it->second;
    return t.dev == dev && t.phi == phi && t.B == B && t.S == S && t.D == D && t.E == E;
}
} // namespace

static int lin_fwd_common(int phi, int den_eps, int sfin_de, const float* Q, const float* K,
                          const float* V, float* O, float* den, float* zc, float* S_buf,
                          float* z_buf, size_t B, size_t S, size_t D, size_t E,
                          cxg_stream_t stream, void* ctx = nullptr, size_t ctx_bytes = 0)
{
    bool empty;
    int st = lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O || !den)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const LinPlan p = lin_plan((int)B, (int)S, (int)D, (int)E, LIN_PASS_FWD);
    // context for the fused backward (shapes the fused kernels take): the
    // segment records are the scan workspace itself
    const size_t need = ctx_bytes > 0 || ctx != nullptr
                            ? lin_ctx_bytes((int)B, (int)S, (int)D, (int)E) : 0;
    if (need > 0) {
        if (ctx == nullptr)
            return CXG_ERR_NULL;
        if (ctx_bytes < need)
            return CXG_ERR_WORKSPACE;
        ctx_record(ctx, need, phi, B, S, D, E);
        if (lin_qs_path((int)B, (int)S, (int)D, (int)E))   // features and score blocks
            return hip_status(lin_qs_fwd_launch(phi, Q, K, V, O, den, zc, den_eps, (int)B,
                                                (int)S, (int)D, (int)E, nullptr, s, ctx));
        const LinCtx c = lin_ctx_split(ctx, (int)B, (int)S, (int)D, (int)E);
        return hip_status(lin_fwd_launch(phi, Q, K, V, O, den, zc, S_buf, z_buf, sfin_de,
                                         den_eps, (int)B, (int)S, (int)D, (int)E, c.rec, s, c.tot,
                                         c.zt, c.anch));
    }
    Scratch ws;
    st = ws.acquire(nullptr, 0, lin_ws_bytes(p, (int)B, (int)D, (int)E), s);
    if (st != CXG_OK)
        return st;
    return hip_status(lin_fwd_launch(phi, Q, K, V, O, den, zc, S_buf, z_buf, sfin_de, den_eps,
                                     (int)B, (int)S, (int)D, (int)E, ws.p, s));
}

static int lin_step1_common(const float* O, const float* dO, const float* den, float* dnum,
                            float* dden, size_t N, size_t E, cxg_stream_t stream)
{
    if (E == 0)
        return CXG_ERR_DIMS;
    if (N == 0)
        return CXG_OK;
    if (!fits_int(E) || N > ((size_t)1 << 40) / E || N * 16 > ((size_t)1 << 31) * 255)
        return CXG_ERR_DIMS;
    if (!O || !dO || !den || !dnum || !dden)
        return CXG_ERR_NULL;
    return hip_status(lin_step1_launch(O, dO, den, dnum, dden, (long)N, (int)E,
                                       (hipStream_t)stream));
}

static int lin_dq_common(int phi, const float* K, const float* V, const float* dnum,
                         const float* dden, const float* zc, const float* Q, float* dQ,
                         size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream)
{
    bool empty;
    int st = lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!K || !V || !dnum || !dden || !zc || !dQ || (phi == PHI_ELU1 && !Q))
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const LinPlan p = lin_plan((int)B, (int)S, (int)D, (int)E, LIN_PASS_DQ);
    Scratch ws;
    st = ws.acquire(nullptr, 0, lin_ws_bytes(p, (int)B, (int)D, (int)E), s);
    if (st != CXG_OK)
        return st;
    return hip_status(lin_dq_launch(phi, K, V, dnum, dden, zc, Q, dQ, (int)B, (int)S, (int)D,
                                    (int)E, ws.p, s));
}

static int lin_dkdv_common(int phi, const float* Q, const float* K, const float* V,
                           const float* dnum, const float* dden, float* dK, float* dV, size_t B,
                           size_t S, size_t D, size_t E, cxg_stream_t stream)
{
    bool empty;
    int st = lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !dnum || !dden || !dK || !dV)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const LinPlan p = lin_plan((int)B, (int)S, (int)D, (int)E, LIN_PASS_DKDV);
    Scratch ws;
    st = ws.acquire(nullptr, 0, lin_ws_bytes(p, (int)B, (int)D, (int)E), s);
    if (st != CXG_OK)
        return st;
    return hip_status(lin_dkdv_launch(phi, Q, K, V, dnum, dden, dK, dV, (int)B, (int)S, (int)D,
                                      (int)E, ws.p, s));
}

static int lin_bwd_common(int phi, const float* Q, const float* K, const float* V,
                          const float* O, const float* dO, const float* den, const void* ctx,
                          float* dQ, float* dK, float* dV, size_t B, size_t S, size_t D, size_t E,
                          cxg_stream_t stream)
{
    bool empty;
    int st = lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Q || !K || !V || !O || !dO || !den || !dQ || !dK || !dV)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    Scratch ws;
    if (!lin_bwd_fused_ok((int)D, (int)E, (long)S)) {
        // wide heads (or very long sequences): the split kernels, intermediates in
        // stream-ordered scratch
        if (B * S > ((size_t)1 << 34) / (D + E + 1))
            return CXG_ERR_DIMS;
        // the block-score path takes the forward's context; other shapes write
        // none and ignore it
        const void* qctx = nullptr;
        if (ctx != nullptr && lin_qs_path((int)B, (int)S, (int)D, (int)E)) {
            if (!ctx_matches(ctx, phi, B, S, D, E))
                return CXG_ERR_WORKSPACE;
            qctx = ctx;
        }
        st = ws.acquire(nullptr, 0, lin_bwd_split_ws_bytes((int)B, (int)S, (int)D, (int)E), s);
        if (st != CXG_OK)
            return st;
        return hip_status(lin_bwd_split_launch(phi, Q, K, V, O, dO, den, dQ, dK, dV, (int)B,
                                               (int)S, (int)D, (int)E, ws.p, s, qctx));
    }
    if (ctx != nullptr && !ctx_matches(ctx, phi, B, S, D, E))
        return CXG_ERR_WORKSPACE;
    st = ws.acquire(nullptr, 0,
                    lin_bwd_fused_ws_bytes((int)B, (int)S, (int)D, (int)E, ctx != nullptr), s);
    if (st != CXG_OK)
        return st;
    return hip_status(lin_bwd_fused_launch(phi, Q, K, V, O, dO, den, dQ, dK, dV, (int)B, (int)S,
                                           (int)D, (int)E, ws.p, s, ctx));
}

int cxg_kattn_fwd(const float* Q, const float* K, const float* V, float* O, float* den_cache,
                  float* z_cache, float* S_buf, float* z_buf, size_t B, size_t S, size_t D,
                  size_t E, cxg_stream_t stream)
{
    return lin_fwd_common(PHI_ELU1, 0, 0, Q, K, V, O, den_cache, z_cache, S_buf, z_buf, B, S, D,
                          E, stream);
}

int cxg_kattn_bwd_step1(const float* O, const float* dO, const float* den_cache, float* dnum,
                        float* dden, size_t N, size_t E, cxg_stream_t stream)
{
    return lin_step1_common(O, dO, den_cache, dnum, dden, N, E, stream);
}

int cxg_kattn_bwd_dQ(const float* K, const float* V, const float* dnum, const float* dden,
                     const float* z_cache, const float* Q, float* dQ, float* S_buf, size_t B,
                     size_t S, size_t D, size_t E, cxg_stream_t stream)
{
    (void)S_buf;   // scratch in the reference; the scan keeps its state on chip
    return lin_dq_common(PHI_ELU1, K, V, dnum, dden, z_cache, Q, dQ, B, S, D, E, stream);
}

int cxg_kattn_bwd_dKdV(const float* Q, const float* K, const float* V, const float* dnum,
                       const float* dden, float* dK, float* dV, size_t B, size_t S, size_t D,
                       size_t E, cxg_stream_t stream)
{
    return lin_dkdv_common(PHI_ELU1, Q, K, V, dnum, dden, dK, dV, B, S, D, E, stream);
}

int cxg_kattn_bwd(const float* Q, const float* K, const float* V, const float* O,
                  const float* dO, const float* den_cache, const void* ctx, float* dQ, float* dK,
                  float* dV, size_t B, size_t S, size_t D, size_t E, cxg_stream_t stream)
{
    return lin_bwd_common(PHI_ELU1, Q, K, V, O, dO, den_cache, ctx, dQ, dK, dV, B, S, D, E,
                          stream);
}

// TwoStageGPT's stage 2 with RoPE fused (two_stage_gpt.hpp:113-122 forward,
// :149-160 backward): Q and K are read unrotated and rotated over their whole
// width (head_dim = D).  The chunked scan (D, E <= 64, longer sequences)
// rotates rows as its kernels stage them and rotates dQ, dK back before their
// stores.  The quadratic form (widths up to 512) would rotate every streamed
// block again in each job that reads it, so a pre-pass forms the features
// phi(rot(Q)), phi(rot(K)) once (library scratch), the forward runs on them,
// and the backward streams them and applies phi' and the inverse rotation in
// its output stage.  Wider heads rotate copies of Q and K in scratch, run the
// ELU+1 kernels and rotate dQ and dK back in place.
static int rope_lin_check(size_t B, size_t S, size_t D, size_t E, bool* empty)
{
    int st = lin_check(B, S, D, E, empty);
    if (st != CXG_OK)
        return st;
    if (D % 2 != 0 || D > (size_t)ROPE_MAX_HEAD_DIM)
        return CXG_ERR_DIMS;
    return CXG_OK;
}

int cxg_kattn_rope_fwd(const float* Q, const float* K, const float* V, float* O,
                       float* den_cache, void* ctx, size_t ctx_bytes, size_t B, size_t S,
                       size_t D, size_t E, cxg_stream_t stream)
{
    bool empty;
    int st = rope_lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (lin_bwd_fused_ok((int)D, (int)E, (long)S))   // the chunked scan
        return lin_fwd_common(PHI_ELU1_ROPE, 0, 0, Q, K, V, O, den_cache, nullptr, nullptr,
                              nullptr, B, S, D, E, stream, ctx, ctx_bytes);
    if (!Q || !K || !V || !O || !den_cache)
        return CXG_ERR_NULL;
    hipStream_t s = (hipStream_t)stream;
    const LinPlan p = lin_plan((int)B, (int)S, (int)D, (int)E, LIN_PASS_FWD);
    const size_t t = round_up(B * S * D * sizeof(float), 256);
    // (the RoPE features are formed up to LIN_ROPE_MAX_D wide; wider, the
    // rotated copies below take the split kernels and the context is unused)
    const size_t need = (ctx_bytes > 0 || ctx != nullptr) && D <= (size_t)LIN_ROPE_MAX_D
                            ? lin_ctx_bytes((int)B, (int)S, (int)D, (int)E) : 0;
    if (need > 0) {
        // the block-score path's context: the RoPE features and the score blocks
        if (ctx == nullptr)
            return CXG_ERR_NULL;
        if (ctx_bytes < need)
            return CXG_ERR_WORKSPACE;
        ctx_record(ctx, need, PHI_ELU1_ROPE, B, S, D, E);
        float* fq = lin_qs_ctx_features(ctx, (int)B, (int)S, (int)D, 0);
        float* fk = lin_qs_ctx_features(ctx, (int)B, (int)S, (int)D, 1);
        hipError_t e = lin_rope_feat_launch(Q, K, fq, fk, (int)B, (int)S, (int)D, s);
        if (e == hipSuccess)
            e = lin_qs_fwd_launch(PHI_NONE, fq, fk, V, O, den_cache, nullptr, 0, (int)B, (int)S,
                                  (int)D, (int)E, nullptr, s, ctx);
        return hip_status(e);
    }
    if (p.quad) {
        Scratch ws;
        st = ws.acquire(nullptr, 0, 2 * t + lin_ws_bytes(p, (int)B, (int)D, (int)E), s);
        if (st != CXG_OK)
            return st;
        float* fq = (float*)ws.p;
        float* fk = (float*)((char*)ws.p + t);
        hipError_t e = lin_rope_feat_launch(Q, K, fq, fk, (int)B, (int)S, (int)D, s);
        if (e == hipSuccess)
            e = lin_wide_fwd_launch(PHI_NONE, fq, fk, V, O, den_cache, nullptr, 0, (int)B,
                                    (int)S, (int)D, (int)E, (char*)ws.p + 2 * t, s);
        return hip_status(e);
    }
    Scratch ws;
    st = ws.acquire(nullptr, 0, 2 * t + lin_ws_bytes(p, (int)B, (int)D, (int)E), s);
    if (st != CXG_OK)
        return st;
    float* rq = (float*)ws.p;
    float* rk = (float*)((char*)ws.p + t);
    hipError_t e = hipMemcpyAsync(rq, Q, B * S * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(rk, K, B * S * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = rope_launch(rq, rk, (long)B, (int)S, (int)D, (int)D, 1.0f, s);
    if (e == hipSuccess)
        e = lin_fwd_launch(PHI_ELU1, rq, rk, V, O, den_cache, nullptr, nullptr, nullptr, 0, 0,
                           (int)B, (int)S, (int)D, (int)E, (char*)ws.p + 2 * t, s);
    return hip_status(e);
}

int cxg_kattn_rope_bwd(const float* Q, const float* K, const float* V, const float* O,
                       const float* dO, const float* den_cache, const void* ctx, float* dQ,
                       float* dK, float* dV, size_t B, size_t S, size_t D, size_t E,
                       cxg_stream_t stream)
{
    bool empty;
    int st = rope_lin_check(B, S, D, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (lin_bwd_fused_ok((int)D, (int)E, (long)S))   // the chunked scan
        return lin_bwd_common(PHI_ELU1_ROPE, Q, K, V, O, dO, den_cache, ctx, dQ, dK, dV, B, S, D,
                              E, stream);
    if (!Q || !K || !V || !O || !dO || !den_cache || !dQ || !dK || !dV)
        return CXG_ERR_NULL;
    if (B * S > ((size_t)1 << 34) / (D + E + 1))
        return CXG_ERR_DIMS;
    hipStream_t s = (hipStream_t)stream;
    const size_t t = round_up(B * S * D * sizeof(float), 256);
    if (ctx != nullptr && D <= (size_t)LIN_ROPE_MAX_D &&
        lin_qs_path((int)B, (int)S, (int)D, (int)E)) {
        // the forward's context: its RoPE features and score blocks
        if (!ctx_matches(ctx, PHI_ELU1_ROPE, B, S, D, E))
            return CXG_ERR_WORKSPACE;
        const size_t N = B * S, tn = round_up(N * E * sizeof(float), 256);
        const size_t tq = lin_wide_bwd_ws_bytes((int)B, (int)S, (int)D, (int)E, 3);
        Scratch ws;
        st = ws.acquire(nullptr, 0, tn + round_up(N * sizeof(float), 256) + tq, s);
        if (st != CXG_OK)
            return st;
        float* dnum = (float*)ws.p;
        float* dden = (float*)((char*)ws.p + tn);
        float* fq = lin_qs_ctx_features(const_cast<void*>(ctx), (int)B, (int)S, (int)D, 0);
        float* fk = lin_qs_ctx_features(const_cast<void*>(ctx), (int)B, (int)S, (int)D, 1);
        hipError_t e = lin_step1_launch(O, dO, den_cache, dnum, dden, (long)N, (int)E, s);
        if (e == hipSuccess)
            e = lin_qs_bwd_launch(PHI_ELU1_ROPE, fq, fk, V, dnum, dden, dQ, dK, dV, (int)B,
                                  (int)S, (int)D, (int)E, 3,
                                  (char*)ws.p + tn + round_up(N * sizeof(float), 256), s, Q, K,
                                  ctx);
        return hip_status(e);
    }
    if (lin_quad_ok((int)D, (int)E, (long)S)) {
        const size_t N = B * S, tn = round_up(N * E * sizeof(float), 256);
        const size_t tq = lin_wide_bwd_ws_bytes((int)B, (int)S, (int)D, (int)E, 3);
        Scratch ws;
        st = ws.acquire(nullptr, 0, 2 * t + tn + round_up(N * sizeof(float), 256) + tq, s);
        if (st != CXG_OK)
            return st;
        float* fq = (float*)ws.p;
        float* fk = (float*)((char*)ws.p + t);
        float* dnum = (float*)((char*)ws.p + 2 * t);
        float* dden = (float*)((char*)ws.p + 2 * t + tn);
        hipError_t e = lin_rope_feat_launch(Q, K, fq, fk, (int)B, (int)S, (int)D, s);
        if (e == hipSuccess)
            e = lin_step1_launch(O, dO, den_cache, dnum, dden, (long)N, (int)E, s);
        if (e == hipSuccess)
            e = lin_wide_bwd_launch(
                PHI_ELU1_ROPE, fq, fk, V, dnum, dden, dQ, dK, dV, (int)B, (int)S, (int)D, (int)E,
                3, s, Q, K,
                tq ? (char*)ws.p + 2 * t + tn + round_up(N * sizeof(float), 256) : nullptr);
        return hip_status(e);
    }
    Scratch ws;
    st = ws.acquire(nullptr, 0,
                    2 * t + lin_bwd_split_ws_bytes((int)B, (int)S, (int)D, (int)E), s);
    if (st != CXG_OK)
        return st;
    float* rq = (float*)ws.p;
    float* rk = (float*)((char*)ws.p + t);
    hipError_t e = hipMemcpyAsync(rq, Q, B * S * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(rk, K, B * S * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = rope_launch(rq, rk, (long)B, (int)S, (int)D, (int)D, 1.0f, s);
    if (e == hipSuccess)
        e = lin_bwd_split_launch(PHI_ELU1, rq, rk, V, O, dO, den_cache, dQ, dK, dV, (int)B,
                                 (int)S, (int)D, (int)E, (char*)ws.p + 2 * t, s);
    if (e == hipSuccess)
        e = rope_launch(dQ, dK, (long)B, (int)S, (int)D, (int)D, -1.0f, s);
    return hip_status(e);
}

size_t cxg_lin_ctx_size(size_t B, size_t S, size_t D, size_t E)
{
    bool empty;
    if (lin_check(B, S, D, E, &empty) != CXG_OK || empty)
        return 0;
    return lin_ctx_bytes((int)B, (int)S, (int)D, (int)E);
}

int cxg_kattn_fwd_ctx(const float* Q, const float* K, const float* V, float* O,
                      float* den_cache, void* ctx, size_t ctx_bytes, size_t B, size_t S,
                      size_t D, size_t E, cxg_stream_t stream)
{
    return lin_fwd_common(PHI_ELU1, 0, 0, Q, K, V, O, den_cache, nullptr, nullptr, nullptr, B, S,
                          D, E, stream, ctx, ctx_bytes);
}

int cxg_lin_fwd_ctx(const float* Q_phi, const float* K_phi, const float* V, float* O,
                    float* den_cache, void* ctx, size_t ctx_bytes, size_t B, size_t S, size_t D,
                    size_t E, cxg_stream_t stream)
{
    return lin_fwd_common(PHI_NONE, 1, 1, Q_phi, K_phi, V, O, den_cache, nullptr, nullptr,
                          nullptr, B, S, D, E, stream, ctx, ctx_bytes);
}

int cxg_lin_fwd(const float* Q_phi, const float* K_phi, const float* V, float* O,
                float* den_cache, float* z_cache, float* S_buf, float* z_buf, size_t B, size_t S,
                size_t D, size_t E, cxg_stream_t stream)
{
    return lin_fwd_common(PHI_NONE, 1, 1, Q_phi, K_phi, V, O, den_cache, z_cache, S_buf, z_buf,
                          B, S, D, E, stream);
}

int cxg_lin_bwd_step1(const float* O, const float* dO, const float* den_cache, float* dnum,
                      float* dden, size_t N, size_t E, cxg_stream_t stream)
{
    return lin_step1_common(O, dO, den_cache, dnum, dden, N, E, stream);
}

int cxg_lin_bwd_dQ(const float* K_phi, const float* V, const float* dnum, const float* dden,
                   const float* z_cache, float* dQ_phi, float* S_buf, size_t B, size_t S,
                   size_t D, size_t E, cxg_stream_t stream)
{
    (void)S_buf;
    return lin_dq_common(PHI_NONE, K_phi, V, dnum, dden, z_cache, nullptr, dQ_phi, B, S, D, E,
                         stream);
}

int cxg_lin_bwd_dKdV(const float* Q_phi, const float* K_phi, const float* V, const float* dnum,
                     const float* dden, float* dK_phi, float* dV, size_t B, size_t S, size_t D,
                     size_t E, cxg_stream_t stream)
{
    return lin_dkdv_common(PHI_NONE, Q_phi, K_phi, V, dnum, dden, dK_phi, dV, B, S, D, E,
                           stream);
}

int cxg_lin_bwd(const float* Q_phi, const float* K_phi, const float* V, const float* O,
                const float* dO, const float* den_cache, const void* ctx, float* dQ_phi,
                float* dK_phi, float* dV, size_t B, size_t S, size_t D, size_t E,
                cxg_stream_t stream)
{
    return lin_bwd_common(PHI_NONE, Q_phi, K_phi, V, O, dO, den_cache, ctx, dQ_phi, dK_phi, dV,
                          B, S, D, E, stream);
}

int cxg_lin_elu_fwd(const float* Xq, const float* Xk, const float* V, float* O,
                    float* den_cache, void* ctx, size_t ctx_bytes, size_t B, size_t S, size_t E,
                    cxg_stream_t stream)
{
    return lin_fwd_common(PHI_ELU1_LG, 1, 1, Xq, Xk, V, O, den_cache, nullptr, nullptr, nullptr,
                          B, S, E, E, stream, ctx, ctx_bytes);
}

int cxg_lin_elu_bwd(const float* Xq, const float* Xk, const float* V, const float* O,
                    const float* dO, const float* den_cache, const void* ctx, float* dXq,
                    float* dXk, float* dV, size_t B, size_t S, size_t E, cxg_stream_t stream)
{
    return lin_bwd_common(PHI_ELU1_LG, Xq, Xk, V, O, dO, den_cache, ctx, dXq, dXk, dV, B, S, E,
                          E, stream);
}

// Hadamard+Exp attention block: the feature map fused into the fused pair's
// kernels (E = D = 64, one Hadamard block, 16-byte aligned rows).  Sequences
// the quadratic form takes (S <= LIN_QUAD_MAX_S) run the feature-map kernels
// into scratch around the PHI_NONE kernels instead; they use no context.
static size_t al256b(size_t b) { return (b + 255) / 256 * 256; }

static int hexp_check(size_t B, size_t S, size_t E, bool* empty)
{
    int st = lin_check(B, S, E, E, empty);
    if (st != CXG_OK || *empty)
        return st;
    if (E != 64 || S >= ((size_t)1 << 22))
        return CXG_ERR_DIMS;
    return CXG_OK;
}

int cxg_lin_hexp_fwd(const float* Xq, const float* Xk, const float* V, float* O,
                     float* den_cache, void* ctx, size_t ctx_bytes, size_t B, size_t S, size_t E,
                     cxg_stream_t stream)
{
    bool empty;
    int st = hexp_check(B, S, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Xq || !Xk || !V || !O || !den_cache)
        return CXG_ERR_NULL;
    if (!al16c(Xq) || !al16c(Xk) || !al16c(V) || !al16c(O))
        return CXG_ERR_ALIGN;
    if (!lin_quad_ok(64, 64, (long)S))
        return lin_fwd_common(PHI_HEXP, 1, 1, Xq, Xk, V, O, den_cache, nullptr, nullptr, nullptr,
                              B, S, 64, 64, stream, ctx, ctx_bytes);
    hipStream_t s = (hipStream_t)stream;
    const size_t N = B * S, t = al256b(N * 64 * sizeof(float));
    Scratch ws;
    st = ws.acquire(nullptr, 0, 2 * t, s);
    if (st != CXG_OK)
        return st;
    float* pq = (float*)ws.p;
    float* pk = (float*)((char*)ws.p + t);
    hipError_t e = phi_hexp_fwd_launch(Xq, pq, (long)N, 64, 64, s);
    if (e == hipSuccess)
        e = phi_hexp_fwd_launch(Xk, pk, (long)N, 64, 64, s);
    if (e == hipSuccess)
        e = lin_wide_fwd_launch(PHI_NONE, pq, pk, V, O, den_cache, nullptr, 1, (int)B, (int)S, 64,
                                64, nullptr, s);
    return hip_status(e);
}

int cxg_lin_hexp_bwd(const float* Xq, const float* Xk, const float* V, const float* O,
                     const float* dO, const float* den_cache, const void* ctx, float* dXq,
                     float* dXk, float* dV, size_t B, size_t S, size_t E, cxg_stream_t stream)
{
    bool empty;
    int st = hexp_check(B, S, E, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!Xq || !Xk || !V || !O || !dO || !den_cache || !dXq || !dXk || !dV)
        return CXG_ERR_NULL;
    if (!al16c(Xq) || !al16c(Xk) || !al16c(V) || !al16c(O) || !al16c(dO) || !al16c(dXq) ||
        !al16c(dXk) || !al16c(dV))
        return CXG_ERR_ALIGN;
    if (!lin_quad_ok(64, 64, (long)S))
        return lin_bwd_common(PHI_HEXP, Xq, Xk, V, O, dO, den_cache, ctx, dXq, dXk, dV, B, S, 64,
                              64, stream);
    hipStream_t s = (hipStream_t)stream;
    const size_t N = B * S, t = al256b(N * 64 * sizeof(float));
    const size_t wsb = lin_bwd_split_ws_bytes((int)B, (int)S, 64, 64);
    Scratch ws;
    st = ws.acquire(nullptr, 0, 4 * t + wsb, s);
    if (st != CXG_OK)
        return st;
    char* p = (char*)ws.p;
    float *pq = (float*)p, *pk = (float*)(p + t), *dpq = (float*)(p + 2 * t),
          *dpk = (float*)(p + 3 * t);
    hipError_t e = phi_hexp_fwd_launch(Xq, pq, (long)N, 64, 64, s);
    if (e == hipSuccess)
        e = phi_hexp_fwd_launch(Xk, pk, (long)N, 64, 64, s);
    if (e == hipSuccess)
        e = lin_bwd_split_launch(PHI_NONE, pq, pk, V, O, dO, den_cache, dpq, dpk, dV, (int)B,
                                 (int)S, 64, 64, p + 4 * t, s);
    if (e == hipSuccess)
        e = phi_hexp_bwd_launch(dpq, Xq, dXq, (long)N, 64, 64, s);
    if (e == hipSuccess)
        e = phi_hexp_bwd_launch(dpk, Xk, dXk, (long)N, 64, 64, s);
    return hip_status(e);
}

static int phi_check(size_t N, size_t D, size_t E, bool hexp, bool* empty)
{
    *empty = (N == 0);
    if (D == 0 || E == 0 || D < E)
        return CXG_ERR_DIMS;
    if (hexp && E % 64 != 0)
        return CXG_ERR_DIMS;
    if (*empty)
        return CXG_OK;
    if (!fits_int(D) || N > ((size_t)1 << 38) / D)
        return CXG_ERR_DIMS;
    return CXG_OK;
}

int cxg_phi_elu_fwd(const float* x, float* phi, size_t N, size_t D, size_t E,
                    cxg_stream_t stream)
{
    bool empty;
    int st = phi_check(N, D, E, false, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!x || !phi)
        return CXG_ERR_NULL;
    return hip_status(phi_elu_fwd_launch(x, phi, (long)N, (int)D, (int)E, (hipStream_t)stream));
}

int cxg_phi_elu_bwd(const float* dphi, const float* x, float* dx, size_t N, size_t D, size_t E,
                    cxg_stream_t stream)
{
    bool empty;
    int st = phi_check(N, D, E, false, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!dphi || !x || !dx)
        return CXG_ERR_NULL;
    return hip_status(
        phi_elu_bwd_launch(dphi, x, dx, (long)N, (int)D, (int)E, (hipStream_t)stream));
}

int cxg_phi_hexp_fwd(const float* x, float* phi, size_t N, size_t D, size_t E,
                     cxg_stream_t stream)
{
    bool empty;
    int st = phi_check(N, D, E, true, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!x || !phi)
        return CXG_ERR_NULL;
    return hip_status(phi_hexp_fwd_launch(x, phi, (long)N, (int)D, (int)E, (hipStream_t)stream));
}

int cxg_phi_hexp_bwd(const float* dphi, const float* x, float* dx, size_t N, size_t D, size_t E,
                     cxg_stream_t stream)
{
    bool empty;
    int st = phi_check(N, D, E, true, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!dphi || !x || !dx)
        return CXG_ERR_NULL;
    return hip_status(
        phi_hexp_bwd_launch(dphi, x, dx, (long)N, (int)D, (int)E, (hipStream_t)stream));
}

// ---------------------------------------------------------------------------
// exact GELU
// ---------------------------------------------------------------------------
static int gelu_common(const float* A, float* C, size_t n, bool deriv, cxg_stream_t stream)
{
    if (n == 0)
        return CXG_OK;
    if (n > ((size_t)1 << 40))
        return CXG_ERR_DIMS;
    if (!A || !C)
        return CXG_ERR_NULL;
    return hip_status(gelu_launch(A, C, (long)n, deriv, (hipStream_t)stream));
}

int cxg_gelu_exact(const float* A, float* C, size_t n, cxg_stream_t stream)
{
    return gelu_common(A, C, n, false, stream);
}

int cxg_gelu_exact_deriv(const float* A, float* C, size_t n, cxg_stream_t stream)
{
    return gelu_common(A, C, n, true, stream);
}

// ---------------------------------------------------------------------------
// expander FFN (Linear -> exact GELU -> Linear, no bias)
// ---------------------------------------------------------------------------
static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static int ffn_check(size_t M, size_t E, size_t F, bool* empty)
{
    *empty = M == 0;
    if (E == 0 || F == 0)
        return CXG_ERR_DIMS;
    if (!fits_int(M) || !fits_int(E) || !fits_int(F) || M * F > ((size_t)1 << 40) ||
        M * E > ((size_t)1 << 40) || E * F > ((size_t)1 << 40))
        return CXG_ERR_DIMS;
    if (E % 4 != 0 || F % 4 != 0)
        return CXG_ERR_ALIGN;
    return CXG_OK;
}

static size_t ffn_fwd_ws(int M, int E, int F)
{
    return std::max(ffn_gemm_ws_floats(M, F, E), ffn_gemm_ws_floats(M, E, F));
}

static size_t ffn_bwd_ws(int M, int E, int F)
{
    size_t part = std::max(std::max(ffn_gemm_ws_floats(M, F, E), ffn_gemm_ws_floats(E, F, M)),
                           std::max(ffn_gemm_ws_floats(M, E, F), ffn_gemm_ws_floats(F, E, M)));
    return round_up((size_t)M * F, 64) + part;
}

size_t cxg_ffn_workspace_size(size_t M, size_t E, size_t F)
{
    bool empty;
    if (ffn_check(M, E, F, &empty) != CXG_OK || empty)
        return 0;
    const size_t fl = std::max(ffn_fwd_ws((int)M, (int)E, (int)F), ffn_bwd_ws((int)M, (int)E, (int)F));
    return round_up(fl * sizeof(float), 256);
}

int cxg_ffn_fwd(const float* X, const float* W1, const float* W2, float* pre, float* act,
                float* Y, size_t M, size_t E, size_t F, void* workspace, size_t ws_bytes,
                cxg_stream_t stream)
{
    bool empty;
    int st = ffn_check(M, E, F, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!X || !W1 || !W2 || !act || !Y)
        return CXG_ERR_NULL;
    for (const void* p : {(const void*)X, (const void*)W1, (const void*)W2, (const void*)pre,
                          (const void*)act, (const void*)Y})
        if (!aligned16(p))
            return CXG_ERR_ALIGN;
    const int m = (int)M, e = (int)E, f = (int)F;
    hipStream_t hs = (hipStream_t)stream;
    Scratch ws;
    st = ws.acquire(workspace, ws_bytes, ffn_fwd_ws(m, e, f) * sizeof(float), hs);
    if (st != CXG_OK)
        return st;
    float* part = (float*)ws.p;
    FfnGemm fc{X, e, true, W1, e, true, m, f, e, FFN_EPI_GELU, act, f, nullptr, pre};
    FfnGemm proj{act, f, true, W2, f, true, m, e, f, FFN_EPI_STORE, Y, e, nullptr, nullptr};
    hipError_t he = ffn_gemm_launch(fc, part, hs);
    if (he == hipSuccess)
        he = ffn_gemm_launch(proj, part, hs);
    return hip_status(he);
}

int cxg_ffn_bwd(const float* X, const float* W1, const float* W2, const float* act,
                const float* G, const float* dY, float* dX, float* dW1, float* dW2, size_t M,
                size_t E, size_t F, void* workspace, size_t ws_bytes, cxg_stream_t stream)
{
    bool empty;
    int st = ffn_check(M, E, F, &empty);
    if (st != CXG_OK || empty)
        return st;
    if (!X || !W1 || !W2 || !act || !G || !dY || !dX || !dW1 || !dW2)
        return CXG_ERR_NULL;
    for (const void* p : {(const void*)X, (const void*)W1, (const void*)W2, (const void*)act,
                          (const void*)G, (const void*)dY, (const void*)dX, (const void*)dW1,
                          (const void*)dW2})
        if (!aligned16(p))
            return CXG_ERR_ALIGN;
    const int m = (int)M, e = (int)E, f = (int)F;
    hipStream_t hs = (hipStream_t)stream;
    Scratch ws;
    st = ws.acquire(workspace, ws_bytes, ffn_bwd_ws(m, e, f) * sizeof(float), hs);
    if (st != CXG_OK)
        return st;
    float* dact = (float*)ws.p;
    float* part = dact + round_up((size_t)M * F, 64);
    FfnGemm dp{dY, e, true, W2, f, false, m, f, e, FFN_EPI_DGELU, dact, f, G, nullptr};
    FfnGemm w2{dY, e, false, act, f, false, e, f, m, FFN_EPI_ACCUM, dW2, f, nullptr, nullptr};
    FfnGemm dx{dact, f, true, W1, e, false, m, e, f, FFN_EPI_STORE, dX, e, nullptr, nullptr};
    FfnGemm w1{dact, f, false, X, e, false, f, e, m, FFN_EPI_ACCUM, dW1, e, nullptr, nullptr};
    hipError_t he = ffn_gemm_launch(dp, part, hs);
    if (he == hipSuccess)
        he = ffn_gemm_launch(w2, part, hs);
    if (he == hipSuccess)
        he = ffn_gemm_launch(dx, part, hs);
    if (he == hipSuccess)
        he = ffn_gemm_launch(w1, part, hs);
    return hip_status(he);
}

// ---------------------------------------------------------------------------
// rotary position embedding
// ---------------------------------------------------------------------------
static int rope_common(float* Q, float* K, size_t B, size_t S, size_t D, size_t head_dim,
                       float sign, cxg_stream_t stream)
{
    if (head_dim < 2 || head_dim % 2 != 0 || head_dim > (size_t)ROPE_MAX_HEAD_DIM ||
        D % head_dim != 0)
        return CXG_ERR_DIMS;
    if (B == 0 || S == 0 || D == 0)
        return CXG_OK;
    if (!fits_int(S) || !fits_int(D) || B > ((size_t)1 << 40) / S ||
        B * S > ((size_t)1 << 42) / D)
        return CXG_ERR_DIMS;
    if (!Q && !K)
        return CXG_ERR_NULL;
    return hip_status(rope_launch(Q, K, (long)B, (int)S, (int)D, (int)head_dim, sign,
                                  (hipStream_t)stream));
}

int cxg_rope_fwd(float* Q, float* K, size_t B, size_t S, size_t D, size_t head_dim,
                 cxg_stream_t stream)
{
    return rope_common(Q, K, B, S, D, head_dim, 1.0f, stream);
}

int cxg_rope_bwd(float* dQ, float* dK, size_t B, size_t S, size_t D, size_t head_dim,
                 cxg_stream_t stream)
{
    return rope_common(dQ, dK, B, S, D, head_dim, -1.0f, stream);
}

// ---------------------------------------------------------------------------
// timing hook
// ---------------------------------------------------------------------------
void cxg_prof_enable(int on)
{
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_on = on != 0;
}

void cxg_prof_reset(void)
{
    std::lock_guard<std::mutex> lk(g_prof_mu);
    for (auto& r : g_prof_recs) {
        (void)hipEventSynchronize(r.b);
        g_prof_free.push_back(r.a);
        g_prof_free.push_back(r.b);
    }
    g_prof_recs.clear();
}

int cxg_prof_query(const char* kernel_name, double* total_ms, int* count)
{
    std::lock_guard<std::mutex> lk(g_prof_mu);
    double tot = 0.0;
    int n = 0;
    for (auto& r : g_prof_recs) {
        if (r.name != kernel_name)
            continue;
        (void)hipEventSynchronize(r.b);
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            tot += ms;
            n++;
        }
    }
    if (total_ms)
        *total_ms = tot;
    if (count)
        *count = n;
    return n > 0 ? 0 : -1;
}

} // extern "C"
