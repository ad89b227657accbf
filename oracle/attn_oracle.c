/*
 * attn_oracle.c -- CPU restatement of CXX-GPT's attention CPU reference.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Build with -ffp-contract=off and without -ffast-math: every routine keeps
 * the reference's fp32 operation sequence, and an FMA contraction would
 * change its rounding.  Citations are relative to the reference tree.
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* thread helper: run fn(ctx, i) for i in [0, n) over nthreads threads */
/* ------------------------------------------------------------------ */
typedef void (*orc_task_fn)(void *ctx, size_t i);
typedef struct {
    orc_task_fn fn;
    void *ctx;
    size_t n;
    size_t next;
    pthread_mutex_t mu;
} orc_pool;

static void *orc_worker(void *arg)
{
    orc_pool *p = (orc_pool *)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        size_t i = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (i >= p->n)
            break;
        p->fn(p->ctx, i);
    }
    return NULL;
}

static void orc_parallel_for(size_t n, int nthreads, orc_task_fn fn, void *ctx)
{
    if (nthreads <= 1 || n <= 1) {
        for (size_t i = 0; i < n; i++)
            fn(ctx, i);
        return;
    }
    if ((size_t)nthreads > n)
        nthreads = (int)n;
    orc_pool p;
    p.fn = fn;
    p.ctx = ctx;
    p.n = n;
    p.next = 0;
    pthread_mutex_init(&p.mu, NULL);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    for (int t = 0; t < nthreads; t++)
        pthread_create(&th[t], NULL, orc_worker, &p);
    for (int t = 0; t < nthreads; t++)
        pthread_join(th[t], NULL);
    free(th);
    pthread_mutex_destroy(&p.mu);
}

/* ------------------------------------------------------------------ */
/* MT19937 (Matsumoto & Nishimura, ACM TOMACS 8(1), 1998)              */
/* ------------------------------------------------------------------ */
void orc_mt_seed(orc_mt19937 *g, uint32_t seed)
{
    g->mt[0] = seed;
    for (int i = 1; i < 624; i++)
        g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
    g->idx = 624;
}

uint32_t orc_mt_next(orc_mt19937 *g)
{
    if (g->idx >= 624) {
        for (int i = 0; i < 624; i++) {
            uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
            uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
            if (y & 1u)
                v ^= 0x9908b0dfu;
            g->mt[i] = v;
        }
        g->idx = 0;
    }
    uint32_t y = g->mt[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* kernel_test.cpp:14: (float)rgen() / (float)rgen.max() * 2.0f - 1.0f */
float orc_mt_frand(orc_mt19937 *g)
{
    return (float)orc_mt_next(g) / (float)4294967295u * 2.0f - 1.0f;
}

void orc_mt_fill_frand(orc_mt19937 *g, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++)
        out[i] = orc_mt_frand(g);
}

/* splitmix64 (Steele, Lea, Flood 2014) feeding Box-Muller (1958). */
static uint64_t orc_splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void orc_fill_normal(uint64_t seed, float mean, float stdev, float *out, size_t n)
{
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        /* u1 in (0,1], u2 in [0,1) from the top 53 bits */
        double u1 = ((double)(orc_splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(orc_splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stdev * r * cos(two_pi * u2));
        if (i + 1 < n)
            out[i + 1] = (float)(mean + stdev * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------------ */
/* softmax MHA                                                          */
/* ------------------------------------------------------------------ */
/* kernel_test.cpp:19-22 */
static inline size_t idx3(size_t b, size_t s, size_t h, size_t c, size_t S, size_t H, size_t Dh)
{
    return ((b * S + s) * H + h) * Dh + c;
}

/* std::max(a, b) == (a < b) ? b : a */
static inline float orc_max(float a, float b) { return (a < b) ? b : a; }

/* ref_mha_fwd (kernel_test.cpp:24-46): one output element. */
static float ref_mha_fwd_elem(const float *Q, const float *K, const float *V, size_t b,
                              size_t s, size_t h, size_t c, size_t S, size_t H, size_t Dh,
                              float *scores)
{
    float scale = 1.0f / sqrtf((float)Dh);
    float m = -1e30f;
    for (size_t t = 0; t <= s; t++) {
        float acc = 0.0f;
        for (size_t d = 0; d < Dh; d++)
            acc += Q[idx3(b, s, h, d, S, H, Dh)] * K[idx3(b, t, h, d, S, H, Dh)];
        scores[t] = acc * scale;
        m = orc_max(m, scores[t]);
    }
    float l = 0.0f;
    for (size_t t = 0; t <= s; t++)
        l += expf(scores[t] - m);
    float out = 0.0f;
    for (size_t t = 0; t <= s; t++)
        out += expf(scores[t] - m) / l * V[idx3(b, t, h, c, S, H, Dh)];
    return out;
}

void orc_mha_fwd_literal(const float *Q, const float *K, const float *V, float *O,
                         size_t B, size_t S, size_t H, size_t Dh)
{
    float *scores = (float *)malloc(sizeof(float) * (S ? S : 1));
    /* call loop of kernel_test.cpp:233-238 */
    for (size_t b = 0; b < B; b++)
        for (size_t s = 0; s < S; s++)
            for (size_t h = 0; h < H; h++)
                for (size_t c = 0; c < Dh; c++)
                    O[idx3(b, s, h, c, S, H, Dh)] =
                        ref_mha_fwd_elem(Q, K, V, b, s, h, c, S, H, Dh, scores);
    free(scores);
}

typedef struct {
    const float *Q, *K, *V, *O, *dO;
    float *Oout, *lse, *dQ, *dK, *dV;
    size_t B, S, H, Dh;
    const size_t *heads;
} mha_ctx;

/* Row form of ref_mha_fwd for one (b,h): identical per-element float ops. */
static void mha_fwd_head(void *vctx, size_t i)
{
    mha_ctx *c = (mha_ctx *)vctx;
    size_t bh = c->heads ? c->heads[i] : i;
    size_t B = c->B, S = c->S, H = c->H, Dh = c->Dh;
    size_t b = bh / H, h = bh % H;
    (void)B;
    float scale = 1.0f / sqrtf((float)Dh);
    float *scores = (float *)malloc(sizeof(float) * S);
    float *ex = (float *)malloc(sizeof(float) * S);
    for (size_t s = 0; s < S; s++) {
        float m = -1e30f;
        for (size_t t = 0; t <= s; t++) {
            float acc = 0.0f;
            for (size_t d = 0; d < Dh; d++)
                acc += c->Q[idx3(b, s, h, d, S, H, Dh)] * c->K[idx3(b, t, h, d, S, H, Dh)];
            scores[t] = acc * scale;
            m = orc_max(m, scores[t]);
        }
        float l = 0.0f;
        for (size_t t = 0; t <= s; t++) {
            ex[t] = expf(scores[t] - m);
            l += ex[t];
        }
        if (c->lse)
            c->lse[bh * S + s] = m + logf(l);
        for (size_t cc = 0; cc < Dh; cc++) {
            float out = 0.0f;
            for (size_t t = 0; t <= s; t++)
                out += ex[t] / l * c->V[idx3(b, t, h, cc, S, H, Dh)];
            c->Oout[idx3(b, s, h, cc, S, H, Dh)] = out;
        }
    }
    free(scores);
    free(ex);
}

void orc_mha_fwd(const float *Q, const float *K, const float *V, float *O, float *lse,
                 size_t B, size_t S, size_t H, size_t Dh, int nthreads)
{
    mha_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.Oout = O; c.lse = lse;
    c.B = B; c.S = S; c.H = H; c.Dh = Dh;
    if (S == 0)
        return;
    orc_parallel_for(B * H, nthreads, mha_fwd_head, &c);
}

void orc_mha_fwd_heads(const float *Q, const float *K, const float *V, float *O,
                       size_t B, size_t S, size_t H, size_t Dh,
                       const size_t *heads, size_t nheads, int nthreads)
{
    mha_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.Oout = O;
    c.B = B; c.S = S; c.H = H; c.Dh = Dh; c.heads = heads;
    if (S == 0)
        return;
    orc_parallel_for(nheads, nthreads, mha_fwd_head, &c);
}

/* ref_mha_bwd (kernel_test.cpp:48-94) for one (b,h).  The reference loops
 * b, s, h, t; for fixed (b,h) the per-element accumulation order over s and
 * t is the same as here. */
static void mha_bwd_head(void *vctx, size_t i)
{
    mha_ctx *c = (mha_ctx *)vctx;
    size_t bh = c->heads ? c->heads[i] : i;
    size_t S = c->S, H = c->H, Dh = c->Dh;
    size_t b = bh / H, h = bh % H;
    const float *Q = c->Q, *K = c->K, *V = c->V, *O = c->O, *dO = c->dO;
    float *dQ = c->dQ, *dK = c->dK, *dV = c->dV;
    float scale = 1.0f / sqrtf((float)Dh);
    for (size_t s = 0; s < S; s++)
        for (size_t cc = 0; cc < Dh; cc++) {
            dQ[idx3(b, s, h, cc, S, H, Dh)] = 0.0f;
            dK[idx3(b, s, h, cc, S, H, Dh)] = 0.0f;
            dV[idx3(b, s, h, cc, S, H, Dh)] = 0.0f;
        }
    float *p = (float *)malloc(sizeof(float) * S);
    float *score = (float *)malloc(sizeof(float) * S);
    for (size_t s = 0; s < S; s++) {
        float m = -1e30f;
        for (size_t t = 0; t <= s; t++) {
            float acc = 0.0f;
            for (size_t d = 0; d < Dh; d++)
                acc += Q[idx3(b, s, h, d, S, H, Dh)] * K[idx3(b, t, h, d, S, H, Dh)];
            score[t] = acc * scale;
            m = orc_max(m, score[t]);
        }
        float l = 0.0f;
        for (size_t t = 0; t <= s; t++) {
            p[t] = expf(score[t] - m);
            l += p[t];
        }
        float gs = 0.0f; /* dO_s . O_s */
        for (size_t cc = 0; cc < Dh; cc++)
            gs += dO[idx3(b, s, h, cc, S, H, Dh)] * O[idx3(b, s, h, cc, S, H, Dh)];
        for (size_t t = 0; t <= s; t++) {
            float pv = p[t] / l;
            float ds = 0.0f; /* dO_s . v_t */
            for (size_t cc = 0; cc < Dh; cc++)
                ds += dO[idx3(b, s, h, cc, S, H, Dh)] * V[idx3(b, t, h, cc, S, H, Dh)];
            float dscore = pv * (ds - gs);
            for (size_t cc = 0; cc < Dh; cc++) {
                dQ[idx3(b, s, h, cc, S, H, Dh)] += scale * dscore * K[idx3(b, t, h, cc, S, H, Dh)];
                dK[idx3(b, t, h, cc, S, H, Dh)] += scale * dscore * Q[idx3(b, s, h, cc, S, H, Dh)];
                dV[idx3(b, t, h, cc, S, H, Dh)] += pv * dO[idx3(b, s, h, cc, S, H, Dh)];
            }
        }
    }
    free(p);
    free(score);
}

void orc_mha_bwd(const float *Q, const float *K, const float *V, const float *O,
                 const float *dO, float *dQ, float *dK, float *dV,
                 size_t B, size_t S, size_t H, size_t Dh, int nthreads)
{
    mha_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.O = O; c.dO = dO;
    c.dQ = dQ; c.dK = dK; c.dV = dV;
    c.B = B; c.S = S; c.H = H; c.Dh = Dh;
    if (S == 0)
        return;
    orc_parallel_for(B * H, nthreads, mha_bwd_head, &c);
}

void orc_mha_bwd_heads(const float *Q, const float *K, const float *V, const float *O,
                       const float *dO, float *dQ, float *dK, float *dV,
                       size_t B, size_t S, size_t H, size_t Dh,
                       const size_t *heads, size_t nheads, int nthreads)
{
    mha_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.O = O; c.dO = dO;
    c.dQ = dQ; c.dK = dK; c.dV = dV;
    c.B = B; c.S = S; c.H = H; c.Dh = Dh; c.heads = heads;
    if (S == 0)
        return;
    orc_parallel_for(nheads, nthreads, mha_bwd_head, &c);
}

/* ------------------------------------------------------------------ */
/* ELU+1 linear attention, two_stage API                               */
/* ------------------------------------------------------------------ */
float orc_phi_elu(float x) { return x > 0.0f ? x + 1.0f : expf(x); }     /* kernel_test.cpp:16 */
float orc_phi_elu_der(float x) { return x > 0.0f ? 1.0f : expf(x); }     /* kernel_test.cpp:17 */

typedef struct {
    const float *Q, *K, *V, *O, *dO, *den, *dnum, *dden, *zc;
    float *Oout, *denout, *zcout, *dQ, *dK, *dV, *Sbuf, *zbuf;
    size_t S, D, E;
} lin_ctx;

/* ref_kernel_attn_fwd (kernel_test.cpp:96-126) for one sequence b. */
static void kattn_fwd_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *z = (float *)calloc(D, sizeof(float));
    float *state = (float *)calloc(E * D, sizeof(float));
    for (size_t t = 0; t < S; t++) {
        size_t idx = b * S + t;
        for (size_t d = 0; d < D; d++) {
            z[d] += orc_phi_elu(c->K[idx * D + d]);
            for (size_t e = 0; e < E; e++)
                state[e * D + d] += orc_phi_elu(c->K[idx * D + d]) * c->V[idx * E + e];
        }
        if (c->zcout)
            for (size_t d = 0; d < D; d++)
                c->zcout[idx * D + d] = z[d];
        float dpart = 0.0f;
        for (size_t d = 0; d < D; d++)
            dpart += orc_phi_elu(c->Q[idx * D + d]) * z[d];
        c->denout[idx] = dpart;
        for (size_t e = 0; e < E; e++) {
            float num = 0.0f;
            for (size_t d = 0; d < D; d++)
                num += orc_phi_elu(c->Q[idx * D + d]) * state[e * D + d];
            c->Oout[idx * E + e] = num / (dpart + 1e-8f);
        }
    }
    free(z);
    free(state);
}

void orc_kattn_fwd(const float *Q, const float *K, const float *V,
                   float *O, float *den, float *z_cache,
                   size_t B, size_t S, size_t D, size_t E, int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.Oout = O; c.denout = den; c.zcout = z_cache;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, kattn_fwd_seq, &c);
}

/* ref_kernel_attn_bwd (kernel_test.cpp:128-193), literally. */
void orc_kattn_bwd_literal(const float *Q, const float *K, const float *V,
                           const float *O, const float *dO, const float *den,
                           float *dQ, float *dK, float *dV,
                           size_t B, size_t S, size_t D, size_t E)
{
    size_t nd = D + 1, ned = E * D + 1;
    float *z = (float *)malloc(sizeof(float) * nd);
    float *state = (float *)malloc(sizeof(float) * ned);
    float *zs = (float *)malloc(sizeof(float) * nd);
    float *Sst = (float *)malloc(sizeof(float) * ned);
    for (size_t b = 0; b < B; b++)
        for (size_t t = 0; t < S; t++) {
            size_t idx = b * S + t;
            memset(z, 0, sizeof(float) * D);
            memset(state, 0, sizeof(float) * E * D);
            for (size_t s = 0; s <= t; s++) {
                size_t j = b * S + s;
                for (size_t d = 0; d < D; d++) {
                    z[d] += orc_phi_elu(K[j * D + d]);
                    for (size_t e = 0; e < E; e++)
                        state[e * D + d] += orc_phi_elu(K[j * D + d]) * V[j * E + e];
                }
            }
            float inv_den = 1.0f / den[idx];
            float dden = 0.0f;
            for (size_t e = 0; e < E; e++)
                dden -= dO[idx * E + e] * O[idx * E + e] * inv_den;
            for (size_t d = 0; d < D; d++) {
                float dnum = z[d] * dden;
                for (size_t e = 0; e < E; e++)
                    dnum += state[e * D + d] * (dO[idx * E + e] * inv_den);
                dQ[idx * D + d] = dnum * orc_phi_elu_der(Q[idx * D + d]);
            }
            memset(zs, 0, sizeof(float) * D);
            memset(Sst, 0, sizeof(float) * E * D);
            for (size_t s = S; s-- > t;) {
                size_t j = b * S + s;
                float dd = 0.0f;
                for (size_t e = 0; e < E; e++)
                    dd -= dO[j * E + e] * O[j * E + e] / den[j];
                for (size_t d = 0; d < D; d++) {
                    zs[d] += orc_phi_elu(Q[j * D + d]) * dd;
                    for (size_t e = 0; e < E; e++)
                        Sst[e * D + d] += orc_phi_elu(Q[j * D + d]) * (dO[j * E + e] / den[j]);
                }
            }
            for (size_t e = 0; e < E; e++) {
                float acc = 0.0f;
                for (size_t d = 0; d < D; d++)
                    acc += Sst[e * D + d] * orc_phi_elu(K[idx * D + d]);
                dV[idx * E + e] = acc;
            }
            for (size_t d = 0; d < D; d++) {
                float acc = zs[d];
                for (size_t e = 0; e < E; e++)
                    acc += Sst[e * D + d] * V[idx * E + e];
                dK[idx * D + d] = acc * orc_phi_elu_der(K[idx * D + d]);
            }
        }
    free(z);
    free(state);
    free(zs);
    free(Sst);
}

/* step1 closed form, kernel_test.cpp:277-286 */
void orc_kattn_bwd_step1(const float *O, const float *dO, const float *den,
                         float *dnum, float *dden, size_t N, size_t E)
{
    for (size_t i = 0; i < N; i++) {
        dden[i] = 0.0f;
        for (size_t e = 0; e < E; e++) {
            dnum[i * E + e] = dO[i * E + e] / den[i];
            dden[i] -= dO[i * E + e] * O[i * E + e] / den[i];
        }
    }
}

/* kernel_attn_bwd_dQ (two_stage_cuda_kernels.cu:1253-1300), one sequence. */
static void kattn_dQ_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *state = (float *)calloc(E * D, sizeof(float));
    for (size_t t = 0; t < S; t++) {
        size_t idx = b * S + t;
        for (size_t e = 0; e < E; e++)
            for (size_t d = 0; d < D; d++)
                state[e * D + d] += orc_phi_elu(c->K[idx * D + d]) * c->V[idx * E + e];
        for (size_t d = 0; d < D; d++) {
            float acc = c->zc[idx * D + d] * c->dden[idx];
            for (size_t e = 0; e < E; e++)
                acc += state[e * D + d] * c->dnum[idx * E + e];
            c->dQ[idx * D + d] = acc * orc_phi_elu_der(c->Q[idx * D + d]);
        }
    }
    free(state);
}

void orc_kattn_bwd_dQ(const float *K, const float *V, const float *dnum,
                      const float *dden, const float *z_cache, const float *Q,
                      float *dQ, size_t B, size_t S, size_t D, size_t E, int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.K = K; c.V = V; c.dnum = dnum; c.dden = dden; c.zc = z_cache; c.Q = Q; c.dQ = dQ;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, kattn_dQ_seq, &c);
}

/* kernel_attn_bwd_dKdV (two_stage_cuda_kernels.cu:1596-1676), one sequence. */
static void kattn_dKdV_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *Sst = (float *)calloc(E * D, sizeof(float));
    float *zs = (float *)calloc(D, sizeof(float));
    for (size_t t = S; t-- > 0;) {
        size_t idx = b * S + t;
        for (size_t e = 0; e < E; e++)
            for (size_t d = 0; d < D; d++)
                Sst[e * D + d] += orc_phi_elu(c->Q[idx * D + d]) * c->dnum[idx * E + e];
        for (size_t d = 0; d < D; d++)
            zs[d] += orc_phi_elu(c->Q[idx * D + d]) * c->dden[idx];
        for (size_t e = 0; e < E; e++) {
            float acc = 0.0f;
            for (size_t d = 0; d < D; d++)
                acc += Sst[e * D + d] * orc_phi_elu(c->K[idx * D + d]);
            c->dV[idx * E + e] = acc;
        }
        for (size_t d = 0; d < D; d++) {
            float acc = zs[d];
            for (size_t e = 0; e < E; e++)
                acc += Sst[e * D + d] * c->V[idx * E + e];
            c->dK[idx * D + d] = acc * orc_phi_elu_der(c->K[idx * D + d]);
        }
    }
    free(Sst);
    free(zs);
}

void orc_kattn_bwd_dKdV(const float *Q, const float *K, const float *V,
                        const float *dnum, const float *dden,
                        float *dK, float *dV, size_t B, size_t S, size_t D, size_t E,
                        int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Q; c.K = K; c.V = V; c.dnum = dnum; c.dden = dden; c.dK = dK; c.dV = dV;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, kattn_dKdV_seq, &c);
}

/* ------------------------------------------------------------------ */
/* linear_cuda API (phi outside), src/LinearAttention/linear_cuda_kernels.cu */
/* ------------------------------------------------------------------ */
/* causal_linear_attn_fwd_kernel (:10-79), one sequence. */
static void lcu_fwd_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *state = (float *)calloc(D * E, sizeof(float));
    float *z = (float *)calloc(D, sizeof(float));
    for (size_t t = 0; t < S; t++) {
        size_t idx = b * S + t;
        for (size_t d = 0; d < D; d++)
            for (size_t e = 0; e < E; e++)
                state[d * E + e] += c->K[idx * D + d] * c->V[idx * E + e];
        for (size_t d = 0; d < D; d++)
            z[d] += c->K[idx * D + d];
        for (size_t d = 0; d < D; d++)
            c->zcout[idx * D + d] = z[d];
        float norm = 0.0f;
        for (size_t d = 0; d < D; d++)
            norm += c->Q[idx * D + d] * z[d];
        float total = norm + 1e-8f;
        c->denout[idx] = total;
        for (size_t e = 0; e < E; e++) {
            float num = 0.0f;
            for (size_t d = 0; d < D; d++)
                num += c->Q[idx * D + d] * state[d * E + e];
            c->Oout[idx * E + e] = num / total;
        }
    }
    if (c->Sbuf)
        memcpy(c->Sbuf + b * D * E, state, sizeof(float) * D * E);
    if (c->zbuf)
        memcpy(c->zbuf + b * D, z, sizeof(float) * D);
    free(state);
    free(z);
}

void orc_lcu_fwd(const float *Qp, const float *Kp, const float *V,
                 float *O, float *den_cache, float *z_cache, float *S_buf, float *z_buf,
                 size_t B, size_t S, size_t D, size_t E, int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Qp; c.K = Kp; c.V = V; c.Oout = O; c.denout = den_cache; c.zcout = z_cache;
    c.Sbuf = S_buf; c.zbuf = z_buf;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, lcu_fwd_seq, &c);
}

/* causal_linear_attn_bwd_step1_kernel (:101-134): multiplies by 1/den. */
void orc_lcu_bwd_step1(const float *O, const float *dO, const float *den_cache,
                       float *dnum, float *dden, size_t N, size_t E)
{
    for (size_t i = 0; i < N; i++) {
        float inv_den = 1.0f / den_cache[i];
        float sum = 0.0f;
        for (size_t e = 0; e < E; e++) {
            dnum[i * E + e] = dO[i * E + e] * inv_den;
            sum += dO[i * E + e] * O[i * E + e];
        }
        dden[i] = -sum * inv_den;
    }
}

/* causal_linear_attn_bwd_dQ_kernel (:152-197), one sequence. */
static void lcu_dQ_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *state = (float *)calloc(D * E, sizeof(float));
    for (size_t t = 0; t < S; t++) {
        size_t idx = b * S + t;
        for (size_t d = 0; d < D; d++)
            for (size_t e = 0; e < E; e++)
                state[d * E + e] += c->K[idx * D + d] * c->V[idx * E + e];
        float dd = c->dden[idx];
        for (size_t d = 0; d < D; d++) {
            float val = c->zc[idx * D + d] * dd;
            for (size_t e = 0; e < E; e++)
                val += state[d * E + e] * c->dnum[idx * E + e];
            c->dQ[idx * D + d] = val;
        }
    }
    free(state);
}

void orc_lcu_bwd_dQ(const float *Kp, const float *V, const float *dnum,
                    const float *dden, const float *z_cache, float *dQp,
                    size_t B, size_t S, size_t D, size_t E, int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.K = Kp; c.V = V; c.dnum = dnum; c.dden = dden; c.zc = z_cache; c.dQ = dQp;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, lcu_dQ_seq, &c);
}

/* causal_linear_attn_bwd_dKdV_kernel (:217-273), one sequence. */
static void lcu_dKdV_seq(void *vctx, size_t b)
{
    lin_ctx *c = (lin_ctx *)vctx;
    size_t S = c->S, D = c->D, E = c->E;
    float *Sst = (float *)calloc(D * E, sizeof(float));
    float *zs = (float *)calloc(D, sizeof(float));
    for (size_t t = S; t-- > 0;) {
        size_t idx = b * S + t;
        for (size_t d = 0; d < D; d++)
            for (size_t e = 0; e < E; e++)
                Sst[d * E + e] += c->Q[idx * D + d] * c->dnum[idx * E + e];
        for (size_t d = 0; d < D; d++)
            zs[d] += c->Q[idx * D + d] * c->dden[idx];
        for (size_t e = 0; e < E; e++) {
            float val = 0.0f;
            for (size_t d = 0; d < D; d++)
                val += Sst[d * E + e] * c->K[idx * D + d];
            c->dV[idx * E + e] = val;
        }
        for (size_t d = 0; d < D; d++) {
            float val = zs[d];
            for (size_t e = 0; e < E; e++)
                val += Sst[d * E + e] * c->V[idx * E + e];
            c->dK[idx * D + d] = val;
        }
    }
    free(Sst);
    free(zs);
}

void orc_lcu_bwd_dKdV(const float *Qp, const float *Kp, const float *V,
                      const float *dnum, const float *dden, float *dKp, float *dV,
                      size_t B, size_t S, size_t D, size_t E, int nthreads)
{
    lin_ctx c;
    memset(&c, 0, sizeof(c));
    c.Q = Qp; c.K = Kp; c.V = V; c.dnum = dnum; c.dden = dden; c.dK = dKp; c.dV = dV;
    c.S = S; c.D = D; c.E = E;
    orc_parallel_for(B, nthreads, lcu_dKdV_seq, &c);
}

/* phi_elu_fwd_kernel (:305-325): (expf(x) - 1) + 1 for x <= 0, kept literal. */
void orc_phi_elu_forward(const float *x, float *phi, size_t N, size_t D, size_t E)
{
    for (size_t i = 0; i < N; i++)
        for (size_t j = 0; j < D; j++) {
            if (j < E) {
                float xv = x[i * E + j];
                float elu = xv > 0.0f ? xv : expf(xv) - 1.0f;
                phi[i * D + j] = elu + 1.0f;
            } else {
                phi[i * D + j] = 0.0f;
            }
        }
}

/* phi_elu_bwd_kernel (:347-364) */
void orc_phi_elu_backward(const float *dphi, const float *x, float *dx,
                          size_t N, size_t D, size_t E)
{
    for (size_t i = 0; i < N; i++)
        for (size_t j = 0; j < E; j++) {
            float xv = x[i * E + j];
            float der = xv > 0.0f ? 1.0f : expf(xv);
            dx[i * E + j] = dphi[i * D + j] * der;
        }
}

/* ------------------------------------------------------------------ */
/* Hadamard+Exp feature map (benchmark-defined; no reference code)      */
/* ------------------------------------------------------------------ */
float orc_hadamard_entry(int i, int j)
{
    return (__builtin_popcount((unsigned)(i & j)) & 1) ? -1.0f : 1.0f;
}

void orc_phi_hexp_forward(const float *x, float *phi, size_t N, size_t D, size_t E)
{
    for (size_t n = 0; n < N; n++) {
        for (size_t blk = 0; blk + 64 <= E; blk += 64)
            for (int i = 0; i < 64; i++) {
                float y = 0.0f;
                for (int j = 0; j < 64; j++)
                    y += orc_hadamard_entry(i, j) * x[n * E + blk + (size_t)j];
                phi[n * D + blk + (size_t)i] = expf(y * 0.125f);
            }
        for (size_t j = E; j < D; j++)
            phi[n * D + j] = 0.0f;
    }
}

void orc_phi_hexp_backward(const float *dphi, const float *x, float *dx,
                           size_t N, size_t D, size_t E)
{
    float phi[64];
    for (size_t n = 0; n < N; n++)
        for (size_t blk = 0; blk + 64 <= E; blk += 64) {
            for (int i = 0; i < 64; i++) {
                float y = 0.0f;
                for (int j = 0; j < 64; j++)
                    y += orc_hadamard_entry(i, j) * x[n * E + blk + (size_t)j];
                phi[i] = expf(y * 0.125f);
            }
            for (int j = 0; j < 64; j++) {
                float acc = 0.0f;
                for (int i = 0; i < 64; i++)
                    acc += orc_hadamard_entry(j, i) * (dphi[n * D + blk + (size_t)i] * phi[i]);
                dx[n * E + blk + (size_t)j] = acc * 0.125f;
            }
        }
}

/* ---------------- rotary position embedding ----------------
 * kernel_test.cpp:451-459 (rope_one) and :460-471 (ref_rope): the same float
 * expressions (powf of a float exponent, the angle as a float product, cosf
 * / sinf of it), rows in order. */
void orc_rope(float *X, size_t B, size_t S, size_t D, size_t head_dim, float sign)
{
    const float base = 10000.0f;
    const size_t rows = B * S;
    for (size_t r = 0; r < rows; r++) {
        const size_t p = r % S;
        for (size_t h = 0; h < D / head_dim; h++)
            for (size_t i = 0; i < head_dim / 2; i++) {
                const float w = powf(base, -2.0f * (float)i / (float)head_dim);
                const float ang = sign * (float)p * w;
                const float c = cosf(ang), s = sinf(ang);
                float *x = X + r * D + h * head_dim + 2 * i;
                const float a = x[0], b = x[1];
                x[0] = a * c - b * s;
                x[1] = a * s + b * c;
            }
    }
}

/* two_stage_cuda_kernels.cu:1888-1895 */
void orc_gelu_exact(const float *A, float *C, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        const float x = A[i];
        C[i] = 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
    }
}

/* two_stage_cuda_kernels.cu:1906-1914 */
void orc_gelu_exact_deriv(const float *A, float *C, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        const float x = A[i];
        const float a = x * 0.7071067811865476f;
        C[i] = 0.5f * (1.0f + erff(a)) + x * expf(-0.5f * x * x) * 0.3989422804014327f;
    }
}

/* ------------------------------------------------------------------ */
/* expander FFN (two_stage_gpt.hpp:86-99, :177-195)                    */
/* ------------------------------------------------------------------ */
/* C[i][j] (= or +=) sum_k A(i,k) B(k,j), double accumulation; ak: A(i,k) at
 * A[i*lda + k] else A[k*lda + i]; bk: B(k,j) at B[j*ldb + k] else B[k*ldb + j]. */
typedef struct {
    const float *A, *B;
    size_t lda, ldb, ldc, N, K;
    int ak, bk, accum;
    float *C;
} orc_gemm_ctx;

static void orc_gemm_row(void *vc, size_t i)
{
    const orc_gemm_ctx *c = (const orc_gemm_ctx *)vc;
    double *acc = (double *)calloc(c->N, sizeof(double));
    for (size_t k = 0; k < c->K; k++) {
        const double a = c->ak ? c->A[i * c->lda + k] : c->A[k * c->lda + i];
        if (c->bk) {
            for (size_t j = 0; j < c->N; j++)
                acc[j] += a * (double)c->B[j * c->ldb + k];
        } else {
            const float *b = c->B + k * c->ldb;
            for (size_t j = 0; j < c->N; j++)
                acc[j] += a * (double)b[j];
        }
    }
    float *out = c->C + i * c->ldc;
    for (size_t j = 0; j < c->N; j++)
        out[j] = c->accum ? (float)((double)out[j] + acc[j]) : (float)acc[j];
    free(acc);
}

static void orc_gemm(const float *A, size_t lda, int ak, const float *B, size_t ldb, int bk,
                     size_t M, size_t N, size_t K, float *C, size_t ldc, int accum, int nthreads)
{
    orc_gemm_ctx c = {A, B, lda, ldb, ldc, N, K, ak, bk, accum, C};
    orc_parallel_for(M, nthreads, orc_gemm_row, &c);
}

/* q_ffn_fc.forward (X W1^T, gpt_gpt.hpp:86-93) -> gelu_exact -> q_ffn_proj.forward */
void orc_ffn_fwd(const float *X, const float *W1, const float *W2, float *pre, float *act,
                 float *Y, size_t M, size_t E, size_t F, int nthreads)
{
    float *p = pre ? pre : (float *)malloc(sizeof(float) * M * F);
    orc_gemm(X, E, 1, W1, E, 1, M, F, E, p, F, 0, nthreads);
    orc_gelu_exact(p, act, M * F);
    orc_gemm(act, F, 1, W2, F, 1, M, E, F, Y, E, 0, nthreads);
    if (!pre)
        free(p);
}

/* q_ffn_proj.backward (dY W2; W2.grad += dY^T act, gpt_gpt.hpp:98-105) ->
 * gelu_exact_deriv(G) -> multiply -> q_ffn_fc.backward (dact W1; W1.grad +=
 * dact^T X), two_stage_gpt.hpp:177-183 */
void orc_ffn_bwd(const float *X, const float *W1, const float *W2, const float *act,
                 const float *G, const float *dY, float *dX, float *dW1, float *dW2, size_t M,
                 size_t E, size_t F, int nthreads)
{
    float *dact = (float *)malloc(sizeof(float) * M * F);
    float *gd = (float *)malloc(sizeof(float) * M * F);
    orc_gemm(dY, E, 1, W2, F, 0, M, F, E, dact, F, 0, nthreads);
    orc_gemm(dY, E, 0, act, F, 0, E, F, M, dW2, F, 1, nthreads);
    orc_gelu_exact_deriv(G, gd, M * F);
    for (size_t i = 0; i < M * F; i++)
        dact[i] *= gd[i];
    orc_gemm(dact, F, 1, W1, E, 0, M, E, F, dX, E, 0, nthreads);
    orc_gemm(dact, F, 0, X, E, 0, F, E, M, dW1, E, 1, nthreads);
    free(gd);
    free(dact);
}
