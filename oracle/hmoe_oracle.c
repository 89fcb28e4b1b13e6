/* hmoe_oracle.c - CPU restatement of chronarion/hecate's routed int4 MoE hot path (see hmoe_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline. Nothing in hecate_amd/ links or calls it.
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). Parity status of each function is listed in the
 * header comment of tests/test_oracle.py, which pins it (golden vectors, closed forms, invariants, brute force).
 */
#include "hmoe_oracle.h"
#include "../include/hmoe_rng.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------------------------
 * synthetic data: thin loops over include/hmoe_rng.h
 * ---------------------------------------------------------------------------------------------------------------- */
uint64_t orc_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t expert) { return hmoe_key(seed, layer, kind, expert); }

void orc_gen_normal_f32(uint64_t key, int64_t n, float mean, float sigma, float* out)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = mean + sigma * hmoe_normal(key, (uint64_t) i);
}

void orc_gen_normal_bf16(uint64_t key, int64_t n, float sigma, uint16_t* out)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = hmoe_f2bf(sigma * hmoe_normal(key, (uint64_t) i));
}

/* codes [N][K/2]: byte (n, k/2) = code(n, k) | code(n, k + 1) << 4 (cpuband.cpp:3-4 row-major, low nibble first) */
void orc_gen_codes(uint64_t key, int N, int K, uint8_t* out)
{
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; k += 16)
        {
            const uint64_t h = hmoe_bits(key, ((uint64_t) n * (uint64_t) K + (uint64_t) k) >> 4);
            for (int j = 0; j < 8; ++j) out[(size_t) n * (K / 2) + k / 2 + j] = (uint8_t) (h >> (8 * j));
        }
}

/* scales [N][K/128] bf16 = |sigma * z| with z the normal of element n * (K / 128) + g */
void orc_gen_scales(uint64_t key, int N, int K, float sigma, uint16_t* out)
{
    const int G = K / 128;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t) N * G; ++i) out[i] = hmoe_f2bf(fabsf(sigma * hmoe_normal(key, (uint64_t) i)));
}

void orc_f32_to_bf16(const float* in, int64_t n, uint16_t* out) { for (int64_t i = 0; i < n; ++i) out[i] = hmoe_f2bf(in[i]); }
void orc_f32_to_f16(const float* in, int64_t n, uint16_t* out) { for (int64_t i = 0; i < n; ++i) out[i] = hmoe_f2h(in[i]); }
void orc_f16_to_f32(const uint16_t* in, int64_t n, float* out) { for (int64_t i = 0; i < n; ++i) out[i] = hmoe_h2f(in[i]); }
float orc_expf(float x) { return hmoe_expf(x); }

/* ------------------------------------------------------------------------------------------------------------------
 * router
 * ---------------------------------------------------------------------------------------------------------------- */
/* logits[r][e] = x[r] . w[e] in fp32 with one fixed order: 8 segments of K / 8; in each, chains of 32 fmaf
 * (k ascending, from 0) whose totals are added in order from 0; the segment totals added in order from 0
 * (K % 256 == 0). The reference accumulates the same products in fp32 with atomics (exl3_router.py:42-71: fp32
 * accumulation of fp16 products, order set by the atomics); here W_g is fp32. */
void orc_router_logits_f32(const float* x, const float* w, int R, int K, int E, float* logits)
{
    #pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < R; ++r)
        for (int e = 0; e < E; ++e)
        {
            const float* xr = x + (size_t) r * K;
            const float* we = w + (size_t) e * K;
            const int SEG = K / ORC_ROUTER_SEGMENTS;
            float t = 0.0f;
            for (int s0 = 0; s0 < K; s0 += SEG)
            {
                float seg = 0.0f;
                for (int c = s0; c < s0 + SEG; c += ORC_ROUTER_CHUNK)
                {
                    float acc = 0.0f;
                    for (int k = c; k < c + ORC_ROUTER_CHUNK; ++k) acc = fmaf(xr[k], we[k], acc);
                    seg = seg + acc;
                }
                t = t + seg;
            }
            logits[(size_t) r * E + e] = t;
        }
}

/* x bf16: widened exactly, then the fp32 form */
void orc_router_logits(const uint16_t* x, const float* w, int R, int K, int E, float* logits)
{
    float* xf = (float*) malloc((size_t) R * K * sizeof(float));
    for (size_t i = 0; i < (size_t) R * K; ++i) xf[i] = hmoe_bf2f(x[i]);
    orc_router_logits_f32(xf, w, R, K, E, logits);
    free(xf);
}

/* exl3_router.py:84-128: a = sigmoid(l); key = okey(a + bias); topk rounds of (max key, lowest index on ties), so
 * sel[r][k] is in descending key order; sum of the selected unbiased a in selection order from 0;
 * rw = f16_rn(a * scale / (sum + 1e-20)) (nr4_kernel.cuh:362 divides with round-to-nearest) */
void orc_router_select(const float* logits, const float* bias, int R, int E, int topk, float scale,
                       int64_t* sel, uint16_t* rw)
{
    for (int r = 0; r < R; ++r)
    {
        float* act = (float*) malloc(sizeof(float) * (size_t) E);
        uint32_t* key = (uint32_t*) malloc(sizeof(uint32_t) * (size_t) E);
        for (int e = 0; e < E; ++e)
        {
            act[e] = hmoe_sigmoid(logits[(size_t) r * E + e]);
            key[e] = hmoe_okey(act[e] + (bias ? bias[e] : 0.0f));
        }
        float wsel[64]; int isel[64]; float sum = 0.0f;
        for (int k = 0; k < topk; ++k)
        {
            int bi = -1; uint32_t bk = 0u;
            for (int e = 0; e < E; ++e)
                if (key[e] > bk || (bi < 0 && key[e] == bk)) { bk = key[e]; bi = e; }
            /* ties: the strict > above keeps the lowest index */
            wsel[k] = act[bi]; isel[k] = bi; sum = sum + act[bi];
            key[bi] = 0u;
        }
        for (int k = 0; k < topk; ++k)
        {
            sel[(size_t) r * topk + k] = isel[k];
            rw[(size_t) r * topk + k] = hmoe_f2h((wsel[k] * scale) / (sum + 1e-20f));
        }
        free(act); free(key);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * dispatch
 * ---------------------------------------------------------------------------------------------------------------- */
/* tier_split.py:404-412: fs = sel.flat; order = argsort(fs, stable); counts = bincount; seg = order[:n4];
 * tok = seg // topk, eid = fs[seg], wt = rw.flat[seg]. Generalised to the window [lo, lo + n) (eid relative to lo,
 * the reference has lo = 0 here); inv[flat] = position of the pick or -1 outside the window. Returns npos. */
int orc_dispatch(const int64_t* sel, const uint16_t* rw, int T, int topk, int lo, int n, int64_t* counts,
                 int32_t* tok, int32_t* eid, float* wt, int32_t* inv)
{
    const int F = T * topk;
    int64_t* off = (int64_t*) calloc((size_t) n + 1, sizeof(int64_t));
    for (int e = 0; e < n; ++e) counts[e] = 0;
    for (int i = 0; i < F; ++i) { const int64_t e = sel[i] - lo; if (e >= 0 && e < n) ++counts[e]; }
    for (int e = 0; e < n; ++e) off[e + 1] = off[e] + counts[e];
    for (int i = 0; i < F; ++i)                          /* flat index ascending within each expert: stable */
    {
        const int64_t e = sel[i] - lo;
        if (e < 0 || e >= n) { if (inv) inv[i] = -1; continue; }
        const int64_t p = off[e]++;
        tok[p] = i / topk; eid[p] = (int32_t) e; wt[p] = hmoe_h2f(rw[i]);
        if (inv) inv[i] = (int32_t) p;
    }
    int npos = 0; for (int e = 0; e < n; ++e) npos += (int) counts[e];
    free(off);
    return npos;
}

/* rtx_split.py:241-254 with one group holding every pick: per expert ceil(c / bm) row blocks; balance gives the
 * first c % nb blocks base + 1 rows (base = c // nb), else blocks of bm and a remainder. Row {expert, first pick,
 * picks, 0}. Returns the number of blocks (or -1 if more than cap). */
int orc_pick_groups(const int64_t* counts, int n, int bm, int balance, int32_t* rbt, int cap)
{
    int nrb = 0; int64_t base_pos = 0;
    for (int e = 0; e < n; ++e)
    {
        const int64_t c = counts[e];
        const int64_t nb = (c + bm - 1) / bm;
        for (int64_t k = 0; k < nb; ++k)
        {
            int64_t rows, start;
            if (balance) { const int64_t b = c / nb, x = c % nb; rows = b + (k < x ? 1 : 0); start = k * b + (k < x ? k : x); }
            else { rows = (c - bm * k) < bm ? (c - bm * k) : bm; start = bm * k; }
            if (nrb >= cap) return -1;
            rbt[4 * nrb + 0] = e; rbt[4 * nrb + 1] = (int32_t) (base_pos + start);
            rbt[4 * nrb + 2] = (int32_t) rows; rbt[4 * nrb + 3] = 0;
            ++nrb;
        }
        base_pos += c;
    }
    return nrb;
}

/* ------------------------------------------------------------------------------------------------------------------
 * expert layer
 * ---------------------------------------------------------------------------------------------------------------- */
/* cpuband.cpp:163-177: picks in first appearance over rows then top-k (ids in [lo, lo + n_hot)), wgt[p][r] = sum of
 * the f16 routing weights as fp32 */
int orc_picks(const int64_t* sel, const uint16_t* rw, int R, int topk, int lo, int n_hot, int32_t* pick, float* wgt)
{
    int P = 0;
    for (int i = 0; i < R * topk; ++i)
    {
        const int64_t e = sel[i] - lo;
        if (e < 0 || e >= n_hot) continue;
        int j = 0; while (j < P && pick[j] != (int32_t) e) ++j;
        if (j == P) { pick[P] = (int32_t) e; for (int r = 0; r < R; ++r) wgt[(size_t) P * R + r] = 0.0f; ++P; }
        wgt[(size_t) j * R + i / topk] += hmoe_h2f(rw[i]);
    }
    return P;
}

void orc_dequant(const uint8_t* codes, const uint16_t* scales, int N, int K, float* out)
{
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k)
        {
            const uint8_t b = codes[(size_t) n * (K / 2) + k / 2];
            const int q = (int) ((k & 1) ? (b >> 4) : (b & 15)) - 8;
            out[(size_t) n * K + k] = (float) q * hmoe_bf2f(scales[(size_t) n * (K / 128) + k / 128]);
        }
}

/* exact mode: y[r][n] = sum_k w[n][k] x[r][k] in fp64 over int4 g128 weights for the rows in rows[0..nr) */
static void gemv_i4_exact(const uint8_t* q, const uint16_t* s, int N, int K, const double* x, int nr, size_t xstride,
                          double* y, size_t ystride, int threads)
{
    #pragma omp parallel for schedule(static) num_threads(threads)
    for (int n = 0; n < N; ++n)
    {
        double acc[16];
        for (int r = 0; r < nr; ++r) acc[r] = 0.0;
        const uint8_t* qr = q + (size_t) n * (K / 2);
        for (int g = 0; g < K / 128; ++g)
        {
            const double sc = (double) hmoe_bf2f(s[(size_t) n * (K / 128) + g]);
            for (int k = g * 128; k < g * 128 + 128; k += 2)
            {
                const uint8_t b = qr[k / 2];
                const double w0 = (double) ((int) (b & 15) - 8) * sc, w1 = (double) ((int) (b >> 4) - 8) * sc;
                for (int r = 0; r < nr; ++r) acc[r] += w0 * x[r * xstride + k] + w1 * x[r * xstride + k + 1];
            }
        }
        for (int r = 0; r < nr; ++r) y[r * ystride + n] = acc[r];
    }
}

/* exact mode dense bf16 GEMV (shared expert) */
static void gemv_bf16_exact(const uint16_t* w, int N, int K, const double* x, int nr, size_t xstride, double* y,
                            size_t ystride, int threads)
{
    #pragma omp parallel for schedule(static) num_threads(threads)
    for (int n = 0; n < N; ++n)
    {
        double acc[16];
        for (int r = 0; r < nr; ++r) acc[r] = 0.0;
        const uint16_t* wr = w + (size_t) n * K;
        for (int k = 0; k < K; ++k)
        {
            const double wv = (double) hmoe_bf2f(wr[k]);
            for (int r = 0; r < nr; ++r) acc[r] += wv * x[r * xstride + k];
        }
        for (int r = 0; r < nr; ++r) y[r * ystride + n] = acc[r];
    }
}

/* cpuband.cpp:106-111: q8_0 group of 32: s = absmax / 127 (1 if 0), q = lrintf(v / s) */
static void quant_group(const float* v, int8_t* q, float* sc)
{
    float m = 0.0f; for (int k = 0; k < 32; ++k) m = fmaxf(m, fabsf(v[k]));
    const float s = m > 0 ? m / 127.0f : 1.0f; *sc = s; const float inv = 1.0f / s;
    for (int k = 0; k < 32; ++k) q[k] = (int8_t) lrintf(v[k] * inv);
}

/* cpuband.cpp:80-104 gemv_rows, with group-128 scales: per 128-group four fp32 lanes accumulate float(dot) * xg over
 * its four 32-blocks (lane i holds the products of k + 4i..4i+3 and k + 16 + 4i..4i+3, as two vdotq_s32 on the zipped
 * nibbles), the lanes fold as (a0 + a1) + (a2 + a3) (vaddvq_f32), and y = fmaf(s[n][g], fold, y) over groups */
static void gemv_i4_q8(const uint8_t* q, const uint16_t* s, int N, int K, const int8_t* xq, const float* xg, int nr,
                       float* y, size_t ystride, int threads)
{
    #pragma omp parallel for schedule(static) num_threads(threads)
    for (int n = 0; n < N; ++n)
    {
        const uint8_t* qr = q + (size_t) n * (K / 2);
        float yr[16];
        for (int r = 0; r < nr; ++r) yr[r] = 0.0f;
        for (int g = 0; g < K / 128; ++g)
        {
            float acc[16][4];
            for (int r = 0; r < nr; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.0f;
            for (int b = 0; b < 4; ++b)
            {
                const int k = g * 128 + b * 32;
                int8_t z[32];
                for (int j = 0; j < 16; ++j) { const uint8_t v = qr[k / 2 + j]; z[2 * j] = (int8_t) ((v & 15) - 8); z[2 * j + 1] = (int8_t) ((v >> 4) - 8); }
                for (int r = 0; r < nr; ++r)
                {
                    const int8_t* xr = xq + (size_t) r * K + k;
                    for (int i = 0; i < 4; ++i)
                    {
                        int32_t d = 0;
                        for (int j = 0; j < 4; ++j) d += (int32_t) z[4 * i + j] * (int32_t) xr[4 * i + j];
                        for (int j = 0; j < 4; ++j) d += (int32_t) z[16 + 4 * i + j] * (int32_t) xr[16 + 4 * i + j];
                        acc[r][i] = fmaf((float) d, xg[(size_t) r * (K / 32) + k / 32], acc[r][i]);
                    }
                }
            }
            const float sc = hmoe_bf2f(s[(size_t) n * (K / 128) + g]);
            for (int r = 0; r < nr; ++r) yr[r] = fmaf(sc, (acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3]), yr[r]);
        }
        for (int r = 0; r < nr; ++r) y[r * ystride + n] = yr[r];
    }
}

/* the q8_0 primitives on their own, for the oracle's tests: every row of x [nr][K] quantised per 32 (quant_group),
 * then y[r][n] = gemv_i4_q8 over packed codes q [N][K/2] (low nibble = even k) and bf16 group scales s [N][K/128];
 * xq / xg receive the quantised rows and their group scales */
int orc_q8_gemv(const uint8_t* q, const uint16_t* s, int N, int K, const float* x, int nr, int8_t* xq, float* xg,
                float* y)
{
    if (nr < 1 || nr > 16 || K % 128 != 0) return -1;
    for (int r = 0; r < nr; ++r)
        for (int g = 0; g < K / 32; ++g)
            quant_group(x + (size_t) r * K + g * 32, xq + (size_t) r * K + g * 32, xg + (size_t) r * (K / 32) + g);
    gemv_i4_q8(q, s, N, K, xq, xg, nr, y, N, 1);
    return 0;
}

/* fp32 dense GEMV of the shared expert in the q8 mode (the adaptation named for the CPU baseline) */
static void gemv_bf16_f32(const uint16_t* w, int N, int K, const float* x, int nr, size_t xstride, float* y,
                          size_t ystride, int threads)
{
    #pragma omp parallel for schedule(static) num_threads(threads)
    for (int n = 0; n < N; ++n)
    {
        float acc[16];
        for (int r = 0; r < nr; ++r) acc[r] = 0.0f;
        const uint16_t* wr = w + (size_t) n * K;
        for (int k = 0; k < K; ++k)
        {
            const float wv = hmoe_bf2f(wr[k]);
            for (int r = 0; r < nr; ++r) acc[r] = fmaf(wv, x[r * xstride + k], acc[r]);
        }
        for (int r = 0; r < nr; ++r) y[r * ystride + n] = acc[r];
    }
}

static double silu_d(double g) { return g / (1.0 + exp(-g)); }

int orc_moe(int mode, int R, int H, int I, const uint16_t* x, const int64_t* sel, const uint16_t* rw, int topk,
            int lo, int n_hot, const uint64_t* gq, const uint64_t* gs, const uint64_t* uq, const uint64_t* us,
            const uint64_t* dq, const uint64_t* ds, const uint16_t* sh_g, const uint16_t* sh_u, const uint16_t* sh_d,
            int accumulate, float* out, int threads)
{
    if (R < 1 || R > 16 || H % 128 || I % 128) return -1;
    if (threads < 1) threads = 1;
    int32_t* pick = (int32_t*) malloc(sizeof(int32_t) * (size_t) (R * topk));
    float* wgt = (float*) malloc(sizeof(float) * (size_t) (R * topk) * (size_t) R);
    const int P = orc_picks(sel, rw, R, topk, lo, n_hot, pick, wgt);
    int rc = 0;
    if (mode == 0)
    {
        double* xd = (double*) malloc(sizeof(double) * (size_t) R * H);
        double* g = (double*) malloc(sizeof(double) * (size_t) R * I);
        double* u = (double*) malloc(sizeof(double) * (size_t) R * I);
        double* a = (double*) malloc(sizeof(double) * (size_t) R * I);
        double* d = (double*) malloc(sizeof(double) * (size_t) R * H);
        double* yr = (double*) calloc((size_t) R * H, sizeof(double));
        double* xs = (double*) malloc(sizeof(double) * (size_t) R * H);
        for (size_t i = 0; i < (size_t) R * H; ++i) xd[i] = (double) hmoe_bf2f(x[i]);
        for (int p = 0; p < P; ++p)
        {
            const int e = pick[p];
            int rows[16], nr = 0;
            for (int r = 0; r < R; ++r) if (wgt[(size_t) p * R + r] != 0.0f) rows[nr++] = r;
            for (int j = 0; j < nr; ++j) memcpy(xs + (size_t) j * H, xd + (size_t) rows[j] * H, sizeof(double) * H);
            gemv_i4_exact((const uint8_t*) gq[e], (const uint16_t*) gs[e], I, H, xs, nr, H, g, I, threads);
            gemv_i4_exact((const uint8_t*) uq[e], (const uint16_t*) us[e], I, H, xs, nr, H, u, I, threads);
            for (int j = 0; j < nr; ++j)
            {
                const double w = (double) wgt[(size_t) p * R + rows[j]];
                for (int i = 0; i < I; ++i) a[(size_t) j * I + i] = silu_d(g[(size_t) j * I + i]) * u[(size_t) j * I + i] * w;
            }
            gemv_i4_exact((const uint8_t*) dq[e], (const uint16_t*) ds[e], H, I, a, nr, I, d, H, threads);
            for (int j = 0; j < nr; ++j)
                for (int n = 0; n < H; ++n) yr[(size_t) rows[j] * H + n] += d[(size_t) j * H + n];
        }
        if (sh_g && sh_u && sh_d)
        {
            gemv_bf16_exact(sh_g, I, H, xd, R, H, g, I, threads);
            gemv_bf16_exact(sh_u, I, H, xd, R, H, u, I, threads);
            for (size_t i = 0; i < (size_t) R * I; ++i) a[i] = silu_d(g[i]) * u[i];
            gemv_bf16_exact(sh_d, H, I, a, R, I, d, H, threads);
            for (size_t i = 0; i < (size_t) R * H; ++i) yr[i] += d[i];
        }
        for (size_t i = 0; i < (size_t) R * H; ++i) out[i] = (float) ((accumulate ? (double) out[i] : 0.0) + yr[i]);
        free(xd); free(g); free(u); free(a); free(d); free(yr); free(xs);
    }
    else if (mode == 1)
    {
        /* cpuband.cpp:147-148 q8_0 of every row of x; :188-218 per pick gather, gate/up, act -> q8_0, down summed over
         * picks in pick order into tmp[r] from 0 */
        int8_t* xq = (int8_t*) malloc((size_t) R * H);
        float* xg = (float*) malloc(sizeof(float) * (size_t) R * H / 32);
        for (int gi = 0; gi < R * H / 32; ++gi)
        {
            float v[32];
            for (int k = 0; k < 32; ++k) v[k] = hmoe_bf2f(x[(size_t) gi * 32 + k]);
            quant_group(v, xq + (size_t) gi * 32, xg + gi);
        }
        int8_t* xqp = (int8_t*) malloc((size_t) R * H);
        float* xgp = (float*) malloc(sizeof(float) * (size_t) R * H / 32);
        float* gy = (float*) malloc(sizeof(float) * (size_t) R * I);
        float* uy = (float*) malloc(sizeof(float) * (size_t) R * I);
        int8_t* aq = (int8_t*) malloc((size_t) P * R * I + 1);
        float* ag = (float*) malloc(sizeof(float) * ((size_t) P * R * I / 32 + 1));
        int* nrs = (int*) malloc(sizeof(int) * (size_t) (P + 1));
        int* rowsl = (int*) malloc(sizeof(int) * (size_t) (P + 1) * 16);
        for (int p = 0; p < P; ++p)
        {
            const int e = pick[p];
            int nr = 0;
            for (int r = 0; r < R; ++r) if (wgt[(size_t) p * R + r] != 0.0f) rowsl[p * 16 + nr++] = r;
            nrs[p] = nr;
            for (int j = 0; j < nr; ++j)
            {
                const int r = rowsl[p * 16 + j];
                memcpy(xqp + (size_t) j * H, xq + (size_t) r * H, (size_t) H);
                memcpy(xgp + (size_t) j * (H / 32), xg + (size_t) r * (H / 32), sizeof(float) * (H / 32));
            }
            gemv_i4_q8((const uint8_t*) gq[e], (const uint16_t*) gs[e], I, H, xqp, xgp, nr, gy, I, threads);
            gemv_i4_q8((const uint8_t*) uq[e], (const uint16_t*) us[e], I, H, xqp, xgp, nr, uy, I, threads);
            for (int j = 0; j < nr; ++j)
            {
                const float wt = wgt[(size_t) p * R + rowsl[p * 16 + j]];
                for (int k0 = 0; k0 < I; k0 += 32)
                {
                    float v[32];
                    for (int k = 0; k < 32; ++k)
                    {
                        const float gg = gy[(size_t) j * I + k0 + k];
                        v[k] = gg / (1.0f + expf(-gg)) * uy[(size_t) j * I + k0 + k] * wt;
                    }
                    quant_group(v, aq + ((size_t) p * R + j) * I + k0, ag + (((size_t) p * R + j) * I + k0) / 32);
                }
            }
        }
        /* down: per output n, picks in order, rows of each pick */
        float* y1 = (float*) malloc(sizeof(float) * 16 * (size_t) H);
        float* tmp = (float*) calloc((size_t) R * H, sizeof(float));
        for (int p = 0; p < P; ++p)
        {
            const int e = pick[p];
            gemv_i4_q8((const uint8_t*) dq[e], (const uint16_t*) ds[e], H, I, aq + (size_t) p * R * I,
                       ag + (size_t) p * R * I / 32, nrs[p], y1, H, threads);
            for (int j = 0; j < nrs[p]; ++j)
            {
                const int r = rowsl[p * 16 + j];
                for (int n = 0; n < H; ++n) tmp[(size_t) r * H + n] += y1[(size_t) j * H + n];
            }
        }
        if (sh_g && sh_u && sh_d)
        {
            float* xf = (float*) malloc(sizeof(float) * (size_t) R * H);
            float* af = (float*) malloc(sizeof(float) * (size_t) R * I);
            float* dd = (float*) malloc(sizeof(float) * (size_t) R * H);
            for (size_t i = 0; i < (size_t) R * H; ++i) xf[i] = hmoe_bf2f(x[i]);
            gemv_bf16_f32(sh_g, I, H, xf, R, H, gy, I, threads);
            gemv_bf16_f32(sh_u, I, H, xf, R, H, uy, I, threads);
            for (size_t i = 0; i < (size_t) R * I; ++i) af[i] = gy[i] / (1.0f + expf(-gy[i])) * uy[i];
            gemv_bf16_f32(sh_d, H, I, af, R, I, dd, H, threads);
            for (size_t i = 0; i < (size_t) R * H; ++i) tmp[i] += dd[i];
            free(xf); free(af); free(dd);
        }
        for (size_t i = 0; i < (size_t) R * H; ++i) out[i] = (accumulate ? out[i] : 0.0f) + tmp[i];
        free(xq); free(xg); free(xqp); free(xgp); free(gy); free(uy); free(aq); free(ag); free(nrs); free(rowsl);
        free(y1); free(tmp);
    }
    else rc = -2;
    free(pick); free(wgt);
    return rc;
}

/* ------------------------------------------------------------------------------------------------------------------
 * RMSNorm in the reduction order of the reference's rms_norm_kernel, which its fused kernels reproduce bit for bit
 * (combine_norm, runtime/tier/cn.cu:1-6,21-31,80-103; norm_route, runtime/core/nr4_kernel.cuh:4-9,176-243):
 * a row of H values is H / 4 float4 columns; thread t of 1024 owns columns t, t + 1024, ... (< H / 4) and runs one
 * fmaf chain from 0 over its columns' elements in order (cn.cu:80-87); reduce_1024 (cn.cu:21-31): within each group
 * of 32 threads an xor butterfly (offsets 16, 8, 4, 2, 1; every lane ends with the group's sum), then the 32 group
 * sums, in group order, by the same butterfly. rmf = 1 / sqrt(sum / H + eps) * cscale (cn.cu:89: rsqrtf under
 * fast math there, the correctly rounded 1 / sqrt here), xn = (v * (w + cbias)) * rmf (cbias added only when nonzero,
 * cn.cu:95-96), rounded to bf16 (xn_bf16 = 1) or f16 (0). v: the residual after the add, [R][H].
 * ---------------------------------------------------------------------------------------------------------------- */
static float butterfly32(const float* in)
{
    float l[32], n[32];
    memcpy(l, in, sizeof(l));
    for (int o = 16; o > 0; o >>= 1)
    {
        for (int i = 0; i < 32; ++i) n[i] = l[i] + l[i ^ o];
        memcpy(l, n, sizeof(l));
    }
    return l[0];
}

float orc_rms_sum(const float* v, int H)
{
    const int C = H / 4;
    float chain[1024], gs[32];
    for (int t = 0; t < 1024; ++t)
    {
        float p = 0.0f;
        for (int c = t; c < C; c += 1024)
            for (int e = 0; e < 4; ++e) p = fmaf(v[4 * c + e], v[4 * c + e], p);
        chain[t] = p;
    }
    for (int g = 0; g < 32; ++g) gs[g] = butterfly32(chain + 32 * g);
    return butterfly32(gs);
}

void orc_rmsnorm_cn(const float* v, const float* w, int R, int H, float eps, float cbias, float cscale, int xn_bf16,
                    uint16_t* xn)
{
    for (int row = 0; row < R; ++row)
    {
        const float* vr = v + (size_t) row * H;
        const float rmf = (1.0f / sqrtf(orc_rms_sum(vr, H) / (float) H + eps)) * cscale;
        for (int k = 0; k < H; ++k)
        {
            const float wk = cbias != 0.0f ? w[k] + cbias : w[k];
            const float o = (vr[k] * wk) * rmf;
            xn[(size_t) row * H + k] = xn_bf16 ? hmoe_f2bf(o) : hmoe_f2h(o);
        }
    }
}

/* residual + RMSNorm between layers (cn.cu:80-103 with f = y = 0 and a the layer output): r = a + r (a may be NULL),
 * then orc_rmsnorm_cn with cbias 0, cscale 1, bf16 out */
void orc_residual_rmsnorm(float* r, const float* a, const float* w, int R, int H, float eps, uint16_t* xn_bf16)
{
    if (a)
        for (size_t i = 0; i < (size_t) R * H; ++i) r[i] = a[i] + r[i];
    orc_rmsnorm_cn(r, w, R, H, eps, 0.0f, 1.0f, 1, xn_bf16);
}
