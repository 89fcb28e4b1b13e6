// prefill.hip - prefill MoE on gfx950: device-side dispatch plan (runtime/tier/tier_split.py:400-420 +
// runtime/tier/rtx_split.py:236-255, no host sync) and the grouped expert GEMMs (runtime/tier/moe4/moe4p.cu:217-245).
//
// Dispatch: picks sorted by (expert, flat index) by a counting sort with per-block histograms and in-block ranks, so
// the order equals a stable argsort of the selection; row blocks {expert, first pick, picks, 0} of at most bm picks.
// GEMMs: workgroup = (row block of <= 64 picks of one expert, 128 output columns). The picks' input rows are gathered,
// converted to f16 and staged per 128-k group in LDS (double buffered); each of the 4 waves owns 32 output rows of
// gate and of up (2 strips of 16 each) and decodes its I4G128 tiles straight from HBM into registers (one 16-byte
// load per lane per tile, exact f16 codes times the f16 group scale), then runs the 16x16x32 MFMA against every
// 16-pick tile of the block. gu fuses act = silu(g) * u * w (f16), down writes d = W_d act (fp32), fin adds each
// token's picks into out in top-k order (or with atomics, as p4_fin_kernel, when no inverse map is given).
#include "hmoe_dev.h"

namespace hmoe {

constexpr int PB = 64;                      // picks per row block
constexpr int PN = 128;                     // output columns per workgroup
constexpr int PT = 256;                     // threads
constexpr int XSTR = 128 + 8;               // LDS row stride (f16) of the staged inputs
constexpr int DBLK = 256;                   // picks per dispatch block

// ---------------------------------------------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(DBLK) disp_count_kernel(const int64_t* __restrict__ sel, int F, int lo, int n,
                                                          int* __restrict__ hist, int* __restrict__ rank)
{
    __shared__ int es[DBLK];
    __shared__ int h[256];
    const int t = threadIdx.x, i = blockIdx.x * DBLK + t;
    h[t] = 0;
    int e = -1;
    if (i < F) { const int64_t v = sel[i] - lo; if (v >= 0 && v < n) e = (int) v; }
    es[t] = e;
    __syncthreads();
    if (e >= 0)
    {
        atomicAdd(&h[e], 1);
        int rk = 0;
        for (int j = 0; j < t; ++j) rk += es[j] == e;
        rank[i] = rk;
    }
    __syncthreads();
    if (t < n) hist[(size_t) blockIdx.x * n + t] = h[t];
}

__global__ void __launch_bounds__(256) disp_scan_kernel(int* __restrict__ hist, int nblk, int n, int bm, int balance,
                                                        int* __restrict__ counts, int* __restrict__ rbt, int nrb_max,
                                                        int* __restrict__ meta)
{
    __shared__ int sc[256], sr[256];
    const int e = threadIdx.x;
    int c = 0;
    if (e < n)
        for (int b = 0; b < nblk; ++b) { const int v = hist[(size_t) b * n + e]; hist[(size_t) b * n + e] = c; c += v; }
    const int nb = e < n ? (c + bm - 1) / bm : 0;
    sc[e] = c; sr[e] = nb;
    __syncthreads();
    // inclusive scans of counts and row blocks (Hillis-Steele over 256)
    for (int off = 1; off < 256; off <<= 1)
    {
        const int a = e >= off ? sc[e - off] : 0, b = e >= off ? sr[e - off] : 0;
        __syncthreads();
        sc[e] += a; sr[e] += b;
        __syncthreads();
    }
    const int off_e = sc[e] - c, rb0 = sr[e] - nb;
    if (e < n)
    {
        counts[e] = c;
        for (int b = 0; b < nblk; ++b) hist[(size_t) b * n + e] += off_e;
        for (int k = 0; k < nb; ++k)
        {
            int rows, start;
            if (balance) { const int bs = c / nb, ex = c % nb; rows = bs + (k < ex ? 1 : 0); start = k * bs + (k < ex ? k : ex); }
            else { rows = min(bm, c - bm * k); start = bm * k; }
            const int r = rb0 + k;
            if (r < nrb_max) { rbt[4 * r + 0] = e; rbt[4 * r + 1] = off_e + start; rbt[4 * r + 2] = rows; rbt[4 * r + 3] = 0; }
        }
    }
    if (e == 255) { meta[0] = sc[255]; meta[1] = min(sr[255], nrb_max); meta[2] = sr[255]; meta[3] = 0; }
}

__global__ void __launch_bounds__(DBLK) disp_place_kernel(const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw,
    int F, int topk, int lo, int n, const int* __restrict__ hist, const int* __restrict__ rank, int* __restrict__ tok,
    int* __restrict__ eid, float* __restrict__ wt, int* __restrict__ inv)
{
    const int i = blockIdx.x * DBLK + threadIdx.x;
    if (i >= F) return;
    const int64_t v = sel[i] - lo;
    if (v < 0 || v >= n) { inv[i] = -1; return; }
    const int e = (int) v;
    const int p = hist[(size_t) blockIdx.x * n + e] + rank[i];
    tok[p] = i / topk; eid[p] = e; wt[p] = (float) __builtin_bit_cast(_Float16, rw[i]); inv[i] = p;
}

// ---------------------------------------------------------------------------------------------------------------
// grouped GEMMs
// ---------------------------------------------------------------------------------------------------------------
struct Block { int e, p0, rows; };

__device__ __forceinline__ bool get_block(const int* rbt, int nrb, const int* meta, int n_tab, Block& b)
{
    const int rb = blockIdx.x;
    if (rb >= nrb || (meta && rb >= meta[1])) return false;
    b.e = rbt[4 * rb]; b.p0 = rbt[4 * rb + 1]; b.rows = min(rbt[4 * rb + 2], PB);
    return b.e >= 0 && b.e < n_tab && b.rows > 0;
}

// stage one 128-k group of the block's input rows (bf16 rows of x, gathered) into LDS as f16: thread t copies
// row t/4, 32 values at (t%4)*32
__device__ __forceinline__ void load_x_bf16(const uint16_t* src_row, int k0, u32x4* v)
{
    #pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = src_row ? *(const u32x4*) (src_row + k0 + 8 * q) : (u32x4) {0u, 0u, 0u, 0u};
}
__device__ __forceinline__ void store_x_bf16(_Float16* xs, const u32x4* v)
{
    const int t = threadIdx.x, r = t >> 2, c = (t & 3) * 32;
    #pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        f16x8 o;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            o[2 * k] = (_Float16) __uint_as_float(v[q][k] << 16);
            o[2 * k + 1] = (_Float16) __uint_as_float(v[q][k] & 0xffff0000u);
        }
        *(f16x8*) (xs + r * XSTR + c + 8 * q) = o;
    }
}
__device__ __forceinline__ void load_x_f16(const _Float16* src_row, int k0, u32x4* v)
{
    #pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = src_row ? *(const u32x4*) (src_row + k0 + 8 * q) : (u32x4) {0u, 0u, 0u, 0u};
}
__device__ __forceinline__ void store_x_f16(_Float16* xs, const u32x4* v)
{
    const int t = threadIdx.x, r = t >> 2, c = (t & 3) * 32;
    #pragma unroll
    for (int q = 0; q < 4; ++q) *(u32x4*) (xs + r * XSTR + c + 8 * q) = v[q];
}

// A operand of one strip for one 128-k group: 4 k steps of 8 f16 per lane
struct AFrag { f16x8 a[4]; };

__device__ __forceinline__ void a_i4(const uint8_t* q, const uint8_t* s, int nb, int kg, int KG, AFrag& f)
{
    const int l = threadIdx.x & 63;
    const u32x4 w = ldw16(q + ((size_t) (nb * KG + kg) * 64 + l) * 16);
    const uint16_t sb = ldg<uint16_t>(s + ((size_t) (nb * 16 + (l & 15)) * KG + kg) * 2);
    const _Float16 sh = (_Float16) bf2f(sb);
    const f16x8 s8 = {sh, sh, sh, sh, sh, sh, sh, sh};
    #pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = dq8(w[t]) * s8;
}
__device__ __forceinline__ void a_dense(const uint8_t* w, int nb, int kg, int KS, AFrag& f)
{
    const int l = threadIdx.x & 63;
    #pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = as_f16x8(ldw16(w + ((size_t) (nb * KS + kg * 4 + t) * 64 + l) * 16));
}

// gate + up + act. DENSE: the shared expert over every token (block b = tokens [64 b, 64 b + 64), weight 1).
template <bool DENSE>
__global__ void __launch_bounds__(PT) pgu_kernel(
    const uint16_t* __restrict__ x, const int* __restrict__ tok, const float* __restrict__ wt,
    const int* __restrict__ rbt, int nrb, const int* __restrict__ meta, int n_tab,
    const int64_t* __restrict__ gw, const int64_t* __restrict__ uw, const int64_t* __restrict__ gs,
    const int64_t* __restrict__ us, const uint8_t* __restrict__ shg, const uint8_t* __restrict__ shu,
    _Float16* __restrict__ ar, int T, int ar_off)
{
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][PB * XSTR];
    Block b;
    if (DENSE) { b.e = 0; b.p0 = blockIdx.x * PB; b.rows = min(PB, T - b.p0); if (b.rows <= 0) return; }
    else if (!get_block(rbt, nrb, meta, n_tab, b)) return;
    constexpr int KG = H / 128;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    const int nb0 = blockIdx.y * (PN / 16) + 2 * w;            // strips nb0, nb0 + 1 of I / 16
    const uint8_t *gq = nullptr, *uq = nullptr, *gsp = nullptr, *usp = nullptr;
    if (!DENSE) { gq = (const uint8_t*) gw[b.e]; uq = (const uint8_t*) uw[b.e]; gsp = (const uint8_t*) gs[b.e]; usp = (const uint8_t*) us[b.e]; }
    // this thread's staged input row
    const int sr = t >> 2;
    const uint16_t* src = nullptr;
    if (sr < b.rows)
    {
        const int tk = DENSE ? b.p0 + sr : tok[b.p0 + sr];
        if ((unsigned) tk < (unsigned) T) src = x + (size_t) tk * H + (t & 3) * 32;
    }
    const int ntt = (b.rows + 15) >> 4;
    f32x4 acc[2][2][4];
    #pragma unroll
    for (int s = 0; s < 2; ++s)
        #pragma unroll
        for (int m = 0; m < 2; ++m)
            #pragma unroll
            for (int tt = 0; tt < 4; ++tt) acc[s][m][tt] = (f32x4) {0.f, 0.f, 0.f, 0.f};
    u32x4 xv[4];
    load_x_bf16(src, 0, xv);
    for (int kg = 0; kg < KG; ++kg)
    {
        _Float16* xb = xs[kg & 1];
        store_x_bf16(xb, xv);
        __syncthreads();
        if (kg + 1 < KG) load_x_bf16(src, (kg + 1) * 128, xv);
        AFrag A[2][2];
        #pragma unroll
        for (int s = 0; s < 2; ++s)
        {
            if (DENSE) { a_dense(shg, nb0 + s, kg, H / 32, A[s][0]); a_dense(shu, nb0 + s, kg, H / 32, A[s][1]); }
            else { a_i4(gq, gsp, nb0 + s, kg, KG, A[s][0]); a_i4(uq, usp, nb0 + s, kg, KG, A[s][1]); }
        }
        #pragma unroll
        for (int tt = 0; tt < 4; ++tt)
        {
            if (tt >= ntt) break;
            const _Float16* bp = xb + (tt * 16 + (l & 15)) * XSTR + 8 * (l >> 4);
            #pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const f16x8 bv = *(const f16x8*) (bp + 32 * k);
                #pragma unroll
                for (int s = 0; s < 2; ++s)
                    #pragma unroll
                    for (int m = 0; m < 2; ++m) acc[s][m][tt] = mfma16(A[s][m].a[k], bv, acc[s][m][tt]);
            }
        }
    }
    // epilogue: lane holds rows 4(l/16)..+4 of pick tt*16 + l%16
    #pragma unroll
    for (int tt = 0; tt < 4; ++tt)
    {
        const int pk = tt * 16 + (l & 15);
        if (pk >= b.rows) continue;
        const float wv = DENSE ? 1.0f : wt[b.p0 + pk];
        #pragma unroll
        for (int s = 0; s < 2; ++s)
        {
            const int n = (nb0 + s) * 16 + 4 * (l >> 4);
            _Float16 o[4];
            #pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (_Float16) (silu(acc[s][0][tt][i]) * acc[s][1][tt][i] * wv);
            *(uint2*) (ar + (size_t) (ar_off + b.p0 + pk) * I + n) = *(const uint2*) o;
        }
    }
}

// down: d[pick] = W_d act[pick] (fp32)
template <bool DENSE>
__global__ void __launch_bounds__(PT) pdown_kernel(
    const _Float16* __restrict__ ar, const int* __restrict__ rbt, int nrb, const int* __restrict__ meta, int n_tab,
    const int64_t* __restrict__ dw, const int64_t* __restrict__ ds, const uint8_t* __restrict__ shd,
    float* __restrict__ d, int T, int off)
{
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][PB * XSTR];
    Block b;
    if (DENSE) { b.e = 0; b.p0 = blockIdx.x * PB; b.rows = min(PB, T - b.p0); if (b.rows <= 0) return; }
    else if (!get_block(rbt, nrb, meta, n_tab, b)) return;
    constexpr int KG = I / 128;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    const int nb0 = blockIdx.y * (PN / 16) + 2 * w;
    const uint8_t *dq = nullptr, *dsp = nullptr;
    if (!DENSE) { dq = (const uint8_t*) dw[b.e]; dsp = (const uint8_t*) ds[b.e]; }
    const int sr = t >> 2;
    const _Float16* src = sr < b.rows ? ar + (size_t) (off + b.p0 + sr) * I + (t & 3) * 32 : nullptr;
    const int ntt = (b.rows + 15) >> 4;
    f32x4 acc[2][4];
    #pragma unroll
    for (int s = 0; s < 2; ++s)
        #pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[s][tt] = (f32x4) {0.f, 0.f, 0.f, 0.f};
    u32x4 xv[4];
    load_x_f16(src, 0, xv);
    for (int kg = 0; kg < KG; ++kg)
    {
        _Float16* xb = xs[kg & 1];
        store_x_f16(xb, xv);
        __syncthreads();
        if (kg + 1 < KG) load_x_f16(src, (kg + 1) * 128, xv);
        AFrag A[2];
        #pragma unroll
        for (int s = 0; s < 2; ++s)
        {
            if (DENSE) a_dense(shd, nb0 + s, kg, I / 32, A[s]);
            else a_i4(dq, dsp, nb0 + s, kg, KG, A[s]);
        }
        #pragma unroll
        for (int tt = 0; tt < 4; ++tt)
        {
            if (tt >= ntt) break;
            const _Float16* bp = xb + (tt * 16 + (l & 15)) * XSTR + 8 * (l >> 4);
            #pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const f16x8 bv = *(const f16x8*) (bp + 32 * k);
                #pragma unroll
                for (int s = 0; s < 2; ++s) acc[s][tt] = mfma16(A[s].a[k], bv, acc[s][tt]);
            }
        }
    }
    #pragma unroll
    for (int tt = 0; tt < 4; ++tt)
    {
        const int pk = tt * 16 + (l & 15);
        if (pk >= b.rows) continue;
        #pragma unroll
        for (int s = 0; s < 2; ++s)
        {
            const int n = (nb0 + s) * 16 + 4 * (l >> 4);
            *(f32x4*) (d + (size_t) (off + b.p0 + pk) * H + n) = acc[s][tt];
        }
    }
}

// fin, deterministic: out[t] += (sum over k in top-k order of d[inv[t][k]]) (+ the shared expert's row)
__global__ void __launch_bounds__(256) pfin_kernel(const float* __restrict__ d, const int* __restrict__ inv, int topk,
                                                   int sh_off, float* __restrict__ out)
{
    const int t = blockIdx.x;
    int pos[HMOE_TOPK];
    #pragma unroll
    for (int k = 0; k < HMOE_TOPK; ++k) pos[k] = k < topk ? inv[(size_t) t * topk + k] : -1;
    for (int n = threadIdx.x * 4; n < H; n += 256 * 4)
    {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int k = 0; k < HMOE_TOPK; ++k)
            if (pos[k] >= 0) s += *(const f32x4*) (d + (size_t) pos[k] * H + n);
        if (sh_off >= 0) s += *(const f32x4*) (d + (size_t) (sh_off + t) * H + n);
        f32x4* o = (f32x4*) (out + (size_t) t * H + n);
        *o = *o + s;
    }
}

// fin with atomics (p4_fin_kernel, moe4p.cu:195-206)
__global__ void __launch_bounds__(256) pfin_atomic_kernel(const float* __restrict__ d, const int* __restrict__ tok,
                                                          int npos, const int* __restrict__ meta, int T,
                                                          float* __restrict__ out)
{
    const int p = blockIdx.x;
    if (p >= npos || (meta && p >= meta[0])) return;
    const int tk = tok[p];
    if ((unsigned) tk >= (unsigned) T) return;
    for (int n = threadIdx.x; n < H; n += 256) atomicAdd(out + (size_t) tk * H + n, d[(size_t) p * H + n]);
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_dispatch_work_bytes(int T, int topk, int n)
{
    const size_t F = (size_t) T * topk, nblk = (F + DBLK - 1) / DBLK;
    return (nblk * (size_t) n + F) * sizeof(int);
}

extern "C" int hmoe_dispatch_nrb_max(int npos_max, int n, int bm)
{
    if (bm <= 0) return 0;
    return n + npos_max / bm;
}

extern "C" int hmoe_dispatch(const int64_t* sel, const uint16_t* rw, int T, int topk, int lo, int n, int bm,
                             int balance, int* counts, int* tok, int* eid, float* wt, int* inv, int* rbt, int nrb_max,
                             int* meta, void* work, void* stream)
{
    HMOE_REQUIRE(sel && rw && counts && tok && eid && wt && inv && rbt && meta && work, "dispatch: null buffer");
    HMOE_REQUIRE(T >= 1 && topk >= 1 && topk <= TOPK && n >= 1 && n <= 256 && lo >= 0 && bm >= 1 && nrb_max >= 1,
                 "dispatch: T %d topk %d n %d bm %d", T, topk, n, bm);
    const int F = T * topk, nblk = (F + DBLK - 1) / DBLK;
    int* hist = (int*) work;
    int* rank = hist + (size_t) nblk * n;
    hipStream_t st = (hipStream_t) stream;
    disp_count_kernel<<<nblk, DBLK, 0, st>>>(sel, F, lo, n, hist, rank);
    disp_scan_kernel<<<1, 256, 0, st>>>(hist, nblk, n, bm, balance, counts, rbt, nrb_max, meta);
    disp_place_kernel<<<nblk, DBLK, 0, st>>>(sel, rw, F, topk, lo, n, hist, rank, tok, eid, wt, inv);
    return HMOE_LAUNCHED("dispatch");
}

extern "C" size_t hmoe_moe4p_scratch_bytes(int which, int ps, int T)
{
    switch (which)
    {
        case 0: return 16;                                              // gu: unused (gate/up fused with act)
        case 1: return (size_t) (ps + T) * I * 2;                       // ar f16 [ps + T][I]
        case 2: return (size_t) (ps + T) * H * 4;                       // d fp32 [ps + T][H]
        default: return 0;
    }
}

extern "C" int hmoe_moe4p_forward(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt,
                                  int npos, int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw,
                                  const int64_t* gs, const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar,
                                  float* d, float* out, int ps, const int* meta, const int* inv, int T, int topk,
                                  const void* sh_gw, const void* sh_uw, const void* sh_dw, void* stream)
{
    (void) gu; (void) eid;
    HMOE_REQUIRE(x && tok && wt && rbt && ar && d && out, "moe4p_forward: null buffer");
    HMOE_REQUIRE(npos >= 0 && nrb >= 0 && npos <= ps && T >= 1 && topk >= 1 && topk <= TOPK,
                 "moe4p_forward: npos %d nrb %d ps %d T %d topk %d", npos, nrb, ps, T, topk);
    HMOE_REQUIRE(n_tab >= 0 && n_tab <= HMOE_MAXE && (n_tab == 0 || (gw && uw && dw && gs && us && ds)),
                 "moe4p_forward: tables");
    HMOE_REQUIRE((!sh_gw && !sh_uw && !sh_dw) || (sh_gw && sh_uw && sh_dw && inv), "moe4p_forward: shared expert");
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) ar & 15) == 0 && ((uintptr_t) d & 15) == 0 &&
                 ((uintptr_t) out & 15) == 0, "moe4p_forward: alignment");
    hipStream_t st = (hipStream_t) stream;
    const uint16_t* xb = (const uint16_t*) x;
    _Float16* a = (_Float16*) ar;
    if (nrb > 0)
    {
        pgu_kernel<false><<<dim3(nrb, I / PN), PT, 0, st>>>(xb, tok, wt, rbt, nrb, meta, n_tab, gw, uw, gs, us, nullptr,
                                                           nullptr, a, T, 0);
        pdown_kernel<false><<<dim3(nrb, H / PN), PT, 0, st>>>(a, rbt, nrb, meta, n_tab, dw, ds, nullptr, d, T, 0);
    }
    const bool sh = sh_gw != nullptr;
    if (sh)
    {
        const int nbk = (T + PB - 1) / PB;
        pgu_kernel<true><<<dim3(nbk, I / PN), PT, 0, st>>>(xb, nullptr, nullptr, nullptr, 0, nullptr, 1, nullptr, nullptr,
                                                          nullptr, nullptr, (const uint8_t*) sh_gw, (const uint8_t*) sh_uw,
                                                          a, T, ps);
        pdown_kernel<true><<<dim3(nbk, H / PN), PT, 0, st>>>(a, nullptr, 0, nullptr, 1, nullptr, nullptr,
                                                            (const uint8_t*) sh_dw, d, T, ps);
    }
    if (inv) pfin_kernel<<<T, 256, 0, st>>>(d, inv, topk, sh ? ps : -1, out);
    else if (npos > 0) pfin_atomic_kernel<<<npos, 256, 0, st>>>(d, tok, npos, meta, T, out);
    return HMOE_LAUNCHED("moe4p_forward");
}
