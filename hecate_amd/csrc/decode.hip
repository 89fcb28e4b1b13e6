// decode.hip - the decode MoE op (runtime/tier/moe4/moe4.cu:828-895 moe4_forward) for 1..16 rows on gfx950, and the
// whole decode layer (router + experts) in the same launches.
//
// Design rules, from measurement on MI355X:
//   * the only vector-memory loads in a streaming loop are the 1 KB weight tiles (one 16-byte load per lane); group
//     scales come 4 k groups per load, and the activations stay in registers for the whole kernel: every extra vector
//     load per tile (a scale, an activation fragment from L2) costs 15-30 % of the achieved HBM bandwidth;
//   * loads are unconditional and double-buffered per item (ping-pong between two register sets), so every wait
//     counts exactly and the next item's tiles are in flight across the item's reduction barrier;
//   * no workgroup waits for another inside a launch (on gfx950 an agent-scope fence writes back and invalidates
//     L2): cross-workgroup sums are cut at a kernel boundary and done in a fixed order (bit-reproducible results).
//
// MFMA roles: the token rows are the A operand (16 x 32 per k step, 16 tokens), the dequantised weight tile the B
// operand (32 k x 16 weight rows), so a lane's outputs share one weight row n = l % 16 and one group scale:
// lane l holds D[tokens 4(l/16)..+4][row l%16].
//
// Launches (main stream; the shared expert runs on a side stream, joined before the reduction):
//   router   logits of two experts per workgroup (fixed fp32 order, see hecate_moe.h)
//   gate/up  every workgroup derives the step's routing (top-k from the logits, or the given sel / rw) and the
//            distinct experts (moe4.cu:86-110), then takes items (slot, 16-row block nb) b, b + G, ...; 12 waves each
//            own 4 k groups of H with the rows' x in registers; the 12 wave partials are summed in wave order through
//            LDS and act[slot][r][n] = f16(silu(g) u w) is written (moe4.cu:645-676)
//   down     items (slot quad, 16-row block of H), contiguous per workgroup; 16 waves = 4 slots x 4 k quarters of I
//            with the slots' act in registers; the 16 partials are summed in order into y32[part] (moe4.cu:443-643)
//   reduce   y[r] (+)= sum of the parts in order (moe4.cu:826-827 accumulates into y), or the layer's bf16 output
//   side     shared gate/up (F16T, act slot SH_SLOT, weight 1), shared down (part 0)
#include "hmoe_dev.h"

namespace hmoe {

constexpr int NW = 8, NT = NW * 64;        // router / shared gate-up workgroup
constexpr int KG_H = H / 128;              // 48 k groups of gate / up
constexpr int KG_I = I / 128;              // 16 k groups of down
constexpr int NB_I = I / 16;               // 128 row blocks of gate / up
constexpr int NB_H = H / 16;               // 384 row blocks of down
constexpr int KS_H = H / 32;               // 192 F16T k steps of gate / up
constexpr int KS_I = I / 32;               // 64 F16T k steps of down
constexpr int GW = 12;                     // gate/up waves: wave w owns k groups [4w, 4w + 4) of H
constexpr int DW = 16;                     // down waves: slot w / 4 of the quad, k groups [4 (w % 4), +4) of I
constexpr int MAX_PARTS = 1 + MAXSLOT / 4;
constexpr int CTR_WORDS = 1024;            // ctr[0]: the part count of the last down launch

struct Route
{
    int m;
    unsigned mask[8];
    short e[MAXSLOT];
    float w[MAXSLOT][MAXR];
};

// distinct experts of the step (ascending local id) and routing weight per (slot, row): moe4.cu:86-110, with the slot
// of each pick from popcounts of the 256-bit mask. sel / rw may be in LDS or global memory. Ends with a barrier.
__device__ void route(const int64_t* sel, const uint16_t* rw, int R, int lo, int n_hot, Route& rt)
{
    const int t = threadIdx.x, np = R * TOPK;
    if (t < 8) rt.mask[t] = 0u;
    for (int i = t; i < MAXSLOT * MAXR; i += blockDim.x) (&rt.w[0][0])[i] = 0.f;
    int e = -1; float wv = 0.f;
    if (t < np)
    {
        const int64_t s = sel[t] - lo;
        if (s >= 0 && s < n_hot) { e = (int) s; wv = (float) __builtin_bit_cast(_Float16, rw[t]); }
    }
    __syncthreads();
    if (e >= 0) atomicOr(&rt.mask[e >> 5], 1u << (e & 31));
    __syncthreads();
    if (e >= 0)
    {
        int slot = __popc(rt.mask[e >> 5] & ((1u << (e & 31)) - 1u));
        for (int wd = 0; wd < (e >> 5); ++wd) slot += __popc(rt.mask[wd]);
        rt.e[slot] = (short) e;
        atomicAdd(&rt.w[slot][t / TOPK], wv);
    }
    if (t == 0) { int m = 0; for (int wd = 0; wd < 8; ++wd) m += __popc(rt.mask[wd]); rt.m = m; }
    __syncthreads();
}

// bf16 group scale k (0..3) of the four packed in s
__device__ __forceinline__ float scale_of(u32x2 s, int k)
{
    const uint32_t v = s[k >> 1];
    return __uint_as_float((k & 1) ? (v & 0xffff0000u) : (v << 16));
}

// 8 bf16 -> 8 f16
__device__ __forceinline__ f16x8 bf8_to_f16(u32x4 v)
{
    f16x8 o;
    #pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        o[2 * k] = (_Float16) __uint_as_float(v[k] << 16);
        o[2 * k + 1] = (_Float16) __uint_as_float(v[k] & 0xffff0000u);
    }
    return o;
}

// one 128-k group of an I4G128 tile (weights as the B operand) against 4 k steps of token rows: scaled into acc
__device__ __forceinline__ void group_i4(const f16x8* xa, u32x4 wq, float s, f32x4& acc, const DqConsts& dq)
{
    f32x4 p = {0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int t = 0; t < 4; ++t) p = mfma16(xa[t], dq8(wq[t], dq), p);
    #pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(s, p[i], acc[i]);
}

// ---- router logits: two experts per 512-thread workgroup (expert_logits) ----
__global__ void __launch_bounds__(NT) router_kernel(const uint16_t* __restrict__ x, int R, const float* __restrict__ wt,
                                                    int E, float* __restrict__ logits)
{
    __shared__ float sums[2][256][MAXR + 1];
    const int half = threadIdx.x >> 8, tid = threadIdx.x & 255;
    expert_logits(x, wt, 2 * blockIdx.x + half, E, R, H, tid, sums[half], logits);
}

// ---- routed gate/up ----
struct GuItem
{
    u32x4 g[4], u[4];                       // the wave's 4 k groups of gate and up (one 16-byte load per lane each)
    u32x2 sg, su;                           // their 4 group scales of the lane's row
};

__global__ void __launch_bounds__(GW * 64) gu5_kernel(
    const void* __restrict__ x, int xf, const float* __restrict__ logits, const float* __restrict__ bias, int E,
    int topk, float scale, int64_t* __restrict__ sel, uint16_t* __restrict__ rw, int R, int lo, int n_hot,
    const int64_t* __restrict__ gate_w, const int64_t* __restrict__ up_w, const int64_t* __restrict__ gate_s,
    const int64_t* __restrict__ up_s, _Float16* __restrict__ act)
{
    __shared__ Route rt;
    __shared__ const uint8_t* ptr[4][MAXSLOT];
    __shared__ int64_t ssel[MAXR * TOPK];
    __shared__ uint16_t srw[MAXR * TOPK];
    __shared__ f32x4 red[2][GW][2][64];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, ks = l >> 4;
    const bool live = tok < R;
    // the rows' x for this wave's k range: k step t covers k = 512 w + 32 t + 8 ks .. + 8 of row tok (A operand)
    f16x8 xa[16];
    {
        const uint16_t* xr = (const uint16_t*) x + (size_t) (live ? tok : 0) * H + 512 * w + 8 * ks;
        #pragma unroll
        for (int t = 0; t < 16; ++t)
        {
            const u32x4 v = ld16(xr + 32 * t);
            xa[t] = live ? (xf ? as_f16x8(v) : bf8_to_f16(v)) : (f16x8) {};
        }
    }
    if (logits)
    {
        if (w < R) select_row(logits + (size_t) w * RMAXE, bias, E, topk, scale, ssel + w * TOPK, srw + w * TOPK);
        if (w + GW < R)
            select_row(logits + (size_t) (w + GW) * RMAXE, bias, E, topk, scale, ssel + (w + GW) * TOPK,
                       srw + (w + GW) * TOPK);
        __syncthreads();
        if (blockIdx.x == 0 && threadIdx.x < R * TOPK) { sel[threadIdx.x] = ssel[threadIdx.x]; rw[threadIdx.x] = srw[threadIdx.x]; }
        route(ssel, srw, R, lo, n_hot, rt);
    }
    else route(sel, rw, R, lo, n_hot, rt);
    const int m = rt.m;
    if (threadIdx.x < m)
    {
        const int e = rt.e[threadIdx.x];
        ptr[0][threadIdx.x] = (const uint8_t*) gate_w[e]; ptr[1][threadIdx.x] = (const uint8_t*) up_w[e];
        ptr[2][threadIdx.x] = (const uint8_t*) gate_s[e]; ptr[3][threadIdx.x] = (const uint8_t*) up_s[e];
    }
    __syncthreads();
    const int G = gridDim.x, total = m * NB_I;
    const int nmine = (int) blockIdx.x < total ? (total - 1 - (int) blockIdx.x) / G + 1 : 0;
    if (nmine == 0) return;                                    // uniform over the workgroup
    const int row = l & 15;
    const DqConsts dq = dq_consts();
    auto load = [&](GuItem& S, int i) {
        const int it = blockIdx.x + i * G, j = it / NB_I, nb = it - j * NB_I;
        const size_t toff = ((size_t) (nb * KG_H + 4 * w) * 64 + l) * 16;
        const size_t soff = ((size_t) (nb * 16 + row) * KG_H + 4 * w) * 2;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            S.g[k] = ldw16(ptr[0][j] + toff + k * 1024);
            S.u[k] = ldw16(ptr[1][j] + toff + k * 1024);
        }
        S.sg = ld8(ptr[2][j] + soff); S.su = ld8(ptr[3][j] + soff);
    };
    auto run = [&](const GuItem& S, int i, int par) {
        const int it = blockIdx.x + i * G, j = it / NB_I, nb = it - j * NB_I;
        f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            group_i4(xa + 4 * k, S.g[k], scale_of(S.sg, k), ag, dq);
            group_i4(xa + 4 * k, S.u[k], scale_of(S.su, k), au, dq);
        }
        red[par][w][0][l] = ag; red[par][w][1][l] = au;
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int ll = threadIdx.x >> 2, ie = threadIdx.x & 3, tk = 4 * (ll >> 4) + ie;
            if (tk < R)
            {
                float g = 0.f, u = 0.f;
                #pragma unroll
                for (int ww = 0; ww < GW; ++ww) { g += red[par][ww][0][ll][ie]; u += red[par][ww][1][ll][ie]; }
                act[((size_t) j * MAXR + tk) * I + nb * 16 + (ll & 15)] = (_Float16) (silu(g) * u * rt.w[j][tk]);
            }
        }
        // red[par] is written again two items later, after the next item's barrier: no second barrier needed
    };
    GuItem A, B;
    load(A, 0);
    for (int i = 0; i < nmine; i += 2)
    {
        load(B, min(i + 1, nmine - 1));
        run(A, i, 0);
        if (i + 1 >= nmine) break;
        load(A, min(i + 2, nmine - 1));
        run(B, i + 1, 1);
    }
}

// ---- routed down ----
struct DnItem
{
    u32x4 d[4];                             // the wave's 4 k groups of one 16-row block of down
    u32x2 s;                                // their 4 group scales of the lane's row
};

__global__ void __launch_bounds__(DW * 64) dn5_kernel(
    const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw, int R, int lo, int n_hot,
    const int64_t* __restrict__ down_w, const int64_t* __restrict__ down_s, const _Float16* __restrict__ act,
    float* __restrict__ y32, int* __restrict__ nparts_out, int part0)
{
    __shared__ Route rt;
    __shared__ const uint8_t* ptr[2][MAXSLOT];
    __shared__ f32x4 red[2][DW][64];
    route(sel, rw, R, lo, n_hot, rt);
    const int m = rt.m, nq = (m + 3) / 4;
    if (threadIdx.x < m)
    {
        const int e = rt.e[threadIdx.x];
        ptr[0][threadIdx.x] = (const uint8_t*) down_w[e]; ptr[1][threadIdx.x] = (const uint8_t*) down_s[e];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *nparts_out = part0 + nq;
    __syncthreads();
    // items (quad, nb), quad-major, a contiguous range per workgroup (the act of a quad stays in registers)
    const int G = gridDim.x, total = nq * NB_H;
    const int i0 = (int) (((long long) total * blockIdx.x) / G), i1 = (int) (((long long) total * (blockIdx.x + 1)) / G);
    const int nmine = i1 - i0;
    if (nmine <= 0) return;                                    // uniform over the workgroup
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, ks = l >> 4, row = l & 15;
    const int sw = w >> 2, kq = w & 3;                          // slot of the quad, k quarter of I
    const bool live = tok < R;
    f16x8 xa[16];
    int cur_q = -1;
    const DqConsts dq = dq_consts();
    auto load = [&](DnItem& S, int i) {
        const int it = i0 + i, qd = it / NB_H, nb = it - qd * NB_H, j = 4 * qd + sw;
        // a slot past m loads one fixed tile of slot m - 1 (the same load count on every path, no HBM traffic)
        const bool ok = j < m;
        const int jj = ok ? j : m - 1, nbb = ok ? nb : 0;
        const size_t toff = ((size_t) (nbb * KG_I + 4 * kq) * 64 + l) * 16;
        const size_t soff = ((size_t) (nbb * 16 + row) * KG_I + 4 * kq) * 2;
        #pragma unroll
        for (int k = 0; k < 4; ++k) S.d[k] = ldw16(ptr[0][jj] + toff + (ok ? k * 1024 : 0));
        S.s = ld8(ptr[1][jj] + soff);
    };
    auto run = [&](const DnItem& S, int i, int par) {
        const int it = i0 + i, qd = it / NB_H, nb = it - qd * NB_H;
        if (qd != cur_q)
        {
            // the quad's act rows for this wave's slot and k quarter (zero for a slot past m)
            cur_q = qd;
            const int j = 4 * qd + sw;
            const bool use = live && j < m;
            const _Float16* ar = act + ((size_t) min(j, m - 1) * MAXR + (live ? tok : 0)) * I + 512 * kq + 8 * ks;
            #pragma unroll
            for (int t = 0; t < 16; ++t)
            {
                const u32x4 v = ld16(ar + 32 * t);
                xa[t] = use ? as_f16x8(v) : (f16x8) {};
            }
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int k = 0; k < 4; ++k) group_i4(xa + 4 * k, S.d[k], scale_of(S.s, k), acc, dq);
        red[par][w][l] = acc;
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int ll = threadIdx.x >> 2, ie = threadIdx.x & 3, tk = 4 * (ll >> 4) + ie;
            if (tk < R)
            {
                float s = 0.f;
                #pragma unroll
                for (int ww = 0; ww < DW; ++ww) s += red[par][ww][ll][ie];
                y32[((size_t) (part0 + qd) * MAXR + tk) * H + nb * 16 + (ll & 15)] = s;
            }
        }
    };
    DnItem A, B;
    load(A, 0);
    for (int i = 0; i < nmine; i += 2)
    {
        load(B, min(i + 1, nmine - 1));
        run(A, i, 0);
        if (i + 1 >= nmine) break;
        load(A, min(i + 2, nmine - 1));
        run(B, i + 1, 1);
    }
}

// the 8 wave partials of a 16-row block, summed in wave order: thread t < 256 gets (row t/16, token t%16) of the
// standard MFMA output layout (lane l: rows 4(l/16)..+4, column l%16)
__device__ __forceinline__ float wave_sum(const float (*red)[64][8], int comp)
{
    const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
    const int ll = (row >> 2) * 16 + tk, ie = row & 3;
    float s = 0.f;
    #pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w][ll][comp + ie];
    return s;
}

// ---- shared gate/up (F16T, full K per item nb): 8 waves on 8 k ranges, act[SH_SLOT] = f16(silu(g) u) ----
template <int D>
__global__ void __launch_bounds__(512) sh_gu_kernel(const void* __restrict__ x, int xf, int R,
                                                    const uint8_t* __restrict__ gw, const uint8_t* __restrict__ uw,
                                                    _Float16* __restrict__ act)
{
    constexpr int KW = KS_H / 8;                                       // 24 k steps per wave
    static_assert(KW % D == 0, "the ring depth divides the k steps of a wave");
    __shared__ float red[8][64][8];
    const int nb = blockIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, ks = l >> 4;
    const bool live = tok < R;
    const size_t xo = (size_t) (live ? tok : 0) * H + 8 * ks;
    const size_t off0 = ((size_t) (nb * KS_H + w * KW) * 64 + l) * 16;
    u32x4 gq[D], uq[D], xq[D];
    auto issue = [&](int q, auto sc) {
        constexpr int s = decltype(sc)::value;
        gq[s] = ldw16(gw + off0 + (size_t) q * 1024); uq[s] = ldw16(uw + off0 + (size_t) q * 1024);
        xq[s] = ld16((const uint16_t*) x + xo + (size_t) (w * KW + q) * 32);   // bf16 or f16: 8 elements
    };
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
    static_for<D>([&](auto sc) { issue(decltype(sc)::value, sc); });
    for (int q0 = 0; q0 < KW; q0 += D)
        static_for<D>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            f16x8 bv = {};
            if (live) bv = xf ? as_f16x8(xq[s]) : bf8_to_f16(xq[s]);
            ag = mfma16(as_f16x8(gq[s]), bv, ag);
            au = mfma16(as_f16x8(uq[s]), bv, au);
            if (q0 + s + D < KW) issue(q0 + s + D, sc);
        });
    #pragma unroll
    for (int i = 0; i < 4; ++i) { red[w][l][i] = ag[i]; red[w][l][4 + i] = au[i]; }
    __syncthreads();
    if (threadIdx.x < 256)
    {
        const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
        if (tk < R)
        {
            const float g = wave_sum(red, 0), u = wave_sum(red, 4);
            act[((size_t) SH_SLOT * MAXR + tk) * I + nb * 16 + row] = (_Float16) (silu(g) * u);
        }
    }
}

// ---- shared down (F16T, item nb of H): 4 waves on 4 k ranges of I -> y32[0] ----
template <int D>
__global__ void __launch_bounds__(256) sh_dn_kernel(int R, const uint8_t* __restrict__ dw,
                                                    const _Float16* __restrict__ act, float* __restrict__ y32)
{
    constexpr int KW = KS_I / 4;                                       // 16 k steps per wave
    static_assert(KW % D == 0, "the ring depth divides the k steps of a wave");
    __shared__ f32x4 red[4][64];
    const int nb = blockIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, ks = l >> 4;
    const bool live = tok < R;
    const _Float16* arow = act + ((size_t) SH_SLOT * MAXR + (live ? tok : 0)) * I + 8 * ks + w * KW * 32;
    const size_t off0 = ((size_t) (nb * KS_I + w * KW) * 64 + l) * 16;
    u32x4 dq[D], xq[D];
    auto issue = [&](int q, auto sc) {
        constexpr int s = decltype(sc)::value;
        dq[s] = ldw16(dw + off0 + (size_t) q * 1024);
        xq[s] = ld16(arow + q * 32);
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    static_for<D>([&](auto sc) { issue(decltype(sc)::value, sc); });
    for (int q0 = 0; q0 < KW; q0 += D)
        static_for<D>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            acc = mfma16(as_f16x8(dq[s]), live ? as_f16x8(xq[s]) : (f16x8) {}, acc);
            if (q0 + s + D < KW) issue(q0 + s + D, sc);
        });
    red[w][l] = acc;
    __syncthreads();
    const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
    const int ll = (row >> 2) * 16 + tk, ie = row & 3;
    if (tk < R)
        y32[(size_t) tk * H + nb * 16 + row] = ((red[0][ll][ie] + red[1][ll][ie]) + red[2][ll][ie]) + red[3][ll][ie];
}

// ---- y (+)= sum of the parts in order; or the layer's bf16 output ----
__global__ void __launch_bounds__(256) dec_d_kernel(const float* __restrict__ y32, const int* __restrict__ nparts_p,
                                                    int R, float* __restrict__ y, uint16_t* __restrict__ out)
{
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= R * H) return;
    const int np = *nparts_p, r = i / H, n = i % H;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < np; ++p) s += *(const f32x4*) (y32 + ((size_t) p * MAXR + r) * H + n);
    if (y)
    {
        f32x4* yp = (f32x4*) (y + i);
        *yp = *yp + s;
    }
    if (out)
    {
        #pragma unroll
        for (int k = 0; k < 4; ++k) out[i + k] = hmoe_f2bf(s[k]);
    }
}

int default_grid(int per_cu)
{
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256 * per_cu;
    if (!cus[dev])
    {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = v;
    }
    return cus[dev] * per_cu;
}

struct DecodeArgs
{
    const void* x; int xf; const int64_t* sel_in; const uint16_t* rw_in; int R; int n_hot; int lo;
    const int64_t *gate_w, *up_w, *down_w, *gate_s, *up_s, *down_s;
    _Float16* act; int* ctr; float* y32; float* y; uint16_t* out;
    const void *sh_gw, *sh_uw, *sh_dw;
    const float* wt; const float* bias; float* logits; int E; int topk; float scale; int64_t* sel_out; uint16_t* rw_out;
    int blocks;
};

static int check(const DecodeArgs& a)
{
    HMOE_REQUIRE(a.R >= 1 && a.R <= MAXR, "moe4: rows %d not in [1, %d]", a.R, MAXR);
    HMOE_REQUIRE(a.n_hot >= 0 && a.n_hot <= HMOE_MAXE && a.lo >= 0, "moe4: window lo %d n_hot %d", a.lo, a.n_hot);
    HMOE_REQUIRE(a.x && a.act && a.ctr && a.y32, "moe4: null buffer");
    HMOE_REQUIRE(a.n_hot == 0 || (a.gate_w && a.up_w && a.down_w && a.gate_s && a.up_s && a.down_s), "moe4: null table");
    HMOE_REQUIRE((!a.sh_gw && !a.sh_uw && !a.sh_dw) || (a.sh_gw && a.sh_uw && a.sh_dw), "moe4: partial shared expert");
    HMOE_REQUIRE(((uintptr_t) a.x & 15) == 0 && ((uintptr_t) a.act & 15) == 0, "moe4: x / act not 16-byte aligned");
    HMOE_REQUIRE(a.blocks >= 0 && a.blocks <= 4096, "moe4: blocks %d", a.blocks);
    return HMOE_OK;
}

// the per-device side stream of the shared expert, joined back before the output reduction
struct SideStream
{
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};

static int side_stream(SideStream*& out)
{
    static SideStream ss[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(HMOE_ERR_HIP, "side stream: device");
    SideStream& d = ss[dev];
    if (!d.s)
    {
        if (hipStreamCreateWithFlags(&d.s, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&d.fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&d.join, hipEventDisableTiming) != hipSuccess)
            return set_error(HMOE_ERR_HIP, "side stream: create");
    }
    out = &d;
    return HMOE_OK;
}

// launches; phase mask bit 0 = router logits (+ the shared gate/up on the side stream), 1 = routed gate/up,
// 2 = routed down (+ the shared down on the side stream), 3 = ordered reduction. blocks: grid of the routed
// gate/up and down kernels (0 = one workgroup per CU).
static int run_decode(const DecodeArgs& a, int phases, hipStream_t st)
{
    const int R = a.R;
    const bool sh = a.sh_gw != nullptr;
    SideStream* ss = nullptr;
    if (sh)
    {
        const int rc = side_stream(ss);
        if (rc) return rc;
    }
    bool forked = false;
    auto fork = [&]() -> int {
        if (forked) return HMOE_OK;
        if (hipEventRecord(ss->fork, st) != hipSuccess || hipStreamWaitEvent(ss->s, ss->fork, 0) != hipSuccess)
            return set_error(HMOE_ERR_HIP, "moe4: fork");
        forked = true;
        return HMOE_OK;
    };
    const int G = a.blocks ? a.blocks : default_grid(1);
    if (phases & 1)
    {
        if (sh)
        {
            if (fork()) return HMOE_ERR_HIP;
            sh_gu_kernel<6><<<NB_I, 512, 0, ss->s>>>(a.x, a.xf, R, (const uint8_t*) a.sh_gw, (const uint8_t*) a.sh_uw,
                                                     a.act);
        }
        if (a.logits) router_kernel<<<(a.E + 1) / 2, NT, 0, st>>>((const uint16_t*) a.x, R, a.wt, a.E, a.logits);
    }
    const int64_t* sel = a.logits ? a.sel_out : a.sel_in;
    const uint16_t* rw = a.logits ? a.rw_out : a.rw_in;
    if (phases & 2)
        gu5_kernel<<<G, GW * 64, 0, st>>>(a.x, a.xf, a.logits, a.bias, a.E, a.topk, a.scale,
                                          a.logits ? a.sel_out : (int64_t*) a.sel_in,
                                          a.logits ? a.rw_out : (uint16_t*) a.rw_in, R, a.lo, a.n_hot, a.gate_w,
                                          a.up_w, a.gate_s, a.up_s, a.act);
    if (phases & 4)
    {
        if (sh)
        {
            if (fork()) return HMOE_ERR_HIP;
            sh_dn_kernel<8><<<NB_H, 256, 0, ss->s>>>(R, (const uint8_t*) a.sh_dw, a.act, a.y32);
        }
        dn5_kernel<<<G, DW * 64, 0, st>>>(sel, rw, R, a.lo, a.n_hot, a.down_w, a.down_s, a.act, a.y32, a.ctr,
                                          sh ? 1 : 0);
    }
    if (forked && (hipEventRecord(ss->join, ss->s) != hipSuccess || hipStreamWaitEvent(st, ss->join, 0) != hipSuccess))
        return set_error(HMOE_ERR_HIP, "moe4: join");
    if (phases & 8) dec_d_kernel<<<(R * H / 4 + 255) / 256, 256, 0, st>>>(a.y32, a.ctr, R, a.y, a.out);
    return HMOE_LAUNCHED("moe4");
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_moe4_scratch_bytes(int which)
{
    switch (which)
    {
        case 0: return (size_t) ACT_SLOTS * MAXR * I * 2;               // act f16 [132][16][2048]
        case 1: return 256;                                             // gu32 (unused: kept for the argument)
        case 2: return (size_t) CTR_WORDS * 4;                          // ctr_a: the part count
        case 3: return (size_t) MAX_PARTS * MAXR * H * 4;               // y32: down part partials
        case 4: return (size_t) CTR_WORDS * 4;                          // ctr_b (unused)
        default: return 0;
    }
}

static DecodeArgs forward_args(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                               const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                               const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s, void* act,
                               int* ctr_a, float* y32, float* y, int blocks, int lo, const void* sh_gw,
                               const void* sh_uw, const void* sh_dw, int xf)
{
    DecodeArgs a = {};
    a.x = x; a.xf = xf; a.sel_in = sel; a.rw_in = rw; a.R = R; a.n_hot = n_hot; a.lo = lo;
    a.gate_w = gate_w; a.up_w = up_w; a.down_w = down_w; a.gate_s = gate_s; a.up_s = up_s; a.down_s = down_s;
    a.act = (_Float16*) act; a.ctr = ctr_a; a.y32 = y32; a.y = y; a.out = nullptr;
    a.sh_gw = sh_gw; a.sh_uw = sh_uw; a.sh_dw = sh_dw; a.blocks = blocks;
    return a;
}

extern "C" int hmoe_moe4_gate_up(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                 const int64_t* gate_w, const int64_t* up_w, const int64_t* gate_s,
                                 const int64_t* up_s, void* act, float* gu32, int* ctr_a, int blocks, int lo,
                                 const void* sh_gw, const void* sh_uw, int xf, void* stream)
{
    (void) gu32;
    DecodeArgs a = forward_args(x, sel, rw, R, n_hot, gate_w, up_w, gate_w, gate_s, up_s, gate_s, act, ctr_a,
                                (float*) act, nullptr, blocks, lo, sh_gw, sh_uw, sh_gw, xf);
    int rc = check(a);
    if (rc) return rc;
    HMOE_REQUIRE(sel && rw, "moe4_gate_up: null selection");
    return run_decode(a, 3, (hipStream_t) stream);
}

extern "C" int hmoe_moe4_down(const int64_t* sel, const uint16_t* rw, int R, int n_hot, const int64_t* down_w,
                              const int64_t* down_s, const void* act, float* y32, int* ctr_b, float* y, int blocks,
                              int lo, const void* sh_dw, void* stream)
{
    // ctr_b holds the part count handed from the down launch to the reduction (ctr_a of forward)
    DecodeArgs a = forward_args(act, sel, rw, R, n_hot, down_w, down_w, down_w, down_s, down_s, down_s, (void*) act,
                                ctr_b, y32, y, blocks, lo, sh_dw, sh_dw, sh_dw, 1);
    int rc = check(a);
    if (rc) return rc;
    HMOE_REQUIRE(sel && rw && y, "moe4_down: null buffer");
    return run_decode(a, 12, (hipStream_t) stream);
}

extern "C" int hmoe_moe4_forward(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                 const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                                 const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s,
                                 void* act, float* gu32, int* ctr_a, float* y32, int* ctr_b, float* y, int blocks,
                                 int blocks_a, int lo, const void* sh_gw, const void* sh_uw, const void* sh_dw,
                                 const void* sh_gs, const void* sh_us, const void* sh_ds, int xf, void* stream)
{
    (void) blocks_a; (void) ctr_b; (void) gu32;
    HMOE_REQUIRE(!sh_gs && !sh_us && !sh_ds, "moe4_forward: shared-expert scales must be 0 (F16T has none)");
    DecodeArgs a = forward_args(x, sel, rw, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, ctr_a, y32, y,
                                blocks, lo, sh_gw, sh_uw, sh_dw, xf);
    int rc = check(a);
    if (rc) return rc;
    HMOE_REQUIRE(sel && rw && y, "moe4_forward: null buffer");
    return run_decode(a, 15, (hipStream_t) stream);
}

extern "C" int hmoe_moe_decode_layer(const void* x, const float* wt, const float* bias, int E, int topk, float scale,
                                     float* logits, int64_t* sel, uint16_t* rw, int R, int n_hot, int lo,
                                     const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                                     const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s,
                                     const void* sh_gw, const void* sh_uw, const void* sh_dw, void* act, float* gu32,
                                     int* ctr_a, float* y32, float* y, uint16_t* out, int blocks, int phases,
                                     void* stream)
{
    (void) gu32;
    HMOE_REQUIRE(wt && logits && sel && rw && E >= TOPK && E <= RMAXE && topk == TOPK, "decode_layer: router arguments");
    HMOE_REQUIRE(y || out, "decode_layer: no output");
    HMOE_REQUIRE(phases >= 1 && phases <= 15, "decode_layer: phases %d", phases);
    DecodeArgs a = forward_args(x, nullptr, nullptr, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, ctr_a,
                                y32, y, blocks, lo, sh_gw, sh_uw, sh_dw, 0);
    a.wt = wt; a.bias = bias; a.logits = logits; a.E = E; a.topk = topk; a.scale = scale; a.sel_out = sel;
    a.rw_out = rw; a.out = out;
    int rc = check(a);
    if (rc) return rc;
    return run_decode(a, phases, (hipStream_t) stream);
}
