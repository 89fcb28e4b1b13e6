// decode.hip - the decode MoE op (runtime/tier/moe4/moe4.cu:828-895 moe4_forward) for 1..16 rows on gfx950, and the
// whole decode layer (router + experts) in the same four launches.
//
// No workgroup waits for another inside a launch (on gfx950 an agent-scope fence writes back and invalidates L2):
// every cross-workgroup sum is split at a kernel boundary and done in a fixed order, so results are bit-reproducible.
//   A (prologue)  router logits of two experts per workgroup (when the layer's router is fused in), the shared
//                 expert's gate/up partials per (16-row block nb, k quarter), and the f16 copy of x.
//   B (gate/up)   every workgroup derives the step's routing (top-k from the logits, or the given sel / rw) and the
//                 distinct experts (moe4.cu:86-110), then takes items b, b + G, ...: (expert slot j, nb) runs gate
//                 and up over all of H with 8 waves on 8 k ranges. A wave streams I4G128 tiles (one 16-byte load per
//                 lane = 16 rows x 128 k), decodes them to exact f16 in registers, multiplies with the rows' f16
//                 input on the 16x16x32 MFMA (16 token columns) and scales each 128-k group's partial by its bf16
//                 group scale in fp32. The 8 partials are summed in wave order through LDS and
//                 act[j][r][n] = f16(silu(g) u w[j][r]) is written (moe4.cu:645-676). Items (nb) of the shared expert
//                 sum its four quarter partials in order and write its act slot (weight 1).
//   C (down)      items (nb of H, part): part 0 = the shared expert's down, parts 1.. = four routed slots each
//                 (moe4.cu:443-643 with g128 scales); each item's 8 wave partials are summed in order and stored.
//   D (reduce)    y[r] (+)= sum of the parts in part order (moe4.cu:826-827 accumulates into y), or the layer's bf16
//                 output.
#include "hmoe_dev.h"

namespace hmoe {

constexpr int NW = 8, NT = NW * 64;        // waves and threads per workgroup
constexpr int KG_H = H / 128;              // 48 k groups of gate / up
constexpr int KG_I = I / 128;              // 16 k groups of down
constexpr int NB_I = I / 16;               // 128 row blocks of gate / up
constexpr int NB_H = H / 16;               // 384 row blocks of down
constexpr int SH_Q = 4;                    // k quarters of a shared-expert gate/up item
constexpr int KS_H = H / 32;               // 192 F16T k steps of gate / up
constexpr int KS_I = I / 32;               // 64 F16T k steps of down
constexpr int ROUTED_PER_PART = 4;         // routed slots per down item
constexpr int MAX_PARTS = 1 + MAXSLOT / ROUTED_PER_PART;
constexpr int CTR_WORDS = 1024;            // ctr_a[0]: the parts of the last down launch

struct Route
{
    int m;
    unsigned mask[8];
    short e[MAXSLOT];
    float w[MAXSLOT][MAXR];
};

// distinct experts of the step (ascending local id) and routing weight per (slot, row): moe4.cu:86-110, with the slot of
// each pick from popcounts of the 256-bit mask. sel / rw may be in LDS or global memory.
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

// four bf16 group scales (rows 4(l/16)..+4 of a tile) -> fp32
__device__ __forceinline__ void scales4(u32x2 s, float* f)
{
    f[0] = __uint_as_float(s[0] << 16); f[1] = __uint_as_float(s[0] & 0xffff0000u);
    f[2] = __uint_as_float(s[1] << 16); f[3] = __uint_as_float(s[1] & 0xffff0000u);
}

// one routed I4G128 tile (16 rows x 128 k) times the B fragments of its 4 k steps -> scaled into acc
__device__ __forceinline__ void tile_i4(u32x4 wq, u32x2 sc, const f16x8* b, f32x4& acc)
{
    f32x4 p = {0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int t = 0; t < 4; ++t) p = mfma16(dq8(wq[t]), b[t], p);
    float s[4]; scales4(sc, s);
    #pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(s[i], p[i], acc[i]);
}

// 8 bf16 -> 8 f16 (the B operand of the shared expert when x arrives as bf16)
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

// the 8 wave partials of a 16-row block, summed in wave order: thread t < 256 gets (row t/16, token t%16)
__device__ __forceinline__ float wave_sum(const float (*red)[64][8], int comp)
{
    const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
    const int ll = (row >> 2) * 16 + tk, ie = row & 3;
    float s = 0.f;
    #pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w][ll][comp + ie];
    return s;
}

union SmemA
{
    float sums[2][256][MAXR + 1];
    float red[NW][64][8];
};

// ---- A: router logits (2 experts per workgroup), shared gate/up quarter partials, f16 copy of x ----
__global__ void __launch_bounds__(NT) dec_a_kernel(
    const void* __restrict__ x, int xf, _Float16* __restrict__ xh_out, int R, const float* __restrict__ wt, int E,
    float* __restrict__ logits, int n_router, const uint8_t* __restrict__ sh_gw, const uint8_t* __restrict__ sh_uw,
    float* __restrict__ gu32, int n_shared)
{
    __shared__ SmemA sm;
    const int b = blockIdx.x;
    if (b < n_router)
    {
        const int half = threadIdx.x >> 8, tid = threadIdx.x & 255;
        expert_logits((const uint16_t*) x, wt, 2 * b + half, E, R, H, tid, sm.sums[half], logits);
    }
    else if (b < n_router + n_shared)
    {
        const int item = b - n_router, nb = item / SH_Q, kq = item % SH_Q;
        const int w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, kslice = l >> 4;
        const bool live = tok < R;
        constexpr int KSW = KS_H / SH_Q / NW;                          // 6 k steps per wave
        const int ks0 = kq * (KS_H / SH_Q) + w * KSW;
        const size_t off = ((size_t) (nb * KS_H + ks0) * 64 + l) * 16;
        u32x4 wg[KSW], wu[KSW];
        #pragma unroll
        for (int i = 0; i < KSW; ++i)
        {
            wg[i] = ldw16(sh_gw + off + (size_t) i * 1024);
            wu[i] = ldw16(sh_uw + off + (size_t) i * 1024);
        }
        f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
        const size_t xo = (size_t) (live ? tok : 0) * H + 8 * kslice;
        #pragma unroll
        for (int i = 0; i < KSW; ++i)
        {
            f16x8 bv = {};
            if (live)
            {
                const size_t k = xo + (size_t) (ks0 + i) * 32;
                bv = xf ? as_f16x8(ld16((const _Float16*) x + k)) : bf8_to_f16(ld16((const uint16_t*) x + k));
            }
            ag = mfma16(as_f16x8(wg[i]), bv, ag);
            au = mfma16(as_f16x8(wu[i]), bv, au);
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i) { sm.red[w][l][i] = ag[i]; sm.red[w][l][4 + i] = au[i]; }
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
            if (tk < R)
            {
                const float g = wave_sum(sm.red, 0), u = wave_sum(sm.red, 4);
                const int n = nb * 16 + row;
                gu32[((size_t) (kq * 2 + 0) * MAXR + tk) * I + n] = g;
                gu32[((size_t) (kq * 2 + 1) * MAXR + tk) * I + n] = u;
            }
        }
    }
    // the f16 copy of x, spread over every workgroup
    if (xh_out)
    {
        const int n = R * H, per = (n + gridDim.x - 1) / gridDim.x, b0 = b * per;
        to_f16_range((const uint16_t*) x, xh_out, b0, min(n, b0 + per), threadIdx.x, blockDim.x);
    }
}

struct SmemB
{
    Route rt;
    float red[NW][64][8];
    int64_t sel[MAXR * TOPK];
    uint16_t rw[MAXR * TOPK];
};

// ---- B: routing, routed gate/up + act, shared act ----
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4)))
dec_b_kernel(const _Float16* __restrict__ xh, const float* __restrict__ logits, const float* __restrict__ bias, int E,
             int topk, float scale, int64_t* __restrict__ sel, uint16_t* __restrict__ rw, int R, int lo, int n_hot,
             const int64_t* __restrict__ gate_w, const int64_t* __restrict__ up_w,
             const int64_t* __restrict__ gate_s, const int64_t* __restrict__ up_s, int has_sh,
             const float* __restrict__ gu32, _Float16* __restrict__ act)
{
    __shared__ SmemB sm;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (logits)
    {
        // the router's selection (every workgroup derives the same one; workgroup 0 publishes it)
        for (int r = w; r < R; r += NW)
            select_row(logits + (size_t) r * RMAXE, bias, E, topk, scale, sm.sel + r * TOPK, sm.rw + r * TOPK);
        __syncthreads();
        if (blockIdx.x == 0 && threadIdx.x < R * TOPK) { sel[threadIdx.x] = sm.sel[threadIdx.x]; rw[threadIdx.x] = sm.rw[threadIdx.x]; }
        route(sm.sel, sm.rw, R, lo, n_hot, sm.rt);
    }
    else route(sel, rw, R, lo, n_hot, sm.rt);
    const int m = sm.rt.m;
    const int n_fin = has_sh ? NB_I : 0;
    const int total = n_fin + m * NB_I;
    const int tok = l & 15, kslice = l >> 4;
    const bool live = tok < R;
    const _Float16* xrow = xh + (size_t) (live ? tok : 0) * H + 8 * kslice;
    for (int item = blockIdx.x; item < total; item += gridDim.x)
    {
        if (item < n_fin)
        {
            // shared expert: sum the four quarter partials in order, act = silu(g) u
            const int nb = item;
            if (threadIdx.x < 256)
            {
                const int row = threadIdx.x >> 4, tk = threadIdx.x & 15, n = nb * 16 + row;
                if (tk < R)
                {
                    float g = 0.f, u = 0.f;
                    #pragma unroll
                    for (int q = 0; q < SH_Q; ++q)
                    {
                        g += gu32[((size_t) (q * 2 + 0) * MAXR + tk) * I + n];
                        u += gu32[((size_t) (q * 2 + 1) * MAXR + tk) * I + n];
                    }
                    act[((size_t) SH_SLOT * MAXR + tk) * I + n] = (_Float16) (silu(g) * u);
                }
            }
            continue;
        }
        const int u_ = item - n_fin, j = u_ / NB_I, nb = u_ % NB_I;
        const int e = sm.rt.e[j];
        constexpr int KGW = KG_H / NW;                                 // 6 k groups per wave
        const int kg0 = w * KGW;
        const uint8_t* gq = (const uint8_t*) gate_w[e];
        const uint8_t* uq = (const uint8_t*) up_w[e];
        const uint8_t* gs = (const uint8_t*) gate_s[e];
        const uint8_t* us = (const uint8_t*) up_s[e];
        const size_t toff = ((size_t) (nb * KG_H + kg0) * 64 + l) * 16;
        const size_t soff = ((size_t) (nb * KG_H + kg0) * 16 + 4 * kslice) * 2;
        u32x4 wg[KGW], wu[KGW]; u32x2 sg[KGW], su[KGW];
        #pragma unroll
        for (int i = 0; i < KGW; ++i)
        {
            wg[i] = ldw16(gq + toff + (size_t) i * 1024); wu[i] = ldw16(uq + toff + (size_t) i * 1024);
            sg[i] = *(const u32x2*) (gs + soff + (size_t) i * 32); su[i] = *(const u32x2*) (us + soff + (size_t) i * 32);
        }
        f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int i = 0; i < KGW; ++i)
        {
            f16x8 bv[4];
            #pragma unroll
            for (int t = 0; t < 4; ++t)
            {
                bv[t] = (f16x8) {};
                if (live) bv[t] = as_f16x8(ld16(xrow + (kg0 + i) * 128 + 32 * t));
            }
            tile_i4(wg[i], sg[i], bv, ag);
            tile_i4(wu[i], su[i], bv, au);
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i) { sm.red[w][l][i] = ag[i]; sm.red[w][l][4 + i] = au[i]; }
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
            if (tk < R)
            {
                const float g = wave_sum(sm.red, 0), uu = wave_sum(sm.red, 4);
                act[((size_t) j * MAXR + tk) * I + nb * 16 + row] = (_Float16) (silu(g) * uu * sm.rt.w[j][tk]);
            }
        }
        __syncthreads();
    }
}

struct SmemC
{
    Route rt;
    float red[NW][64][4];
};

// ---- C: down parts ----
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4)))
dec_c_kernel(const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw, int R, int lo, int n_hot,
             const int64_t* __restrict__ down_w, const int64_t* __restrict__ down_s, const uint8_t* __restrict__ sh_dw,
             const _Float16* __restrict__ act, float* __restrict__ y32, int* __restrict__ nparts_out)
{
    __shared__ SmemC sm;
    route(sel, rw, R, lo, n_hot, sm.rt);
    const int m = sm.rt.m;
    const int has_sh = sh_dw != nullptr ? 1 : 0;
    const int nparts = has_sh + (m + ROUTED_PER_PART - 1) / ROUTED_PER_PART;
    if (blockIdx.x == 0 && threadIdx.x == 0) *nparts_out = nparts;
    const int total = nparts * NB_H;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int tok = l & 15, kslice = l >> 4;
    const bool live = tok < R;
    for (int item = blockIdx.x; item < total; item += gridDim.x)
    {
        const int nb = item % NB_H, part = item / NB_H;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (has_sh && part == 0)
        {
            constexpr int KSW = KS_I / NW;                              // 8 k steps per wave
            const int ks0 = w * KSW;
            const size_t off = ((size_t) (nb * KS_I + ks0) * 64 + l) * 16;
            const _Float16* arow = act + ((size_t) SH_SLOT * MAXR + (live ? tok : 0)) * I + 8 * kslice;
            u32x4 wd[KSW];
            #pragma unroll
            for (int i = 0; i < KSW; ++i) wd[i] = ldw16(sh_dw + off + (size_t) i * 1024);
            #pragma unroll
            for (int i = 0; i < KSW; ++i)
            {
                f16x8 bv = {};
                if (live) bv = as_f16x8(ld16(arow + (ks0 + i) * 32));
                acc = mfma16(as_f16x8(wd[i]), bv, acc);
            }
        }
        else
        {
            const int j = (part - has_sh) * ROUTED_PER_PART + (w >> 1);
            if (j < m)
            {
                const int e = sm.rt.e[j];
                constexpr int KGW = KG_I / 2;                           // 8 k groups per wave (two waves per slot)
                const int kg0 = (w & 1) * KGW;
                const uint8_t* dq = (const uint8_t*) down_w[e];
                const uint8_t* ds = (const uint8_t*) down_s[e];
                const size_t toff = ((size_t) (nb * KG_I + kg0) * 64 + l) * 16;
                const size_t soff = ((size_t) (nb * KG_I + kg0) * 16 + 4 * kslice) * 2;
                const _Float16* arow = act + ((size_t) j * MAXR + (live ? tok : 0)) * I + 8 * kslice;
                u32x4 wd[KGW]; u32x2 sd[KGW];
                #pragma unroll
                for (int i = 0; i < KGW; ++i)
                {
                    wd[i] = ldw16(dq + toff + (size_t) i * 1024);
                    sd[i] = *(const u32x2*) (ds + soff + (size_t) i * 32);
                }
                #pragma unroll
                for (int i = 0; i < KGW; ++i)
                {
                    f16x8 bv[4];
                    #pragma unroll
                    for (int t = 0; t < 4; ++t)
                    {
                        bv[t] = (f16x8) {};
                        if (live) bv[t] = as_f16x8(ld16(arow + (kg0 + i) * 128 + 32 * t));
                    }
                    tile_i4(wd[i], sd[i], bv, acc);
                }
            }
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i) sm.red[w][l][i] = acc[i];
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
            const int ll = (row >> 2) * 16 + tk, ie = row & 3;
            if (tk < R)
            {
                float s = 0.f;
                #pragma unroll
                for (int ww = 0; ww < NW; ++ww) s += sm.red[ww][ll][ie];
                y32[((size_t) part * MAXR + tk) * H + nb * 16 + row] = s;
            }
        }
        __syncthreads();
    }
}

// ---- D: y (+)= sum of the parts in order; or the layer's bf16 output ----
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
    _Float16* act; float* gu32; int* ctr; float* y32; float* y; uint16_t* out;
    const void *sh_gw, *sh_uw, *sh_dw;
    const float* wt; const float* bias; float* logits; int E; int topk; float scale; int64_t* sel_out; uint16_t* rw_out;
    int blocks;
};

static int check(const DecodeArgs& a)
{
    HMOE_REQUIRE(a.R >= 1 && a.R <= MAXR, "moe4: rows %d not in [1, %d]", a.R, MAXR);
    HMOE_REQUIRE(a.n_hot >= 0 && a.n_hot <= HMOE_MAXE && a.lo >= 0, "moe4: window lo %d n_hot %d", a.lo, a.n_hot);
    HMOE_REQUIRE(a.x && a.act && a.gu32 && a.ctr && a.y32, "moe4: null buffer");
    HMOE_REQUIRE(a.n_hot == 0 || (a.gate_w && a.up_w && a.down_w && a.gate_s && a.up_s && a.down_s), "moe4: null table");
    HMOE_REQUIRE((!a.sh_gw && !a.sh_uw && !a.sh_dw) || (a.sh_gw && a.sh_uw && a.sh_dw), "moe4: partial shared expert");
    HMOE_REQUIRE(((uintptr_t) a.x & 15) == 0 && ((uintptr_t) a.act & 15) == 0, "moe4: x / act not 16-byte aligned");
    HMOE_REQUIRE(a.blocks >= 0, "moe4: blocks %d", a.blocks);
    return HMOE_OK;
}

// launches A..D; phase mask bit 0 = A, 1 = B, 2 = C, 3 = D
static int run_decode(const DecodeArgs& a, int phases, hipStream_t st)
{
    const int R = a.R;
    _Float16* xc = a.act + (size_t) (SH_SLOT + 1) * MAXR * I;      // f16 copy of x (when x arrives as bf16)
    const _Float16* xh = a.xf ? (const _Float16*) a.x : xc;
    const int G = a.blocks > 0 ? a.blocks : default_grid(2);
    if (phases & 1)
    {
        const int n_router = a.logits ? (a.E + 1) / 2 : 0;
        const int n_shared = a.sh_gw ? NB_I * SH_Q : 0;
        int ga = n_router + n_shared;
        if (!a.xf && ga < 16) ga = 16;                              // workgroups for the f16 copy of x
        if (ga > 0)
            dec_a_kernel<<<ga, NT, 0, st>>>(a.x, a.xf, a.xf ? nullptr : xc, R, a.wt, a.E, a.logits, n_router,
                                            (const uint8_t*) a.sh_gw, (const uint8_t*) a.sh_uw, a.gu32, n_shared);
    }
    if (phases & 2)
        dec_b_kernel<<<G, NT, 0, st>>>(xh, a.logits, a.bias, a.E, a.topk, a.scale, a.logits ? a.sel_out : (int64_t*) a.sel_in,
                                       a.logits ? a.rw_out : (uint16_t*) a.rw_in, R, a.lo, a.n_hot, a.gate_w, a.up_w,
                                       a.gate_s, a.up_s, a.sh_gw ? 1 : 0, a.gu32, a.act);
    const int64_t* sel = a.logits ? a.sel_out : a.sel_in;
    const uint16_t* rw = a.logits ? a.rw_out : a.rw_in;
    if (phases & 4)
        dec_c_kernel<<<G, NT, 0, st>>>(sel, rw, R, a.lo, a.n_hot, a.down_w, a.down_s, (const uint8_t*) a.sh_dw, a.act,
                                       a.y32, a.ctr);
    if (phases & 8) dec_d_kernel<<<(R * H / 4 + 255) / 256, 256, 0, st>>>(a.y32, a.ctr, R, a.y, a.out);
    return HMOE_LAUNCHED("moe4");
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_moe4_scratch_bytes(int which)
{
    switch (which)
    {
        case 0: return (size_t) ACT_SLOTS * MAXR * I * 2;               // act f16 [132][16][2048] (+ x copy)
        case 1: return (size_t) SH_Q * 2 * MAXR * I * 4;                // gu32: shared gate/up quarter partials
        case 2: return (size_t) CTR_WORDS * 4;                          // ctr_a
        case 3: return (size_t) MAX_PARTS * MAXR * H * 4;               // y32: down part partials
        case 4: return (size_t) CTR_WORDS * 4;                          // ctr_b (unused)
        default: return 0;
    }
}

static DecodeArgs forward_args(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                               const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                               const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s, void* act,
                               float* gu32, int* ctr_a, float* y32, float* y, int blocks, int lo, const void* sh_gw,
                               const void* sh_uw, const void* sh_dw, int xf)
{
    DecodeArgs a = {};
    a.x = x; a.xf = xf; a.sel_in = sel; a.rw_in = rw; a.R = R; a.n_hot = n_hot; a.lo = lo;
    a.gate_w = gate_w; a.up_w = up_w; a.down_w = down_w; a.gate_s = gate_s; a.up_s = up_s; a.down_s = down_s;
    a.act = (_Float16*) act; a.gu32 = gu32; a.ctr = ctr_a; a.y32 = y32; a.y = y; a.out = nullptr;
    a.sh_gw = sh_gw; a.sh_uw = sh_uw; a.sh_dw = sh_dw; a.blocks = blocks;
    return a;
}

extern "C" int hmoe_moe4_gate_up(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                 const int64_t* gate_w, const int64_t* up_w, const int64_t* gate_s,
                                 const int64_t* up_s, void* act, float* gu32, int* ctr_a, int blocks, int lo,
                                 const void* sh_gw, const void* sh_uw, int xf, void* stream)
{
    DecodeArgs a = forward_args(x, sel, rw, R, n_hot, gate_w, up_w, gate_w, gate_s, up_s, gate_s, act, gu32, ctr_a,
                                gu32, nullptr, blocks, lo, sh_gw, sh_uw, sh_gw, xf);
    int rc = check(a);
    if (rc) return rc;
    HMOE_REQUIRE(sel && rw, "moe4_gate_up: null selection");
    return run_decode(a, 3, (hipStream_t) stream);
}

extern "C" int hmoe_moe4_down(const int64_t* sel, const uint16_t* rw, int R, int n_hot, const int64_t* down_w,
                              const int64_t* down_s, const void* act, float* y32, int* ctr_b, float* y, int blocks,
                              int lo, const void* sh_dw, void* stream)
{
    // ctr_b holds the part count handed from C to D (ctr_a of forward)
    DecodeArgs a = forward_args(act, sel, rw, R, n_hot, down_w, down_w, down_w, down_s, down_s, down_s, (void*) act,
                                y32, ctr_b, y32, y, blocks, lo, sh_dw, sh_dw, sh_dw, 1);
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
    (void) blocks_a; (void) ctr_b;
    HMOE_REQUIRE(!sh_gs && !sh_us && !sh_ds, "moe4_forward: shared-expert scales must be 0 (F16T has none)");
    DecodeArgs a = forward_args(x, sel, rw, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, gu32, ctr_a, y32,
                                y, blocks, lo, sh_gw, sh_uw, sh_dw, xf);
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
    HMOE_REQUIRE(wt && logits && sel && rw && E >= TOPK && E <= RMAXE && topk == TOPK, "decode_layer: router arguments");
    HMOE_REQUIRE(y || out, "decode_layer: no output");
    HMOE_REQUIRE(phases >= 1 && phases <= 15, "decode_layer: phases %d", phases);
    DecodeArgs a = forward_args(x, nullptr, nullptr, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, gu32,
                                ctr_a, y32, y, blocks, lo, sh_gw, sh_uw, sh_dw, 0);
    a.wt = wt; a.bias = bias; a.logits = logits; a.E = E; a.topk = topk; a.scale = scale; a.sel_out = sel;
    a.rw_out = rw; a.out = out;
    int rc = check(a);
    if (rc) return rc;
    return run_decode(a, phases, (hipStream_t) stream);
}
