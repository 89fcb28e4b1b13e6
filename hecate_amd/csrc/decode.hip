// decode.hip - the decode MoE op (runtime/tier/moe4/moe4.cu:828-895 moe4_forward) for 1..16 rows on gfx950.
//
// Two persistent kernels over a dynamic work queue (an atomic item counter that the last workgroup to leave resets,
// so the launch shape is static and the scratch self-cleaning, as moe4.cu:14-19):
//   gu   : items (expert slot j, 16-row block nb of I) run gate and up over all of H: 8 waves split H into 8 k ranges,
//          each wave streams its I4G128 tiles (one 16-byte load per lane = 16 rows x 128 k), decodes them to exact f16
//          in registers and multiplies with the rows' f16 input on the 16x16x32 MFMA (rows = the 16 token columns);
//          each 128-k group's partial sum is scaled by its bf16 group scale in fp32. The 8 partials are summed in wave
//          order through LDS and act[j][r][n] = f16(silu(g) * u * w[j][r]) is written (moe4.cu:645-676).
//          The shared expert (F16T) runs as items (nb, k quarter) of the same size; the last quarter to arrive sums
//          the four partials in order and writes its act slot (weight 1).
//   down : items (16-row block nb of H, part): part 0 the shared expert's down over its act slot, parts 1.. four
//          routed slots each (moe4.cu:443-643 with the row scale replaced by g128 scales); parts of one nb are summed
//          in part order by the last to arrive and added into y (fp32, accumulated into, moe4.cu:826-827).
// Every sum has a fixed order, so results are bit-reproducible run to run.
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
// counters: ctr_a [0, 128) shared arrivals per nb, [256, 258) queue; ctr_b [0, 384) arrivals per nb, [512, 514) queue
constexpr int CTR_WORDS = 1024;

struct Route
{
    int m;
    unsigned mask[8];
    short e[MAXSLOT];
    float w[MAXSLOT][MAXR];
};

// distinct experts of the step (ascending local id), routing weight per (slot, row): moe4.cu:86-110, with the slot of
// each pick computed from popcounts of the 256-bit mask instead of a serial scan
__device__ void route(const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw, int R, int lo, int n_hot,
                      Route& rt)
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

__device__ __forceinline__ int next_item(int* q, int* s_item)
{
    __syncthreads();
    if (threadIdx.x == 0) *s_item = atomicAdd(q, 1);
    __syncthreads();
    return *s_item;
}

// the last workgroup to leave resets the queue for the next launch
__device__ __forceinline__ void leave_queue(int* q)
{
    if (threadIdx.x == 0)
    {
        __threadfence();
        if (atomicAdd(q + 1, 1) == (int) gridDim.x - 1)
        {
            __hip_atomic_store(q, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(q + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__device__ __forceinline__ float ld_coherent(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

__global__ void __launch_bounds__(NT) gu_kernel(
    const _Float16* __restrict__ xh, const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw, int R, int lo,
    int n_hot, const int64_t* __restrict__ gate_w, const int64_t* __restrict__ up_w,
    const int64_t* __restrict__ gate_s, const int64_t* __restrict__ up_s, const uint8_t* __restrict__ sh_gw,
    const uint8_t* __restrict__ sh_uw, _Float16* __restrict__ act, float* __restrict__ gu32, int* __restrict__ ctr)
{
    __shared__ Route rt;
    __shared__ float red[NW][64][8];
    __shared__ int s_item, s_last;
    route(sel, rw, R, lo, n_hot, rt);
    const int m = rt.m;
    const bool has_sh = sh_gw != nullptr;
    const int n_sh = has_sh ? NB_I * SH_Q : 0;
    const int total = n_sh + m * NB_I;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int tok = l & 15, kslice = l >> 4;
    const bool live = tok < R;
    const _Float16* xrow = xh + (size_t) (live ? tok : 0) * H + 8 * kslice;
    const f16x8 zero8 = {};
    int* q = ctr + 256;
    for (;;)
    {
        const int item = next_item(q, &s_item);
        if (item >= total) break;
        f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
        int nb, j = -1, kq = 0;
        if (item < n_sh)
        {
            nb = item / SH_Q; kq = item % SH_Q;
            constexpr int KSW = KS_H / SH_Q / NW;                      // 6 k steps per wave
            const int ks0 = kq * (KS_H / SH_Q) + w * KSW;
            const size_t off = ((size_t) (nb * KS_H + ks0) * 64 + l) * 16;
            u32x4 wg[KSW], wu[KSW];
            #pragma unroll
            for (int i = 0; i < KSW; ++i) { wg[i] = ldw16(sh_gw + off + (size_t) i * 1024); wu[i] = ldw16(sh_uw + off + (size_t) i * 1024); }
            #pragma unroll
            for (int i = 0; i < KSW; ++i)
            {
                const f16x8 b = live ? as_f16x8(ld16(xrow + (ks0 + i) * 32)) : zero8;
                ag = mfma16(as_f16x8(wg[i]), b, ag);
                au = mfma16(as_f16x8(wu[i]), b, au);
            }
        }
        else
        {
            const int u = item - n_sh;
            j = u / NB_I; nb = u % NB_I;
            const int e = rt.e[j];
            constexpr int KGW = KG_H / NW;                             // 6 k groups per wave
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
            #pragma unroll
            for (int i = 0; i < KGW; ++i)
            {
                f16x8 b[4];
                #pragma unroll
                for (int t = 0; t < 4; ++t) b[t] = live ? as_f16x8(ld16(xrow + (kg0 + i) * 128 + 32 * t)) : zero8;
                tile_i4(wg[i], sg[i], b, ag);
                tile_i4(wu[i], su[i], b, au);
            }
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i) { red[w][l][i] = ag[i]; red[w][l][4 + i] = au[i]; }
        __syncthreads();
        const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;       // output (row of the block, token) for t < 256
        const int ll = (row >> 2) * 16 + tk, ie = row & 3;
        float g = 0.f, uu = 0.f;
        if (threadIdx.x < 256)
        {
            #pragma unroll
            for (int ww = 0; ww < NW; ++ww) { g += red[ww][ll][ie]; uu += red[ww][ll][4 + ie]; }
        }
        const int n = nb * 16 + row;
        if (j >= 0)
        {
            if (threadIdx.x < 256 && tk < R)
                act[((size_t) j * MAXR + tk) * I + n] = (_Float16) (silu(g) * uu * rt.w[j][tk]);
        }
        else
        {
            // shared expert: publish this quarter's partial; the last quarter of nb sums the four in order
            if (threadIdx.x < 256 && tk < R)
            {
                gu32[((size_t) (kq * 2 + 0) * MAXR + tk) * I + n] = g;
                gu32[((size_t) (kq * 2 + 1) * MAXR + tk) * I + n] = uu;
            }
            __threadfence();
            __syncthreads();
            if (threadIdx.x == 0) s_last = atomicAdd(ctr + nb, 1) == SH_Q - 1;
            __syncthreads();
            if (s_last)
            {
                __threadfence();
                if (threadIdx.x < 256 && tk < R)
                {
                    float gs_ = 0.f, us_ = 0.f;
                    #pragma unroll
                    for (int k = 0; k < SH_Q; ++k)
                    {
                        gs_ += ld_coherent(gu32 + ((size_t) (k * 2 + 0) * MAXR + tk) * I + n);
                        us_ += ld_coherent(gu32 + ((size_t) (k * 2 + 1) * MAXR + tk) * I + n);
                    }
                    act[((size_t) SH_SLOT * MAXR + tk) * I + n] = (_Float16) (silu(gs_) * us_);
                }
                if (threadIdx.x == 0) __hip_atomic_store(ctr + nb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    leave_queue(q);
}

__global__ void __launch_bounds__(NT) down_kernel(
    const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw, int R, int lo, int n_hot,
    const int64_t* __restrict__ down_w, const int64_t* __restrict__ down_s, const uint8_t* __restrict__ sh_dw,
    const _Float16* __restrict__ act, float* __restrict__ y, float* __restrict__ y32, int* __restrict__ ctr)
{
    __shared__ Route rt;
    __shared__ float red[NW][64][4];
    __shared__ int s_item, s_last;
    route(sel, rw, R, lo, n_hot, rt);
    const int m = rt.m;
    const int has_sh = sh_dw != nullptr ? 1 : 0;
    const int nparts = has_sh + (m + ROUTED_PER_PART - 1) / ROUTED_PER_PART;
    const int total = nparts * NB_H;
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int tok = l & 15, kslice = l >> 4;
    const bool live = tok < R;
    const f16x8 zero8 = {};
    int* q = ctr + 512;
    for (;;)
    {
        const int item = next_item(q, &s_item);
        if (item >= total) break;
        const int nb = item / nparts, part = item % nparts;
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
                const f16x8 b = live ? as_f16x8(ld16(arow + (ks0 + i) * 32)) : zero8;
                acc = mfma16(as_f16x8(wd[i]), b, acc);
            }
        }
        else
        {
            const int j = (part - has_sh) * ROUTED_PER_PART + (w >> 1);
            if (j < m)
            {
                const int e = rt.e[j];
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
                    f16x8 b[4];
                    #pragma unroll
                    for (int t = 0; t < 4; ++t) b[t] = live ? as_f16x8(ld16(arow + (kg0 + i) * 128 + 32 * t)) : zero8;
                    tile_i4(wd[i], sd[i], b, acc);
                }
            }
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i) red[w][l][i] = acc[i];
        __syncthreads();
        const int row = threadIdx.x >> 4, tk = threadIdx.x & 15;
        const int ll = (row >> 2) * 16 + tk, ie = row & 3;
        float tot = 0.f;
        if (threadIdx.x < 256)
        {
            #pragma unroll
            for (int ww = 0; ww < NW; ++ww) tot += red[ww][ll][ie];
        }
        const int n = nb * 16 + row;
        if (nparts == 1)
        {
            if (threadIdx.x < 256 && tk < R) y[(size_t) tk * H + n] += tot;
        }
        else
        {
            if (threadIdx.x < 256 && tk < R) y32[((size_t) part * MAXR + tk) * H + n] = tot;
            __threadfence();
            __syncthreads();
            if (threadIdx.x == 0) s_last = atomicAdd(ctr + nb, 1) == nparts - 1;
            __syncthreads();
            if (s_last)
            {
                __threadfence();
                if (threadIdx.x < 256 && tk < R)
                {
                    float s = 0.f;
                    for (int p = 0; p < nparts; ++p) s += ld_coherent(y32 + ((size_t) p * MAXR + tk) * H + n);
                    y[(size_t) tk * H + n] += s;
                }
                if (threadIdx.x == 0) __hip_atomic_store(ctr + nb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    leave_queue(q);
}

// x bf16 [R][H] -> f16 copy (the decode kernels' B operand)
__global__ void to_f16_kernel(const uint16_t* __restrict__ x, _Float16* __restrict__ xh, int n)
{
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i >= n) return;
    const u32x4 v = *(const u32x4*) (x + i);
    f16x8 o;
    #pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        o[2 * k] = (_Float16) __uint_as_float(v[k] << 16);
        o[2 * k + 1] = (_Float16) __uint_as_float(v[k] & 0xffff0000u);
    }
    *(f16x8*) (xh + i) = o;
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
        case 4: return (size_t) CTR_WORDS * 4;                          // ctr_b
        default: return 0;
    }
}

static int check_forward(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot, int lo,
                         const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w, const int64_t* gate_s,
                         const int64_t* up_s, const int64_t* down_s, const void* act, const void* sh_gw,
                         const void* sh_uw, const void* sh_dw, int blocks)
{
    HMOE_REQUIRE(R >= 1 && R <= MAXR, "moe4: rows %d not in [1, %d]", R, MAXR);
    HMOE_REQUIRE(n_hot >= 0 && n_hot <= HMOE_MAXE && lo >= 0, "moe4: window lo %d n_hot %d", lo, n_hot);
    HMOE_REQUIRE(x && sel && rw && act, "moe4: null buffer");
    HMOE_REQUIRE(n_hot == 0 || (gate_w && up_w && down_w && gate_s && up_s && down_s), "moe4: null table");
    HMOE_REQUIRE((!sh_gw && !sh_uw && !sh_dw) || (sh_gw && sh_uw && sh_dw), "moe4: partial shared expert");
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) act & 15) == 0, "moe4: x / act not 16-byte aligned");
    HMOE_REQUIRE(blocks >= 0, "moe4: blocks %d", blocks);
    return HMOE_OK;
}

// phase 1 of moe4_forward: (x -> f16 copy unless xf) + gate / up / act of the routed experts and the shared expert
extern "C" int hmoe_moe4_gate_up(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                 const int64_t* gate_w, const int64_t* up_w, const int64_t* gate_s,
                                 const int64_t* up_s, void* act, float* gu32, int* ctr_a, int blocks, int lo,
                                 const void* sh_gw, const void* sh_uw, int xf, void* stream)
{
    int rc = check_forward(x, sel, rw, R, n_hot, lo, gate_w, up_w, gate_w, gate_s, up_s, gate_s, act, sh_gw, sh_uw,
                           sh_gw, blocks);
    if (rc) return rc;
    HMOE_REQUIRE(gu32 && ctr_a, "moe4_gate_up: null scratch");
    hipStream_t st = (hipStream_t) stream;
    _Float16* a = (_Float16*) act;
    const _Float16* xh = (const _Float16*) x;
    if (!xf)
    {
        _Float16* xc = a + (size_t) (SH_SLOT + 1) * MAXR * I;
        const int n = R * H;
        to_f16_kernel<<<(n / 8 + 255) / 256, 256, 0, st>>>((const uint16_t*) x, xc, n);
        xh = xc;
    }
    const int grid = blocks > 0 ? blocks : default_grid(2);
    gu_kernel<<<grid, NT, 0, st>>>(xh, sel, rw, R, lo, n_hot, gate_w, up_w, gate_s, up_s, (const uint8_t*) sh_gw,
                                   (const uint8_t*) sh_uw, a, gu32, ctr_a);
    return HMOE_LAUNCHED("moe4_gate_up");
}

// phase 2 of moe4_forward: down projections of the routed experts and the shared expert, added into y
extern "C" int hmoe_moe4_down(const int64_t* sel, const uint16_t* rw, int R, int n_hot, const int64_t* down_w,
                              const int64_t* down_s, const void* act, float* y32, int* ctr_b, float* y, int blocks,
                              int lo, const void* sh_dw, void* stream)
{
    int rc = check_forward(act, sel, rw, R, n_hot, lo, down_w, down_w, down_w, down_s, down_s, down_s, act, sh_dw,
                           sh_dw, sh_dw, blocks);
    if (rc) return rc;
    HMOE_REQUIRE(y32 && ctr_b && y, "moe4_down: null buffer");
    const int grid = blocks > 0 ? blocks : default_grid(2);
    down_kernel<<<grid, NT, 0, (hipStream_t) stream>>>(sel, rw, R, lo, n_hot, down_w, down_s, (const uint8_t*) sh_dw,
                                                       (const _Float16*) act, y, y32, ctr_b);
    return HMOE_LAUNCHED("moe4_down");
}

extern "C" int hmoe_moe4_forward(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                 const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                                 const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s,
                                 void* act, float* gu32, int* ctr_a, float* y32, int* ctr_b, float* y, int blocks,
                                 int blocks_a, int lo, const void* sh_gw, const void* sh_uw, const void* sh_dw,
                                 const void* sh_gs, const void* sh_us, const void* sh_ds, int xf, void* stream)
{
    (void) blocks_a;
    HMOE_REQUIRE(!sh_gs && !sh_us && !sh_ds, "moe4_forward: shared-expert scales must be 0 (F16T has none)");
    int rc = check_forward(x, sel, rw, R, n_hot, lo, gate_w, up_w, down_w, gate_s, up_s, down_s, act, sh_gw, sh_uw,
                           sh_dw, blocks);
    if (rc) return rc;
    rc = hmoe_moe4_gate_up(x, sel, rw, R, n_hot, gate_w, up_w, gate_s, up_s, act, gu32, ctr_a, blocks, lo, sh_gw,
                           sh_uw, xf, stream);
    if (rc) return rc;
    return hmoe_moe4_down(sel, rw, R, n_hot, down_w, down_s, act, y32, ctr_b, y, blocks, lo, sh_dw, stream);
}
