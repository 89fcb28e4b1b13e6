// decode.hip - the decode MoE op (runtime/tier/moe4/moe4.cu:828-895 moe4_forward) for 1..16 rows on gfx950, and the
// whole decode layer (router + experts) in the same launches.
//
// Design rules, from measurement on MI355X:
//   * the only vector-memory loads in a streaming loop are the 1 KB weight tiles (one 16-byte load per lane); group
//     scales come 4 k groups per load, and the activations stay in registers for the whole kernel: every extra vector
//     load per tile (a scale, an activation fragment from L2) costs 15-30 % of the achieved HBM bandwidth;
//   * the expert pointer tables go to LDS at kernel start, so the routing prologue ends in LDS reads;
//   * loads are unconditional and double-buffered per item (ping-pong between two register sets), so every wait
//     counts exactly and the next item's tiles are in flight across the item's reduction barrier;
//   * no workgroup waits for another inside a launch (on gfx950 an agent-scope fence writes back and invalidates
//     L2): cross-workgroup sums are cut at a kernel boundary and done in a fixed order (bit-reproducible results).
//
// MFMA roles: the token rows are the A operand (16 x 32 per k step, 16 tokens), the dequantised weight tile the B
// operand (32 k x 16 weight rows), so a lane's outputs share one weight row n = l % 16 and one group scale:
// lane l holds D[tokens 4(l/16)..+4][row l%16].
//
// Launches (on the caller's stream):
//   router   logits of two experts per workgroup (fixed fp32 order, see hecate_moe.h)
//   gate/up  256 workgroups; each first sums one matrix (gate or up) of one 16-row block of the shared expert over
//            the full K (its loads go out before the routing prologue and cover it; fp32 sums into act), then
//            derives the step's routing (top-k from the logits, or the given sel / rw) and the distinct experts
//            (moe4.cu:86-110), which workgroup 0 records in act for the down launch (slot count, local expert of
//            each slot), and takes routed items (slot, 16-row block nb) b, b + G, ...; 12 waves each own 4 k
//            groups of H with the rows' x in registers; the 12 wave partials are summed in wave order through LDS
//            and act[slot][r][n] = f16(silu(g) u w) is written (moe4.cu:645-676)
//   down     first the shared expert's 16-row blocks of H (part 0, its act formed from the fp32 sums; their loads
//            cover the read of the routing record), then routed items (slot quad, 16-row block of H), contiguous per
//            workgroup; 16 waves = 4 slots x 4 k quarters of I with the slots' act in registers; the 16 partials
//            are summed in order into y32[part] (moe4.cu:443-643)
//   reduce   y[r] (+)= sum of the parts in order (moe4.cu:826-827 accumulates into y), or the layer's bf16 output
#include "hmoe_dev.h"

#include <atomic>
#include <mutex>

namespace hmoe {

constexpr int NW = 8, NT = NW * 64;        // router workgroup
constexpr int KG_H = H / 128;              // 48 k groups of gate / up
constexpr int KG_I = I / 128;              // 16 k groups of down
constexpr int NB_I = I / 16;               // 128 row blocks of gate / up
constexpr int NB_H = H / 16;               // 384 row blocks of down
constexpr int KS_H = H / 32;               // 192 F16T k steps of gate / up
constexpr int KS_I = I / 32;               // 64 F16T k steps of down
constexpr int GW = 12;                     // gate/up waves: wave w owns k groups [4w, 4w + 4) of H
constexpr int DW = 16;                     // down waves: slot w / 4 of the quad, k groups [4 (w % 4), +4) of I
constexpr int CTR_WORDS = 1024;            // ctr[0]: the part count of the last down launch

struct __attribute__((aligned(16))) Route
{
    float w[MAXSLOT][MAXR];
    int m;
    unsigned mask[8];
    short e[MAXSLOT];
};

// one pick (expert id, f16 routing weight) of the step
struct Pick { int64_t s; uint16_t w; };

// distinct experts of the step (ascending local id) and routing weight per (slot, row): moe4.cu:86-110, with the slot
// of each pick from popcounts of the 256-bit mask. Ends with a barrier.
__device__ void route_picks(Pick pk, int R, int lo, int n_hot, Route& rt)
{
    const int t = threadIdx.x, np = R * TOPK;
    if (t < 8) rt.mask[t] = 0u;
    for (int i = t; i < MAXSLOT * MAXR; i += blockDim.x) (&rt.w[0][0])[i] = 0.f;
    int e = -1; float wv = 0.f;
    if (t < np)
    {
        const int64_t s = pk.s - lo;
        if (s >= 0 && s < n_hot) { e = (int) s; wv = (float) __builtin_bit_cast(_Float16, pk.w); }
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

// lanes of one wave exchanging data through LDS: the stores before are done before the loads after. LDS operations of
// one wave take effect in issue order; this keeps the compiler from moving a lane's load above another lane's store
// (which a lane's own program order does not forbid).
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// route_picks() for a selection in LDS (sel / rw, R rows of TOPK), done by wave 0 alone (it returns at once in the other
// waves) and with no workgroup barrier: its phases (zeroing, ors, reads, results) are separated by wave_lds_sync(). Within one row the picks are distinct experts, so every (slot, row)
// weight has at most one pick and is stored, not added. The caller's next barrier publishes rt.
__device__ void route_wave(const int64_t* sel, const uint16_t* rw, int R, int lo, int n_hot, Route& rt)
{
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x, np = R * TOPK;
    if (lane < 8) rt.mask[lane] = 0u;
    #pragma unroll
    for (int i = 0; i < MAXSLOT * MAXR / 256; ++i)
        *(f32x4*) &(&rt.w[0][0])[(i * 64 + lane) * 4] = (f32x4) {0.f, 0.f, 0.f, 0.f};
    wave_lds_sync();
    int e[2];
    float wv[2];
    #pragma unroll
    for (int h = 0; h < 2; ++h)
    {
        const int p = lane + 64 * h;
        e[h] = -1; wv[h] = 0.f;
        if (p < np)
        {
            const int64_t s = sel[p] - lo;
            if (s >= 0 && s < n_hot) { e[h] = (int) s; wv[h] = (float) __builtin_bit_cast(_Float16, rw[p]); }
        }
        if (e[h] >= 0) atomicOr(&rt.mask[e[h] >> 5], 1u << (e[h] & 31));
    }
    wave_lds_sync();
    unsigned mk[8];
    #pragma unroll
    for (int wd = 0; wd < 8; ++wd) mk[wd] = rt.mask[wd];
    #pragma unroll
    for (int h = 0; h < 2; ++h)
        if (e[h] >= 0)
        {
            int slot = __popc(mk[e[h] >> 5] & ((1u << (e[h] & 31)) - 1u));
            #pragma unroll
            for (int wd = 0; wd < 8; ++wd) slot += wd < (e[h] >> 5) ? __popc(mk[wd]) : 0;
            rt.e[slot] = (short) e[h];
            rt.w[slot][(lane + 64 * h) / TOPK] = wv[h];
        }
    if (lane == 0) { int m = 0; for (int wd = 0; wd < 8; ++wd) m += __popc(mk[wd]); rt.m = m; }
    wave_lds_sync();
}

// route() from sel / rw in LDS or global memory (generic loads)
__device__ void route(const int64_t* sel, const uint16_t* rw, int R, int lo, int n_hot, Route& rt)
{
    const int i = min((int) threadIdx.x, R * TOPK - 1);
    route_picks({sel[i], rw[i]}, R, lo, n_hot, rt);
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

// ---- router logits: one expert per 256-thread workgroup (pair_logits), so the 6.3 MB of weight rows spread over
// every CU (two per workgroup halve the x staging but leave half the CUs idle) ----
__global__ void __launch_bounds__(256) router_kernel(const uint16_t* __restrict__ x, int R, const float* __restrict__ wt,
                                                     int E, float* __restrict__ logits)
{
    pair_logits<false, 1>(x, NormIn{}, wt, blockIdx.x, E, R, logits);
}

// ---- RMSNorm of the residual + router logits (nr4_kernel.cuh:122-381), the same workgroups ----
__global__ void __launch_bounds__(NT) norm_router_kernel(NormIn nin, int R, const float* __restrict__ wt, int E,
                                                         float* __restrict__ logits)
{
    pair_logits<true>(nullptr, nin, wt, 2 * blockIdx.x, E, R, logits);
}

// ---- gate/up: the shared expert's unit first (it needs no routing), then the routed items ----
struct GuItem
{
    u32x4 g[4], u[4];                       // the wave's 4 k groups of gate and up (one 16-byte load per lane each)
    u32x2 sg, su;                           // their 4 group scales of the lane's row
};

constexpr int GU_SH_GRID = 2 * NB_I;        // with the shared expert: workgroup b owns matrix b & 1 of row block b >> 1

// SH: workgroup b first computes the full-K sum of one shared matrix (gate for even b, up for odd b) over 16 rows of I
// as two 8-tile units (wave w: k steps 16 w + 8 j .. + 8 of F16T, against its own x fragments), loaded before the
// routing prologue so that their loads cover it; the wave-ordered fp32 sums go to the SHP_SLOT area of act, and the
// down launch forms the shared act f16(silu(g) u) from them. Then the routed items b, b + G, ... (slot, 16-row block).
template <bool SH>
__global__ void __launch_bounds__(GW * 64) gu7_kernel(
    const void* __restrict__ x, int xf, const float* __restrict__ logits, const float* __restrict__ bias, int E,
    int topk, float scale, int64_t* __restrict__ sel, uint16_t* __restrict__ rw, int R, int lo, int n_hot,
    const int64_t* __restrict__ gate_w, const int64_t* __restrict__ up_w, const int64_t* __restrict__ gate_s,
    const int64_t* __restrict__ up_s, const uint8_t* __restrict__ sh_gw, const uint8_t* __restrict__ sh_uw,
    _Float16* __restrict__ act, int G)
{
    __shared__ Route rt;
    __shared__ const uint8_t* tab[4][HMOE_MAXE];
    __shared__ const uint8_t* ptr[4][MAXSLOT];
    __shared__ int64_t ssel[MAXR * TOPK];
    __shared__ uint16_t srw[MAXR * TOPK];
    __shared__ f32x4 red[2][GW][2][64];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, tok = l & 15, ks = l >> 4, row = l & 15;
    const int b = blockIdx.x;                                 // (G: the grid, passed: gridDim reads the dispatch packet)
    const bool live = tok < R;
    // the arguments in the kernel-argument segment's last cache line, read with the first ones: read where first used
    // (the compiler's choice), that scalar load's wait would come at the first workgroup barrier, under the stream
    asm volatile("" :: "s"(act), "s"(G));
    // Loads are issued in the order they are consumed (the wait counter is in order) and unconditionally (a load
    // under a branch makes the compiler wait for every outstanding load where the paths meet): the window's pointer
    // tables (x standing in without a window), the given picks, the logits of the wave's rows and the bias, the first
    // half of x, then both shared units; the second half of x follows the routing prologue.
    const int te = min((int) threadIdx.x, max(n_hot - 1, 0));
    const bool hot = n_hot > 0;
    const int64_t* xt = (const int64_t*) x;
    const int64_t t0 = ldg<int64_t>(hot ? gate_w + te : xt), t1 = ldg<int64_t>(hot ? up_w + te : xt);
    const int64_t t2 = ldg<int64_t>(hot ? gate_s + te : xt), t3 = ldg<int64_t>(hot ? up_s + te : xt);
    // the given picks (used without logits; with logits sel / rw are the output buffers, read and ignored)
    const int pi = min((int) threadIdx.x, R * TOPK - 1);
    const Pick pk = {ldg<int64_t>(sel + pi), ldg<uint16_t>(rw + pi)};
    RowIn r0, r1;                                              // rows w and w + GW (one bias)
    if (logits)
    {
        load_logits_global(logits + (size_t) min(w, R - 1) * RMAXE, E, r0.lg);
        load_logits_global(logits + (size_t) min(w + GW, R - 1) * RMAXE, E, r1.lg);
        load_bias_global(bias, logits, E, r0.b);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the rows' x for this wave's k range: k step t covers k = 512 w + 32 t + 8 ks .. + 8 of row tok (A operand), read
    // as buffer loads in two halves of 8 k steps: a lane of a row past R reads out of range (no memory traffic; its MFMA
    // row is never stored). The first half (the first shared unit's k steps) goes out now, the second after the
    // routing prologue, so that both shared units' tiles fit the registers while the prologue runs.
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*) x, (short) 0, R * H * 2, 0x00020000);
    const int xoff = live ? (tok * H + 512 * w + 8 * ks) * 2 : 0x40000000;
    u32x4 raw[16];
    #pragma unroll
    for (int t = 0; t < 8; ++t) raw[t] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff + 64 * t, 0, 0);
    // both shared units (k steps 16 w .. + 8 and + 8 .. + 16) go out before the routing prologue, so their loads cover it
    GuItem A, B;
    const uint8_t* shm = (b & 1) ? sh_uw : sh_gw;
    const uint8_t* shbase = shm + ((size_t) ((b >> 1) * KS_H + 16 * w) * 64 + l) * 16;
    if (SH)
    {
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            A.g[q] = ldw16(shbase + q * 1024); A.u[q] = ldw16(shbase + (4 + q) * 1024);
        }
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            B.g[q] = ldw16(shbase + (8 + q) * 1024); B.u[q] = ldw16(shbase + (12 + q) * 1024);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    f16x8 xa[16];
    #pragma unroll
    for (int t = 0; t < 8; ++t) xa[t] = xf ? as_f16x8(raw[t]) : bf8_to_f16(raw[t]);
    // every thread stores (threads past n_hot repeat entry n_hot - 1 with its own value)
    tab[0][te] = (const uint8_t*) t0; tab[1][te] = (const uint8_t*) t1;
    tab[2][te] = (const uint8_t*) t2; tab[3][te] = (const uint8_t*) t3;
    if (logits)
    {
        bias_or_zero(r0.b, bias != nullptr);
        if (w < R) select_from(r0, E, topk, scale, ssel + w * TOPK, srw + w * TOPK);
        #pragma unroll
        for (int i = 0; i < 4; ++i) r1.b[i] = r0.b[i];
        if (w + GW < R) select_from(r1, E, topk, scale, ssel + (w + GW) * TOPK, srw + (w + GW) * TOPK);
        __syncthreads();
        // wave 0: the selection out (workgroup 0), the distinct experts, then their pointers and the routing record
        if (w == 0)
        {
            if (b == 0)
            {
                #pragma unroll
                for (int h = 0; h < 2; ++h)
                    if (l + 64 * h < R * TOPK) { sel[l + 64 * h] = ssel[l + 64 * h]; rw[l + 64 * h] = srw[l + 64 * h]; }
            }
            route_wave(ssel, srw, R, lo, n_hot, rt);
            const int m = rt.m;
            #pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                const int j = l + 64 * h;
                if (j < m)
                {
                    const int e = rt.e[j];
                    ptr[0][j] = tab[0][e]; ptr[1][j] = tab[1][e]; ptr[2][j] = tab[2][e]; ptr[3][j] = tab[3][e];
                }
            }
            if (b == 0)
            {
                int* rec = (int*) (act + (size_t) REC_SLOT * MAXR * I);
                if (l == 0) rec[0] = m;
                #pragma unroll
                for (int h = 0; h < 2; ++h)
                {
                    const int j = l + 64 * h;
                    rec[REC_E + j] = (j < m ? rt.e[j] : 0) | (m << 16);
                }
            }
            if (m == 0 && l < 4) ptr[l][0] = shm;
        }
    }
    else
    {
        route_picks(pk, R, lo, n_hot, rt);
        const int m = rt.m;
        if (threadIdx.x < m)
        {
            const int e = rt.e[threadIdx.x];
            ptr[0][threadIdx.x] = tab[0][e]; ptr[1][threadIdx.x] = tab[1][e];
            ptr[2][threadIdx.x] = tab[2][e]; ptr[3][threadIdx.x] = tab[3][e];
        }
        // the routing record for the down launch: m and the local expert id of every slot
        if (b == 0)
        {
            int* rec = (int*) (act + (size_t) REC_SLOT * MAXR * I);
            if (threadIdx.x == 0) rec[0] = m;
            if (threadIdx.x < MAXSLOT) rec[REC_E + threadIdx.x] = ((int) threadIdx.x < m ? rt.e[threadIdx.x] : 0) | (m << 16);
        }
        if (m == 0 && threadIdx.x < 4) ptr[threadIdx.x][0] = shm;
    }
    // (no routed expert: slot 0 stands in as the shared matrix, 25 MB, beyond every offset a stand-in load reaches)
    __syncthreads();
    const int m = rt.m;
    const int total = m * NB_I;
    const int nr = b < total ? (total - 1 - b) / G + 1 : 0;
    if (!SH && nr == 0) return;                                // uniform over the workgroup
    // the second half of x (k steps 8 .. 16), ahead of the routed loads, so that waiting for it waits for none of them
    #pragma unroll
    for (int t = 8; t < 16; ++t) raw[t] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff + 64 * t, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    const DqConsts dq = dq_consts();
    // routed item i < nr; past the end (the ring's last prefetch, or no routed item at all) the four loads of a
    // matrix all read one tile (k stride 0): 1 KB instead of repeating the item's 4 KB (an integer select: a pointer
    // select here becomes a branch whose register copies wait for every load in flight)
    auto load = [&](GuItem& S, int i) {
        const int it = b + min(i, max(nr - 1, 0)) * G, j = min(it / NB_I, max(m - 1, 0)), nb = it - (it / NB_I) * NB_I;
        const size_t toff = ((size_t) (nb * KG_H + 4 * w) * 64 + l) * 16;
        const size_t soff = sc_index(nb * 16 + row, 4 * w, KG_H) * 2;
        const int kst = i < nr ? 1024 : 0;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            S.g[k] = ldw16(ptr[0][j] + toff + k * kst);
            S.u[k] = ldw16(ptr[1][j] + toff + k * kst);
        }
        S.sg = ld8(ptr[2][j] + soff); S.su = ld8(ptr[3][j] + soff);
    };
    auto run = [&](const GuItem& S, int i, int par) {
        const int it = b + i * G, j = it / NB_I, nb = it - j * NB_I;
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
    if (SH)
    {
        // the shared units: A against x's first half, then routed item 0's loads into A's registers, then B against
        // the second half
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int q = 0; q < 4; ++q) acc = mfma16(xa[q], as_f16x8(A.g[q]), acc);
        #pragma unroll
        for (int q = 0; q < 4; ++q) acc = mfma16(xa[4 + q], as_f16x8(A.u[q]), acc);
        __builtin_amdgcn_sched_barrier(0);
        load(A, 0);
        __builtin_amdgcn_sched_barrier(0);
        #pragma unroll
        for (int t = 8; t < 16; ++t) xa[t] = xf ? as_f16x8(raw[t]) : bf8_to_f16(raw[t]);
        #pragma unroll
        for (int q = 0; q < 4; ++q) acc = mfma16(xa[8 + q], as_f16x8(B.g[q]), acc);
        #pragma unroll
        for (int q = 0; q < 4; ++q) acc = mfma16(xa[12 + q], as_f16x8(B.u[q]), acc);
        // wave-ordered sum through red[1] (routed item 0 writes red[0] next; item 1 writes red[1] after item 0's
        // barrier, which every reader here has passed)
        red[1][w][0][l] = acc;
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int ll = threadIdx.x >> 2, ie = threadIdx.x & 3, tk = 4 * (ll >> 4) + ie;
            if (tk < R)
            {
                float sum = 0.f;
                #pragma unroll
                for (int ww = 0; ww < GW; ++ww) sum += red[1][ww][0][ll][ie];
                float* shp = (float*) (act + (size_t) SHP_SLOT * MAXR * I);
                shp[((size_t) (b & 1) * MAXR + tk) * I + (b >> 1) * 16 + (ll & 15)] = sum;
            }
        }
    }
    else
    {
        load(A, 0);
        __builtin_amdgcn_sched_barrier(0);
        #pragma unroll
        for (int t = 8; t < 16; ++t) xa[t] = xf ? as_f16x8(raw[t]) : bf8_to_f16(raw[t]);
    }
    // A holds routed item 0 (or a stand-in)
    for (int i = 0; i < nr; i += 2)
    {
        load(B, i + 1);
        run(A, i, 0);
        if (i + 1 >= nr) break;
        load(A, i + 2);
        run(B, i + 1, 1);
    }
}

// ---- down: the shared expert's items first (they need no routing), then the routed (slot quad, row block) items ----
struct DnItem
{
    u32x4 d[4];                             // the wave's 4 tiles of one 16-row block of down
    u32x2 s;                                // their 4 group scales of the lane's row (routed items)
};

constexpr int DN_GMIN = NB_H / 2, DN_GMAX = NB_H;   // grid range: one or two shared items per workgroup
constexpr int XSH_LD = I + 8;                       // row stride (f16) of the down launch's shared act in LDS
// the cost of a slot-quad change inside a workgroup's down range, in items (its act reload, 16 R KB, mostly from L2)
#ifndef DN_XC_NUM
#define DN_XC_NUM 4
#endif
#define DN_XCOST(R) (((R) * DN_XC_NUM) / 16)

// workgroup b: (SH) shared items nb = b and b + G (when < NB_H), then a contiguous range of the routed items
// (quad-major, so a quad's act stays in registers). Every item moves the same 64 KB; the ranges give every workgroup
// floor or ceil of (shared + routed) / G items in total. The shared act, f16(silu(g) u), is formed here from the fp32
// gate and up sums the gate/up launch left in the SHP_SLOT area of act, NJ float4 steps per thread (NJ * 4096
// elements per workgroup cover the R live rows: the host picks the smallest of 1, 2, 4, 8 that does).
template <bool SH, int NJ>
__global__ void __launch_bounds__(DW * 64) dn6_kernel(
    int R, int n_hot, const int64_t* __restrict__ down_w, const int64_t* __restrict__ down_s,
    const _Float16* __restrict__ act, const uint8_t* __restrict__ sh_dw, float* __restrict__ y32,
    int* __restrict__ nparts_out, int G)
{
    // one LDS block laid out by hand: the reduction buffer and the tables at the bottom, so that every access in the
    // item loop is one base register plus an immediate offset (below 64 KB), then the shared act
    constexpr int O_RED = 0, O_TAB = O_RED + 2 * DW * 64 * 16, O_PTR = O_TAB + 2 * HMOE_MAXE * 8;
    constexpr int O_XSH = O_PTR + 2 * MAXSLOT * 8, N_SMEM = O_XSH + (SH ? MAXR * XSH_LD * 2 : 0);
    static_assert(O_XSH <= 65536, "the item loop's LDS must sit below 64 KB");
    __shared__ __attribute__((aligned(16))) uint8_t smem[N_SMEM];
    auto& tab = *reinterpret_cast<const uint8_t* (*)[2][HMOE_MAXE]>(smem + O_TAB);
    auto& ptr = *reinterpret_cast<const uint8_t* (*)[2][MAXSLOT]>(smem + O_PTR);
    auto& red = *reinterpret_cast<f32x4 (*)[2][DW][64]>(smem + O_RED);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int sw = w >> 2, kq = w & 3;                          // routed items: slot of the quad, k quarter of I
    const int b = blockIdx.x;                                 // (G: the grid, passed: gridDim reads the dispatch packet)
    asm volatile("" :: "s"(sh_dw), "s"(G));                   // (read with the first arguments, as in gu7_kernel)
    const int part0 = SH ? 1 : 0, nsh = SH ? NB_H : 0;
    const int s_mine = SH ? (b + G < NB_H ? 2 : 1) : 0;       // (G <= NB_H: every workgroup has one)
    // loads in issue order: pointer tables, the gate/up launch's routing record (slot count and the local expert of
    // each slot), the shared act, the shared items (all independent of routing)
    // (every load here is unconditional, with a valid stand-in address where there is nothing to load: a load under a
    // branch makes the compiler wait for all outstanding loads where the paths meet)
    const int te = min((int) threadIdx.x, max(n_hot - 1, 0));
    const int* rec = (const int*) (act + (size_t) REC_SLOT * MAXR * I);
    const int64_t t0 = ldg<int64_t>(n_hot > 0 ? down_w + te : (const int64_t*) rec);
    const int64_t t1 = ldg<int64_t>(n_hot > 0 ? down_s + te : (const int64_t*) rec);
    // (the slot count comes with every slot's entry, read by lane loads: word 0 read from its uniform address would be a
    // scalar load, whose wait, on the scalar counter, comes before the shared tiles' loads and holds them back)
    const int re = ldg<int>(rec + REC_E + min((int) threadIdx.x, MAXSLOT - 1));
    __builtin_amdgcn_sched_barrier(0);                          // keep the routing loads ahead of the item loads
    // shared items: wave w owns k group w of I (4 k steps of F16T) with the shared act of its k group as the A operand.
    // The act f16(silu(g) u) of the R live rows is formed once per workgroup into xsh, 4 elements per thread in each
    // of NJ steps, from the fp32 sums loaded first, so forming it does not wait for the tiles; the waves read their
    // fragments after the table barrier. Past R * I / 4 the loads repeat the last float4 (one cache line per wave)
    // and nothing is stored. The second shared item is the first one again when there is none (an L2 hit).
    auto& xsh = *reinterpret_cast<_Float16 (*)[MAXR][XSH_LD]>(smem + O_XSH);     // (SH only)
    u32x4 S0[4], S1[4];
    if (SH)
    {
        const float* shp = (const float*) (act + (size_t) SHP_SLOT * MAXR * I);
        const int nq4 = R * (I / 4);
        u32x4 gv[NJ], uv[NJ];
        #pragma unroll
        for (int j = 0; j < NJ; ++j)
        {
            const int q = min((int) threadIdx.x + DW * 64 * j, nq4 - 1);
            const size_t o = (size_t) (q >> 9) * I + (q & 511) * 4;
            gv[j] = ld16(shp + o);
            uv[j] = ld16(shp + MAXR * I + o);
        }
        const uint8_t* w0 = sh_dw + ((size_t) (b * KS_I + 4 * w) * 64 + l) * 16;
        const uint8_t* w1 = sh_dw + ((size_t) ((s_mine == 2 ? b + G : b) * KS_I + 4 * w) * 64 + l) * 16;
        #pragma unroll
        for (int k = 0; k < 4; ++k) S0[k] = ldw16(w0 + k * 1024);
        #pragma unroll
        for (int k = 0; k < 4; ++k) S1[k] = ldw16(w1 + k * 1024);
        __builtin_amdgcn_sched_barrier(0);
        #pragma unroll
        for (int j = 0; j < NJ; ++j)
        {
            const int q = (int) threadIdx.x + DW * 64 * j;
            f16x4 v;
            #pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (_Float16) (silu(__uint_as_float(gv[j][e])) * __uint_as_float(uv[j][e]));
            if (q < nq4) *(f16x4*) &xsh[q >> 9][(q & 511) * 4] = v;
        }
    }
    // every thread stores (threads past n_hot repeat entry n_hot - 1 with its own value): a store under a branch
    // would pull the table loads into it, behind the item loads
    tab[0][te] = (const uint8_t*) t0; tab[1][te] = (const uint8_t*) t1;
    __syncthreads();
    const int m = min(max(__builtin_amdgcn_readfirstlane(re) >> 16, 0), min(n_hot, MAXSLOT)), nq = (m + 3) / 4;
    if (threadIdx.x < m)
    {
        const int e = min(re & 0xffff, n_hot - 1);
        ptr[0][threadIdx.x] = tab[0][e]; ptr[1][threadIdx.x] = tab[1][e];
    }
    // no routed expert: slot 0 stands in as act, so the first routed load below stays unconditional and in bounds
    if (m == 0 && threadIdx.x == 0) { ptr[0][0] = (const uint8_t*) act; ptr[1][0] = (const uint8_t*) act; }
    if (b == 0 && threadIdx.x == 0) *nparts_out = part0 + nq;
    __syncthreads();
    int r0, nr;
    {
        // the routed items are split by cost, not by count: a workgroup whose range crosses into the next slot quad
        // reloads that quad's act (4 slots x R rows x I), so every quad is preceded by xc virtual items; a range that
        // starts among them starts at the quad's first item, one that ends among them ends at the quad's end
        const long long xc = DN_XCOST(R), span = NB_H + xc, V = (long long) nq * span, T = nsh + V;
        auto start = [&](int bb) {                              // routed items before workgroup bb
            const long long sh_before = (long long) (nsh / G) * bb + min(bb, nsh % G);
            const long long v = max(0ll, min(V, T * bb / G - sh_before));
            const long long q = v / span;
            return (int) (q * NB_H + max(v - q * span - xc, 0ll));
        };
        r0 = start(b);
        nr = max(0, start(b + 1) - r0);
    }
    if (s_mine + nr == 0) return;                              // uniform over the workgroup
    const DqConsts dq = dq_consts();
    // routed item i; a slot past m reads one fixed tile of slot m - 1 with the same loads (no HBM traffic), and past
    // the end (the ring's last prefetch) the four loads read the last item's first tile (k stride 0: 1 KB, not 4 KB)
    auto load = [&](DnItem& S, int i) {
        const int it = r0 + min(i, max(nr - 1, 0)), qd = it / NB_H, nb = it - qd * NB_H, j = 4 * qd + sw;
        const bool ok = j < m;
        const int jj = max(min(j, m - 1), 0), nbb = ok ? nb : 0;
        // (offsets in 32-bit arithmetic, zero-extended per item: a 64-bit lane term would stay live across the loop)
        const size_t toff = (uint32_t) (((nbb * KG_I + 4 * kq) * 64 + l) * 16);
        const size_t soff = (uint32_t) (sc_index(nbb * 16 + (l & 15), 4 * kq, KG_I) * 2);
        const int kst = (ok && i < nr) ? 1024 : 0;
        #pragma unroll
        for (int k = 0; k < 4; ++k) S.d[k] = ldw16(ptr[0][jj] + toff + k * kst);
        S.s = ld8(ptr[1][jj] + soff);
    };
    // the sum of the 16 wave partials of a 16-row block in wave order -> y32[part]
    auto reduce = [&](const f32x4& acc, int par, int part, int nb) {
        red[par][w][l] = acc;
        __syncthreads();
        if (threadIdx.x < 256)
        {
            const int ll = threadIdx.x >> 2, ie = threadIdx.x & 3, tk = 4 * (ll >> 4) + ie;
            if (tk < R)
            {
                float sum = 0.f;
                #pragma unroll
                for (int ww = 0; ww < DW; ++ww) sum += red[par][ww][ll][ie];
                y32[((size_t) part * MAXR + tk) * H + nb * 16 + (ll & 15)] = sum;
            }
        }
        // red[par] is written again two items later, after the next item's barrier
    };
    DnItem A, B;
    load(A, 0);                                                 // (unconditional: a stand-in tile when nr == 0)
    // the act rows of quad qd for this wave's slot and k quarter, loaded with no select after them (a select would
    // wait for the loads where it stands): rows past R read row 0 (their outputs are never stored), a slot past m
    // reads slot m - 1 and its wave's partial is zeroed
    // (buffer loads: the slot offset is scalar and the lane's offset one 32-bit register, where a 64-bit lane address
    // would not fit the register budget)
    f16x8 xa[16];
    const __amdgpu_buffer_rsrc_t act_rs = __builtin_amdgcn_make_buffer_rsrc((void*) act, (short) 0,
                                                                           (int) (ACT_SLOTS * MAXR * I * 2), 0x00020000);
    auto load_act = [&](int qd) {
        const int j = __builtin_amdgcn_readfirstlane(min(4 * qd + sw, max(m - 1, 0)));
        // the lane's byte offset in a slot, formed here from an opaque copy of the thread index so that it is not
        // kept in a register across the loop (the loop has none to spare)
        int tid;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int) threadIdx.x));
        // (a row past R reads out of range: no memory traffic, and its MFMA row is never stored)
        const int tl = tid & 15, act_lane = tl < R ? (tl * I + 512 * ((tid >> 6) & 3) + 8 * ((tid >> 4) & 3)) * 2
                                                   : 0x10000000;
        #pragma unroll
        for (int t = 0; t < 16; ++t)
            xa[t] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(act_rs, act_lane + 64 * t,
                                                                                    j * MAXR * I * 2, 0));
    };
    if (SH)
    {
        // the wave's A fragments of the shared act (rows past R are zero), addressed from an opaque copy of the thread
        // index so that nothing derived here is shared with (and kept live into) the item loop
        f16x8 xs[4];
        {
            int tid;
            asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int) threadIdx.x));
            const int tk = tid & 15;
            const bool lv = tk < R;
            const _Float16* xr = &xsh[lv ? tk : 0][128 * (tid >> 6) + 8 * ((tid >> 4) & 3)];
            #pragma unroll
            for (int t = 0; t < 4; ++t)
            {
                const f16x8 v = *(const f16x8*) (xr + 32 * t);
                xs[t] = lv ? v : (f16x8) {};
            }
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int t = 0; t < 4; ++t) acc = mfma16(xs[t], as_f16x8(S0[t]), acc);
        reduce(acc, 0, 0, b);
        if (s_mine == 2)
        {
            acc = (f32x4) {0.f, 0.f, 0.f, 0.f};
            #pragma unroll
            for (int t = 0; t < 4; ++t) acc = mfma16(xs[t], as_f16x8(S1[t]), acc);
            reduce(acc, 1, 0, b + G);
        }
    }
    load_act(r0 / NB_H);
    auto run = [&](const DnItem& S, int i, int par) {
        const int it = r0 + i, qd = it / NB_H, nb = it - qd * NB_H;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int k = 0; k < 4; ++k) group_i4(xa + 4 * k, S.d[k], scale_of(S.s, k), acc, dq);
        if (4 * qd + sw >= m) acc = (f32x4) {0.f, 0.f, 0.f, 0.f};     // a slot past m adds nothing
        // the next item's act when it opens a new quad: issued after this item's MFMAs and before the next prefetch,
        // so waiting for it does not wait for that prefetch as well
        if (i + 1 < nr && it + 1 == (qd + 1) * NB_H) load_act(qd + 1);
        reduce(acc, par, part0 + qd, nb);
    };
    const int p0 = s_mine & 1;                                  // red parity of the first routed item
    for (int i = 0; i < nr; i += 2)
    {
        load(B, i + 1);
        __builtin_amdgcn_sched_barrier(0);                      // the prefetch goes out before this item's MFMAs
        run(A, i, p0);
        if (i + 1 >= nr) break;
        load(A, i + 2);
        __builtin_amdgcn_sched_barrier(0);
        run(B, i + 1, p0 ^ 1);
    }
}

// ---- down for one row: output rows owned, no part buffer and no reduction launch ----
// Workgroup b owns the 24 output rows [24 b, 24 b + 24): one whole 16-row tile (nbF) and one half tile (rows
// 8 ph .. 8 ph + 8 of tile nbH), so 256 workgroups cover H with equal work. It runs every part of the step for those
// rows, the shared expert (part 0) and each slot quad, with the waves in dn6_kernel's roles (routed: slot w / 4 of the
// quad, k quarter w % 4; shared: k group w), the same MFMA chains and the same wave-ordered part sums, and adds the
// parts in order into one fp32 sum per output: the bits of dn6_kernel followed by dec_d_kernel. The half tile's loads
// let lanes l and l ^ 8 read the same 16 bytes (its 8 rows, whole 128-byte lines); its MFMA columns of the other half
// are duplicates, never stored. A quad item runs as two sub-items of 2 k groups.
// At one row a step has at most 8 distinct experts (2 slot quads, 4 sub-items per wave), so nothing needs a ring:
// each wave issues its shared tiles, then (after the pointer tables) its first two routed sub-items, and the last two
// as soon as the shared tiles' registers are free. The act rows of the 8 slots (32 KB) and the shared act go to LDS at
// the start (their loads are issued ahead of every tile), so no act load waits behind a tile. The MFMA A rows of
// tokens past row 0 read row 0 again: those output rows are never stored, and MFMA rows do not interact.
// (With more rows the act of a step no longer fits LDS, and a variant of this kernel holding each quad's act in
// registers could keep too few tiles in flight: 16 waves at 128 registers each; it measured slower than the part-sum
// form at 4 rows, so rows past the first take that form.)
constexpr int DN8_GRID = H / 24;                      // 256 workgroups of 24 rows

template <bool SH>
__global__ void __launch_bounds__(DW * 64) dn8_kernel(
    int n_hot, const int64_t* __restrict__ down_w, const int64_t* __restrict__ down_s,
    const _Float16* __restrict__ act, const uint8_t* __restrict__ sh_dw, float* __restrict__ y,
    uint16_t* __restrict__ out)
{
    constexpr int XL = I + 8;                                   // LDS row stride (f16) of an act row
    constexpr int O_RED = 0, O_TAB = O_RED + 2 * DW * 2 * 64 * 16, O_PTR = O_TAB + 2 * HMOE_MAXE * 8;
    constexpr int O_ACT = O_PTR + 2 * MAXSLOT * 8, O_XSH = O_ACT + 8 * XL * 2, N_SMEM = O_XSH + XL * 2;
    __shared__ __attribute__((aligned(16))) uint8_t smem[N_SMEM];
    auto& tab = *reinterpret_cast<const uint8_t* (*)[2][HMOE_MAXE]>(smem + O_TAB);
    auto& ptr = *reinterpret_cast<const uint8_t* (*)[2][MAXSLOT]>(smem + O_PTR);
    auto& red = *reinterpret_cast<f32x4 (*)[2][DW][2][64]>(smem + O_RED);
    auto& act8 = *reinterpret_cast<_Float16 (*)[8][XL]>(smem + O_ACT);
    auto& xsh = *reinterpret_cast<_Float16 (*)[XL]>(smem + O_XSH);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int sw = w >> 2, kq = w & 3;
    const int b = blockIdx.x;
    const int ph = b & 1;
    const int nbF = (3 * b + ph) >> 1, nbH = ph ? nbF - 1 : nbF + 1;
    const int lh = (l & ~8) | (ph << 3);
    asm volatile("" :: "s"(sh_dw), "s"(out));
    const int te = min((int) threadIdx.x, max(n_hot - 1, 0));
    const int* rec = (const int*) (act + (size_t) REC_SLOT * MAXR * I);
    const int64_t t0 = ldg<int64_t>(n_hot > 0 ? down_w + te : (const int64_t*) rec);
    const int64_t t1 = ldg<int64_t>(n_hot > 0 ? down_s + te : (const int64_t*) rec);
    const int re = ldg<int>(rec + REC_E + min((int) threadIdx.x, MAXSLOT - 1));
    // row 0 of act slots 0..7 (2 pieces of 8 f16 per thread; slots past m hold stale values, never used)
    u32x4 av[2];
    #pragma unroll
    for (int c = 0; c < 2; ++c)
    {
        const int p = (int) threadIdx.x + DW * 64 * c;
        av[c] = ld16(act + (size_t) (p >> 8) * MAXR * I + (p & 255) * 8);
    }
    u32x4 gv = {}, uv = {};
    if (SH)
    {
        const float* shp = (const float*) (act + (size_t) SHP_SLOT * MAXR * I);
        const int q = min((int) threadIdx.x, I / 4 - 1);
        gv = ld16(shp + q * 4);
        uv = ld16(shp + MAXR * I + q * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 SF[4], SH4[4];
    if (SH)
    {
        const uint8_t* wf = sh_dw + ((size_t) (nbF * KS_I + 4 * w) * 64 + l) * 16;
        const uint8_t* wh = sh_dw + ((size_t) (nbH * KS_I + 4 * w) * 64 + lh) * 16;
        #pragma unroll
        for (int k = 0; k < 4; ++k) SF[k] = ldw16(wf + k * 1024);
        #pragma unroll
        for (int k = 0; k < 4; ++k) SH4[k] = ldw16(wh + k * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
    for (int c = 0; c < 2; ++c)
    {
        const int p = (int) threadIdx.x + DW * 64 * c;
        *(u32x4*) &act8[p >> 8][(p & 255) * 8] = av[c];
    }
    if (SH && threadIdx.x < I / 4)
    {
        f16x4 v;
        #pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (_Float16) (silu(__uint_as_float(gv[e])) * __uint_as_float(uv[e]));
        *(f16x4*) &xsh[threadIdx.x * 4] = v;
    }
    tab[0][te] = (const uint8_t*) t0; tab[1][te] = (const uint8_t*) t1;
    __syncthreads();
    const int m = min(max(__builtin_amdgcn_readfirstlane(re) >> 16, 0), min(n_hot, 8)), nq = (m + 3) / 4;
    if (threadIdx.x < m)
    {
        const int e = min(re & 0xffff, n_hot - 1);
        ptr[0][threadIdx.x] = tab[0][e]; ptr[1][threadIdx.x] = tab[1][e];
    }
    if (m == 0 && threadIdx.x == 0) { ptr[0][0] = (const uint8_t*) act; ptr[1][0] = (const uint8_t*) act; }
    __syncthreads();
    // reducing threads: thread o < 24 owns output row 24 b + o (token 0, element 0 of its lane)
    const int o = threadIdx.x;
    const bool ored = o < 24;
    const int on = 24 * b + o, of = (on >> 4) == nbF ? 0 : 1, oll = on & 15;
    float s = 0.f;
    auto reduce = [&](const f32x4& af, const f32x4& ah, int par) {
        red[par][w][0][l] = af; red[par][w][1][l] = ah;
        __syncthreads();
        if (ored)
        {
            float sum = 0.f;
            #pragma unroll
            for (int ww = 0; ww < DW; ++ww) sum += red[par][ww][of][oll][0];
            s = s + sum;
        }
    };
    const DqConsts dq = dq_consts();
    struct Sub { u32x4 f[2], h[2]; uint32_t sf, shh; };
    const int nsub = 2 * nq;
    auto load = [&](Sub& S, int i) {
        const int qd = i >> 1, hf = i & 1, j = 4 * qd + sw;
        const int jj = max(min(j, m - 1), 0);
        const int g0 = 4 * kq + 2 * hf;
        const size_t tf = (uint32_t) (((nbF * KG_I + g0) * 64 + l) * 16);
        const size_t th = (uint32_t) (((nbH * KG_I + g0) * 64 + lh) * 16);
        const size_t sf = (uint32_t) (sc_index(nbF * 16 + (l & 15), g0, KG_I) * 2);
        const size_t sh = (uint32_t) (sc_index(nbH * 16 + (lh & 15), g0, KG_I) * 2);
        const int kst = (j < m && i < nsub) ? 1024 : 0;
        #pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            S.f[k] = ldw16(ptr[0][jj] + tf + k * kst);
            S.h[k] = ldw16(ptr[0][jj] + th + k * kst);
        }
        S.sf = ldg<uint32_t>(ptr[1][jj] + sf);
        S.shh = ldg<uint32_t>(ptr[1][jj] + sh);
    };
    Sub S0, S1, S2, S3;
    load(S0, 0);
    load(S1, 1);
    f32x4 af = {0.f, 0.f, 0.f, 0.f}, ah = af;
    int par = 0;
    // the A fragments of k group g of a 512-k range starting at k0 in an LDS act row (every lane reads the row)
    auto frag = [&](const _Float16* rowp, int k0, int g, f16x8 (&xa)[4]) {
        #pragma unroll
        for (int t = 0; t < 4; ++t) xa[t] = *(const f16x8*) (rowp + k0 + 128 * g + 32 * t + 8 * (l >> 4));
    };
    if (SH)
    {
        f16x8 xs[4];
        frag(&xsh[0], 128 * w, 0, xs);
        #pragma unroll
        for (int t = 0; t < 4; ++t) af = mfma16(xs[t], as_f16x8(SF[t]), af);
        #pragma unroll
        for (int t = 0; t < 4; ++t) ah = mfma16(xs[t], as_f16x8(SH4[t]), ah);
        reduce(af, ah, 0);
        par = 1;
    }
    __builtin_amdgcn_sched_barrier(0);
    load(S2, 2);
    load(S3, 3);
    __builtin_amdgcn_sched_barrier(0);
    auto scale2 = [](uint32_t v, int k) { return __uint_as_float(k ? (v & 0xffff0000u) : (v << 16)); };
    auto run = [&](const Sub& S, int qd, auto hfc) {
        constexpr int HF = decltype(hfc)::value;
        if (HF == 0) { af = (f32x4) {0.f, 0.f, 0.f, 0.f}; ah = af; }
        const _Float16* rowp = &act8[min(4 * qd + sw, 7)][0];
        #pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            f16x8 xa[4];
            frag(rowp, 512 * kq, 2 * HF + k, xa);
            group_i4(xa, S.f[k], scale2(S.sf, k), af, dq);
            group_i4(xa, S.h[k], scale2(S.shh, k), ah, dq);
        }
        if (HF == 1)
        {
            if (4 * qd + sw >= m) { af = (f32x4) {0.f, 0.f, 0.f, 0.f}; ah = af; }
            reduce(af, ah, par);
            par ^= 1;
        }
    };
    if (nq > 0)
    {
        run(S0, 0, ic<0>{});
        run(S1, 0, ic<1>{});
    }
    if (nq > 1)
    {
        run(S2, 1, ic<0>{});
        run(S3, 1, ic<1>{});
    }
    if (ored)
    {
        if (y) y[on] = y[on] + s;
        if (out) out[on] = hmoe_f2bf(s);
    }
}

// ---- y (+)= sum of the parts in order; or the layer's bf16 output ----
// one thread per element: the parts are loaded 8 at a time (the first 8 before the part count arrives; a part past the
// count is read, from inside the buffer, and not added), then added in part order
__global__ void __launch_bounds__(256) dec_d_kernel(const float* __restrict__ y32, const int* __restrict__ nparts_p,
                                                    int R, float* __restrict__ y, uint16_t* __restrict__ out)
{
    static_assert(MAX_PARTS >= 8, "the first batch of parts is read before the part count");
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= R * H) return;
    const int r = i / H, n = i - r * H;
    const float* yp = y32 + (size_t) r * H + n;
    constexpr size_t PS = (size_t) MAXR * H;                   // one part
    float v[8];
    #pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = yp[k * PS];
    const int np = *nparts_p;
    float s = 0.f;
    for (int p = 0;;)
    {
        #pragma unroll
        for (int k = 0; k < 8; ++k) s = p + k < np ? s + v[k] : s;
        p += 8;
        if (p >= np) break;
        #pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = yp[(size_t) min(p + k, MAX_PARTS - 1) * PS];
    }
    if (y) y[i] = y[i] + s;
    if (out) out[i] = hmoe_f2bf(s);
}

// per_cu workgroups per CU of the current device (the CU count cached per device; threads that race to fill an
// entry store the same value)
int default_grid(int per_cu)
{
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256 * per_cu;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (!v)
    {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return v * per_cu;
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
    // a.xf: 0 bf16, 1 fp16 (mapped from HMOE_XF_BF16 / HMOE_XF_F16); -1 any other flag, the reference's fragment-order
    // x (HMOE_XF_FRAG) included
    HMOE_REQUIRE(a.xf == 0 || a.xf == 1, "moe4: xf must be HMOE_XF_BF16 (0) or HMOE_XF_F16 (2); the reference's "
                 "fragment-order x (xf = 1) is not supported, pass row-major x");
    HMOE_REQUIRE(a.R >= 1 && a.R <= MAXR, "moe4: rows %d not in [1, %d]", a.R, MAXR);
    HMOE_REQUIRE(a.n_hot >= 0 && a.n_hot <= HMOE_MAXE && a.lo >= 0, "moe4: window lo %d n_hot %d", a.lo, a.n_hot);
    HMOE_REQUIRE(a.x && a.act && a.ctr && a.y32, "moe4: null buffer");
    HMOE_REQUIRE(a.n_hot == 0 || (a.gate_w && a.up_w && a.down_w && a.gate_s && a.up_s && a.down_s), "moe4: null table");
    HMOE_REQUIRE((!a.sh_gw && !a.sh_uw && !a.sh_dw) || (a.sh_gw && a.sh_uw && a.sh_dw), "moe4: partial shared expert");
    HMOE_REQUIRE(((uintptr_t) a.x & 15) == 0 && ((uintptr_t) a.act & 15) == 0, "moe4: x / act not 16-byte aligned");
    HMOE_REQUIRE(a.blocks >= 0 && a.blocks <= 4096, "moe4: blocks %d", a.blocks);
    return HMOE_OK;
}

// launches; phase mask bit 0 = router logits, 1 = shared + routed gate/up, 2 = shared + routed down, 3 = ordered
// reduction (nothing to do after the owning down form of one row); bit 4 takes the part-sum down form
// (down, then reduction) at any row count. blocks: grid of the gate/up and down kernels (0 = one workgroup per CU);
// with the shared expert the gate/up grid is GU_SH_GRID (one shared matrix slice each) and the part-sum down grid is
// kept in [DN_GMIN, DN_GMAX].
static int run_decode(const DecodeArgs& a, int phases, hipStream_t st)
{
    const int R = a.R;
    const bool sh = a.sh_gw != nullptr;
    const int G = a.blocks ? a.blocks : default_grid(1);
    if ((phases & 1) && a.logits)
        router_kernel<<<a.E, 256, 0, st>>>((const uint16_t*) a.x, R, a.wt, a.E, a.logits);
    if (phases & 2)
    {
        int64_t* so = a.logits ? a.sel_out : (int64_t*) a.sel_in;
        uint16_t* ro = a.logits ? a.rw_out : (uint16_t*) a.rw_in;
        if (sh)
            gu7_kernel<true><<<GU_SH_GRID, GW * 64, 0, st>>>(a.x, a.xf, a.logits, a.bias, a.E, a.topk, a.scale, so, ro, R,
                                                             a.lo, a.n_hot, a.gate_w, a.up_w, a.gate_s, a.up_s,
                                                             (const uint8_t*) a.sh_gw, (const uint8_t*) a.sh_uw, a.act,
                                                             GU_SH_GRID);
        else
            gu7_kernel<false><<<G, GW * 64, 0, st>>>(a.x, a.xf, a.logits, a.bias, a.E, a.topk, a.scale, so, ro, R,
                                                     a.lo, a.n_hot, a.gate_w, a.up_w, a.gate_s, a.up_s, nullptr,
                                                     nullptr, a.act, G);
    }
    // at one row the down launch owns its output rows and writes y / out itself (no part buffer, no reduction
    // launch: phase 8 has nothing left to do); more rows take the part-sum form (down, then reduce)
    const bool own = R == 1 && !(phases & 16);
    if ((phases & 4) && own)
    {
        if (sh)
            dn8_kernel<true><<<DN8_GRID, DW * 64, 0, st>>>(a.n_hot, a.down_w, a.down_s, a.act, (const uint8_t*) a.sh_dw,
                                                           a.y, a.out);
        else
            dn8_kernel<false><<<DN8_GRID, DW * 64, 0, st>>>(a.n_hot, a.down_w, a.down_s, a.act, nullptr, a.y, a.out);
    }
    if ((phases & 4) && !own)
    {
        const int gd = min(max(G, DN_GMIN), DN_GMAX);
        if (sh)
        {
            // NJ: float4 steps per thread to form the shared act of R rows (R * 512 float4 over 1024 threads)
            auto k = R <= 2 ? dn6_kernel<true, 1> : R <= 4 ? dn6_kernel<true, 2> : R <= 8 ? dn6_kernel<true, 4>
                                                                                        : dn6_kernel<true, 8>;
            k<<<gd, DW * 64, 0, st>>>(R, a.n_hot, a.down_w, a.down_s, a.act, (const uint8_t*) a.sh_dw, a.y32, a.ctr, gd);
        }
        else
            dn6_kernel<false, 1><<<gd, DW * 64, 0, st>>>(R, a.n_hot, a.down_w, a.down_s, a.act, nullptr, a.y32, a.ctr,
                                                         gd);
    }
    if ((phases & 8) && !own) dec_d_kernel<<<(R * H + 255) / 256, 256, 0, st>>>(a.y32, a.ctr, R, a.y, a.out);
    return HMOE_LAUNCHED("moe4");
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_moe4_scratch_bytes(int which)
{
    switch (which)
    {
        case 0: return (size_t) ACT_SLOTS * MAXR * I * 2;               // act f16 [134][16][2048]
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
    a.x = x; a.xf = xf == HMOE_XF_F16 ? 1 : xf == HMOE_XF_BF16 ? 0 : -1; a.sel_in = sel; a.rw_in = rw; a.R = R; a.n_hot = n_hot; a.lo = lo;
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
                                ctr_b, y32, y, blocks, lo, sh_dw, sh_dw, sh_dw, HMOE_XF_F16);
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

// ---- the allocation-free decode op: hmoe_moe4_forward with its workspace (act, part count, part partials) in one
// file-scope device array, for callers that cannot allocate (under graph capture, in a serving loop that forbids it).
// Each device holds its own copy of the array; its address is taken once per device with the device current, and
// only that address (never the array's name, which in host code is a stand-in, not a device address) reaches a kernel.
namespace hmoe {
constexpr size_t NA_ACT = (size_t) ACT_SLOTS * MAXR * I * 2;           // act f16 [134][16][2048]
constexpr size_t NA_CTR = (size_t) CTR_WORDS * 4;                      // ctr: the part count
constexpr size_t NA_Y32 = (size_t) MAX_PARTS * MAXR * H * 4;           // y32: part partials [33][16][6144]
constexpr size_t NA_BYTES = NA_ACT + NA_CTR + NA_Y32;                  // 21,762,048 bytes
static_assert(NA_ACT % 256 == 0 && NA_CTR % 256 == 0, "each piece stays 256-byte aligned");
}  // namespace hmoe

static __device__ __align__(256) uint8_t scratch[hmoe::NA_BYTES];

namespace hmoe {
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// the device address of `scratch` on the current device (looked up on the first call there)
static int scratch_ptr(uint8_t** out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(HMOE_ERR_HIP, "moe4_forward_noalloc: current device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev])
    {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(HMOE_ERR_HIP, "moe4_forward_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = (uint8_t*) g_scratch_ptr[dev];
    return HMOE_OK;
}
}  // namespace hmoe

extern "C" size_t hmoe_moe4_noalloc_bytes(void) { return NA_BYTES; }

extern "C" int hmoe_moe4_forward_noalloc(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                                         const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                                         const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s, float* y,
                                         int lo, const void* sh_gw, const void* sh_uw, const void* sh_dw, int xf,
                                         void* stream)
{
    HMOE_REQUIRE(R >= 1 && R <= MAXR, "moe4_forward_noalloc: rows %d beyond the static workspace (at most %d rows, %zu "
                 "bytes)", R, MAXR, NA_BYTES);
    uint8_t* ws = nullptr;
    if (int rc = scratch_ptr(&ws)) return rc;
    DecodeArgs a = forward_args(x, sel, rw, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, ws + 0,
                                (int*) (ws + NA_ACT), (float*) (ws + NA_ACT + NA_CTR), y, 0, lo, sh_gw, sh_uw, sh_dw, xf);
    int rc = check(a);
    if (rc) return rc;
    HMOE_REQUIRE(sel && rw && y, "moe4_forward_noalloc: null buffer");
    return run_decode(a, 15, (hipStream_t) stream);
}

extern "C" int hmoe_norm_router(const float* h, const float* norm_w, float eps, int R, const float* wt, int E,
                                float* logits, uint16_t* xn, void* xh, void* stream)
{
    HMOE_REQUIRE(h && norm_w && wt && logits && xn && R >= 1 && R <= MAXR && E >= TOPK && E <= RMAXE,
                 "norm_router: arguments (rows %d experts %d)", R, E);
    HMOE_REQUIRE(((uintptr_t) h & 15) == 0 && ((uintptr_t) norm_w & 15) == 0 && ((uintptr_t) wt & 15) == 0 &&
                 ((uintptr_t) xn & 15) == 0 && ((uintptr_t) xh & 15) == 0, "norm_router: alignment");
    norm_router_kernel<<<(E + 1) / 2, NT, 0, (hipStream_t) stream>>>(NormIn{h, norm_w, eps, xn, (_Float16*) xh}, R, wt,
                                                                     E, logits);
    return HMOE_LAUNCHED("norm_router");
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
    HMOE_REQUIRE(wt && logits && sel && rw && E >= TOPK && E <= RMAXE && topk == TOPK && ((uintptr_t) wt & 15) == 0,
                 "decode_layer: router arguments");
    HMOE_REQUIRE(y || out, "decode_layer: no output");
    HMOE_REQUIRE(phases >= 1 && phases <= 31 && (phases & 15), "decode_layer: phases %d", phases);
    DecodeArgs a = forward_args(x, nullptr, nullptr, R, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, ctr_a,
                                y32, y, blocks, lo, sh_gw, sh_uw, sh_dw, HMOE_XF_BF16);
    a.wt = wt; a.bias = bias; a.logits = logits; a.E = E; a.topk = topk; a.scale = scale; a.sel_out = sel;
    a.rw_out = rw; a.out = out;
    int rc = check(a);
    if (rc) return rc;
    return run_decode(a, phases, (hipStream_t) stream);
}
