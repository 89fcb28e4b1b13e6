// router.hip - sigmoid + bias top-k router (runtime/core/exl3_router.py:21-146 router_fused; selection and weights as
// nr4_kernel.cuh:307-366) on gfx950, with fp32 logits in one fixed summation order so the selection is reproducible:
// logit = sum over 8 segments (in order, from 0) of [sum over the segment's 32-element chunks (in order, from 0) of
// a fmaf chain over the chunk's k ascending from 0].
//   small (R <= 16): one launch. Workgroup e computes expert e's logits for every row, one chunk per thread; the
//                    chunk sums fold through LDS; the last workgroup to finish (self-resetting counter, as
//                    exl3_router.py:74-83,130) selects each row's top-k and writes sel / rw.
//   large (R > 16) : a register-tiled fp32 GEMM per (64 rows, 64 experts, segment) with the same chain order, then a
//                    select kernel that folds the 8 segment sums and picks each row's top-k (one wave per row).
#include "hmoe_dev.h"

namespace hmoe {

constexpr int RCHUNK = 32, RSEG = 8, RMAXE = 256;

// top-k of one row by a wave: keys of experts lane + 64 i; each round takes the largest (key, -index) pair, so ties
// go to the lowest index (exl3_router.py:106-121); the sum runs over the selected unbiased activations in order
__device__ void select_row(const float* __restrict__ lg, const float* __restrict__ bias, int E, int topk, float scale,
                           int64_t* __restrict__ sel, uint16_t* __restrict__ rw)
{
    const int lane = threadIdx.x & 63;
    float a[4]; uint32_t key[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = lane + 64 * i;
        if (e < E)
        {
            a[i] = hmoe_sigmoid(lg[e]);
            key[i] = hmoe_okey(a[i] + (bias ? bias[e] : 0.0f));
        }
        else { a[i] = 0.f; key[i] = 0u; }
    }
    float sum = 0.f, wsel = 0.f; int isel = 0;
    for (int k = 0; k < topk; ++k)
    {
        uint64_t best = 0ull;
        #pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const uint64_t v = ((uint64_t) key[i] << 32) | (uint32_t) (0xffffu - (lane + 64 * i));
            best = v > best ? v : best;
        }
        #pragma unroll
        for (int off = 32; off > 0; off >>= 1)
        {
            const uint32_t lo = __shfl_xor((uint32_t) best, off), hi = __shfl_xor((uint32_t) (best >> 32), off);
            const uint64_t o = ((uint64_t) hi << 32) | lo;
            best = o > best ? o : best;
        }
        const int e = 0xffff - (int) (best & 0xffffu);
        float mine = 0.f;
        if ((e & 63) == lane)
        {
            #pragma unroll
            for (int i = 0; i < 4; ++i) if (i == (e >> 6)) { mine = a[i]; key[i] = 0u; }
        }
        const float av = __shfl(mine, e & 63);
        sum = sum + av;
        if (lane == k) { wsel = av; isel = e; }
    }
    if (lane < topk)
    {
        sel[lane] = isel;
        rw[lane] = hmoe_f2h((wsel * scale) / (sum + 1e-20f));
    }
}

// small path: blockIdx.x = expert, thread c = chunk (K / 32 chunks <= blockDim), every row
__global__ void __launch_bounds__(256) router_small_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ wt, const float* __restrict__ bias,
    float* __restrict__ logits, int* __restrict__ ctr, int64_t* __restrict__ sel, uint16_t* __restrict__ rw, int R,
    int K, int E, int topk, float scale, _Float16* __restrict__ xh)
{
    __shared__ float sums[256][MAXR + 1];
    __shared__ int s_last;
    const int e = blockIdx.x, c = threadIdx.x, nch = K / RCHUNK;
    if (c < nch)
    {
        const float* w = wt + (size_t) e * K + c * RCHUNK;
        float wv[RCHUNK];
        #pragma unroll
        for (int i = 0; i < RCHUNK; i += 4) { const f32x4 v = *(const f32x4*) (w + i); wv[i] = v[0]; wv[i + 1] = v[1]; wv[i + 2] = v[2]; wv[i + 3] = v[3]; }
        for (int r = 0; r < R; ++r)
        {
            const uint16_t* xr = x + (size_t) r * K + c * RCHUNK;
            float acc = 0.f;
            #pragma unroll
            for (int i = 0; i < RCHUNK; i += 8)
            {
                const u32x4 v = *(const u32x4*) (xr + i);
                #pragma unroll
                for (int k = 0; k < 4; ++k)
                {
                    acc = __builtin_fmaf(__uint_as_float(v[k] << 16), wv[i + 2 * k], acc);
                    acc = __builtin_fmaf(__uint_as_float(v[k] & 0xffff0000u), wv[i + 2 * k + 1], acc);
                }
            }
            sums[c][r] = acc;
        }
    }
    // the f16 copy of x for the decode kernels: this workgroup's slice
    if (xh)
    {
        const int n = R * K, per = (n + gridDim.x - 1) / gridDim.x, b0 = e * per, b1 = min(n, b0 + per);
        for (int i = b0 + c; i < b1; i += blockDim.x) xh[i] = (_Float16) bf2f(x[i]);
    }
    __syncthreads();
    if (c < R)
    {
        const int cps = nch / RSEG;
        float t = 0.f;
        for (int s = 0; s < RSEG; ++s)
        {
            float seg = 0.f;
            for (int q = s * cps; q < (s + 1) * cps; ++q) seg = seg + sums[q][c];
            t = t + seg;
        }
        logits[(size_t) c * RMAXE + e] = t;
    }
    __threadfence();
    __syncthreads();
    if (c == 0) s_last = atomicAdd(ctr, 1) == (int) gridDim.x - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int wave = c >> 6, nw = blockDim.x >> 6;
    for (int r = wave; r < R; r += nw)
    {
        float* lg = logits + (size_t) r * RMAXE;
        // coherent reads of the other workgroups' logits
        __shared__ float lrow[4][RMAXE];
        for (int i = c & 63; i < E; i += 64) lrow[wave][i] = __hip_atomic_load(lg + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        select_row(lrow[wave], bias, E, topk, scale, sel + (size_t) r * topk, rw + (size_t) r * topk);
    }
    if (c == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// large path, 1: segment sums seg[s][r][e] for a 64-row x 64-expert tile, 4 x 4 outputs per thread
__global__ void __launch_bounds__(256) router_seg_kernel(const uint16_t* __restrict__ x, const float* __restrict__ wt,
                                                         float* __restrict__ seg, int R, int K, int E)
{
    __shared__ float xs[64][RCHUNK + 1];
    __shared__ float ws[64][RCHUNK + 1];
    const int r0 = blockIdx.x * 64, e0 = blockIdx.y * 64, s = blockIdx.z;
    const int t = threadIdx.x, ty = t >> 4, tx = t & 15;
    const int segk = K / RSEG, k0 = s * segk;
    float acc[4][4], tot[4][4];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
        #pragma unroll
        for (int j = 0; j < 4; ++j) { acc[i][j] = 0.f; tot[i][j] = 0.f; }
    for (int c = k0; c < k0 + segk; c += RCHUNK)
    {
        // stage 64 x 32 of x (bf16 -> fp32) and of w: 2048 values each, 8 per thread
        {
            const int rr = t >> 2, kk = (t & 3) * 8;
            const int gr = r0 + rr, ge = e0 + rr;
            if (gr < R)
            {
                const u32x4 v = *(const u32x4*) (x + (size_t) gr * K + c + kk);
                #pragma unroll
                for (int q = 0; q < 4; ++q) { xs[rr][kk + 2 * q] = __uint_as_float(v[q] << 16); xs[rr][kk + 2 * q + 1] = __uint_as_float(v[q] & 0xffff0000u); }
            }
            else
            {
                #pragma unroll
                for (int q = 0; q < 8; ++q) xs[rr][kk + q] = 0.f;
            }
            if (ge < E)
            {
                const f32x4 a = *(const f32x4*) (wt + (size_t) ge * K + c + kk), b = *(const f32x4*) (wt + (size_t) ge * K + c + kk + 4);
                #pragma unroll
                for (int q = 0; q < 4; ++q) { ws[rr][kk + q] = a[q]; ws[rr][kk + 4 + q] = b[q]; }
            }
            else
            {
                #pragma unroll
                for (int q = 0; q < 8; ++q) ws[rr][kk + q] = 0.f;
            }
        }
        __syncthreads();
        #pragma unroll 8
        for (int k = 0; k < RCHUNK; ++k)
        {
            float xv[4], wv[4];
            #pragma unroll
            for (int i = 0; i < 4; ++i) { xv[i] = xs[ty + 16 * i][k]; wv[i] = ws[tx + 16 * i][k]; }
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                #pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(xv[i], wv[j], acc[i][j]);
        }
        #pragma unroll
        for (int i = 0; i < 4; ++i)
            #pragma unroll
            for (int j = 0; j < 4; ++j) { tot[i][j] = tot[i][j] + acc[i][j]; acc[i][j] = 0.f; }
        __syncthreads();
    }
    #pragma unroll
    for (int i = 0; i < 4; ++i)
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int r = r0 + ty + 16 * i, e = e0 + tx + 16 * j;
            if (r < R && e < E) seg[((size_t) s * R + r) * RMAXE + e] = tot[i][j];
        }
}

// large path, 2: fold the segments in order, select; one wave per row; optional f16 copy of x
__global__ void __launch_bounds__(256) router_select_kernel(const float* __restrict__ seg, const float* __restrict__ bias,
    int R, int E, int topk, float scale, int64_t* __restrict__ sel, uint16_t* __restrict__ rw,
    const uint16_t* __restrict__ x, _Float16* __restrict__ xh, int K)
{
    __shared__ float lrow[4][RMAXE];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= R) return;
    for (int e = lane; e < E; e += 64)
    {
        float t = 0.f;
        for (int s = 0; s < RSEG; ++s) t = t + seg[((size_t) s * R + r) * RMAXE + e];
        lrow[wave][e] = t;
    }
    select_row(lrow[wave], bias, E, topk, scale, sel + (size_t) r * topk, rw + (size_t) r * topk);
    if (xh)
        for (int k = lane * 8; k < K; k += 64 * 8)
        {
            const u32x4 v = *(const u32x4*) (x + (size_t) r * K + k);
            f16x8 o;
            #pragma unroll
            for (int q = 0; q < 4; ++q) { o[2 * q] = (_Float16) __uint_as_float(v[q] << 16); o[2 * q + 1] = (_Float16) __uint_as_float(v[q] & 0xffff0000u); }
            *(f16x8*) (xh + (size_t) r * K + k) = o;
        }
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_router_scratch_bytes(int R, int E)
{
    (void) E;
    return (size_t) RSEG * (size_t) (R > 0 ? R : 1) * RMAXE * sizeof(float);
}

extern "C" int hmoe_router_fused(const void* x, const float* wt, const float* bias, float* logits, int* ctr,
                                 int64_t* sel, uint16_t* rw, int R, int K, int E, int topk, float scale, void* xh,
                                 void* stream)
{
    HMOE_REQUIRE(x && wt && logits && ctr && sel && rw, "router_fused: null buffer");
    HMOE_REQUIRE(R >= 1 && E >= 1 && E <= RMAXE && topk >= 1 && topk <= TOPK && topk <= E,
                 "router_fused: rows %d experts %d topk %d", R, E, topk);
    HMOE_REQUIRE(K > 0 && K % (RCHUNK * RSEG) == 0 && K / RCHUNK <= 256, "router_fused: K %d", K);
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) wt & 15) == 0, "router_fused: x / wt not 16-byte aligned");
    hipStream_t st = (hipStream_t) stream;
    if (R <= MAXR)
    {
        router_small_kernel<<<E, 256, 0, st>>>((const uint16_t*) x, wt, bias, logits, ctr, sel, rw, R, K, E, topk, scale,
                                               (_Float16*) xh);
        return HMOE_LAUNCHED("router_fused");
    }
    dim3 g((R + 63) / 64, (E + 63) / 64, RSEG);
    router_seg_kernel<<<g, 256, 0, st>>>((const uint16_t*) x, wt, logits, R, K, E);
    router_select_kernel<<<(R + 3) / 4, 256, 0, st>>>(logits, bias, R, E, topk, scale, sel, rw, (const uint16_t*) x,
                                                      (_Float16*) xh, K);
    return HMOE_LAUNCHED("router_fused");
}
