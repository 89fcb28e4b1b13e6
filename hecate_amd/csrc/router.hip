// router.hip - sigmoid + bias top-k router (runtime/core/exl3_router.py:21-146 router_fused; selection and weights as
// nr4_kernel.cuh:307-366) on gfx950, with fp32 logits in one fixed summation order so the selection is reproducible:
// logit = sum over 8 segments (in order, from 0) of [sum over the segment's 32-element chunks (in order, from 0) of
// a fmaf chain over the chunk's k ascending from 0].
//   small (R <= 16): a logits kernel (two experts per workgroup, one 32-element chunk per thread, chunk sums folded
//                    through LDS) and a select kernel (one wave per row); the kernel boundary replaces the reference's
//                    last-block counter (exl3_router.py:74-83,130), whose cross-workgroup fences are costly on gfx950.
//   large (R > 16) : a register-tiled fp32 GEMM per (64 rows, 64 experts, segment) with the same chain order, then a
//                    select kernel that folds the 8 segment sums and picks each row's top-k (one wave per row).
#include "hmoe_dev.h"

namespace hmoe {


// small path, 1: two experts per 512-thread workgroup, optional f16 copy of x; K = H through LDS (pair_logits),
// other K straight from global memory (expert_logits)
__global__ void __launch_bounds__(512) router_logits_h_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ wt, float* __restrict__ logits, int R, int E,
    _Float16* __restrict__ xh)
{
    pair_logits<false>(x, NormIn{}, wt, 2 * blockIdx.x, E, R, logits);
    if (xh)
    {
        const int n = R * H, per = (n + gridDim.x - 1) / gridDim.x, b0 = blockIdx.x * per;
        to_f16_range(x, xh, b0, min(n, b0 + per), threadIdx.x, blockDim.x);
    }
}

__global__ void __launch_bounds__(512) router_logits_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ wt, float* __restrict__ logits, int R, int K, int E,
    _Float16* __restrict__ xh)
{
    __shared__ float sums[2][256][MAXR + 1];
    const int half = threadIdx.x >> 8, tid = threadIdx.x & 255;
    expert_logits(x, wt, 2 * blockIdx.x + half, E, R, K, tid, sums[half], logits);
    if (xh)
    {
        const int n = R * K, per = (n + gridDim.x - 1) / gridDim.x, b0 = blockIdx.x * per;
        to_f16_range(x, xh, b0, min(n, b0 + per), threadIdx.x, blockDim.x);
    }
}

// small path, 2: one wave per row selects the top-k from the finished logits
__global__ void __launch_bounds__(1024) router_select_small_kernel(const float* __restrict__ logits,
    const float* __restrict__ bias, int R, int E, int topk, float scale, int64_t* __restrict__ sel,
    uint16_t* __restrict__ rw)
{
    const int r = threadIdx.x >> 6;
    if (r >= R) return;
    select_row(logits + (size_t) r * RMAXE, bias, E, topk, scale, sel + (size_t) r * topk, rw + (size_t) r * topk);
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
    // R <= MAXR: one logits row per row (the small path); more rows: the segment planes of the large path
    const size_t r = R > 0 ? (size_t) R : 1;
    return (R <= MAXR ? 1 : RSEG) * r * RMAXE * sizeof(float);
}

extern "C" int hmoe_router_fused(const void* x, const float* wt, const float* bias, float* logits, int* ctr,
                                 int64_t* sel, uint16_t* rw, int R, int K, int E, int topk, float scale, void* xh,
                                 void* stream)
{
    HMOE_REQUIRE(x && wt && logits && sel && rw, "router_fused: null buffer");
    (void) ctr;
    HMOE_REQUIRE(R >= 1 && E >= 1 && E <= RMAXE && topk >= 1 && topk <= TOPK && topk <= E,
                 "router_fused: rows %d experts %d topk %d", R, E, topk);
    HMOE_REQUIRE(K > 0 && K % (RCHUNK * RSEG) == 0 && K / RCHUNK <= 256, "router_fused: K %d", K);
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) wt & 15) == 0, "router_fused: x / wt not 16-byte aligned");
    hipStream_t st = (hipStream_t) stream;
    if (R <= MAXR)
    {
        if (K == H)
            router_logits_h_kernel<<<(E + 1) / 2, 512, 0, st>>>((const uint16_t*) x, wt, logits, R, E, (_Float16*) xh);
        else
            router_logits_kernel<<<(E + 1) / 2, 512, 0, st>>>((const uint16_t*) x, wt, logits, R, K, E, (_Float16*) xh);
        router_select_small_kernel<<<1, 1024, 0, st>>>(logits, bias, R, E, topk, scale, sel, rw);
        return HMOE_LAUNCHED("router_fused");
    }
    dim3 g((R + 63) / 64, (E + 63) / 64, RSEG);
    router_seg_kernel<<<g, 256, 0, st>>>((const uint16_t*) x, wt, logits, R, K, E);
    router_select_kernel<<<(R + 3) / 4, 256, 0, st>>>(logits, bias, R, E, topk, scale, sel, rw, (const uint16_t*) x,
                                                      (_Float16*) xh, K);
    return HMOE_LAUNCHED("router_fused");
}
