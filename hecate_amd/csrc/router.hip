// router.hip - sigmoid + bias top-k router (runtime/core/exl3_router.py:21-146 router_fused; selection and weights as
// nr4_kernel.cuh:307-366) on gfx950, with fp32 logits in one fixed summation order so the selection is reproducible:
// logit = sum over 8 segments (in order, from 0) of [sum over the segment's 32-element chunks (in order, from 0) of
// a fmaf chain over the chunk's k ascending from 0].
//   small (R <= 16): a logits kernel (two experts per workgroup, one 32-element chunk per thread, chunk sums folded
//                    through LDS) and a select kernel (one wave per row); the kernel boundary replaces the reference's
//                    last-block counter (exl3_router.py:74-83,130), whose cross-workgroup fences are costly on gfx950.
//   large (R > 16) : an fp32 MFMA GEMM per (128 rows, 64 experts, segment) with the same chain order, then a select
//                    kernel that folds the 8 segment sums and picks each row's top-k (one wave per row).
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
        const int nb = (E + 1) / 2, n = R * H, per = (n + nb - 1) / nb, b0 = blockIdx.x * per;   // (nb: the grid)
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
        const int nb = (E + 1) / 2, n = R * K, per = (n + nb - 1) / nb, b0 = blockIdx.x * per;   // (nb: the grid)
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

// large path, 1: the segment sums seg[s][r][e] on the matrix cores. v_mfma_f32_16x16x4f32 computes each output as a
// fmaf chain over its 4 k in order from the accumulator (measured bit-equal to that chain on every output of
// random, signed-zero and denormal operands), so a chunk's 32-element chain is 8 MFMAs from a zero accumulator, in the
// order of the small path and the oracle. Workgroup = 128 rows x 64 experts of one segment, 4 waves; wave w owns rows
// 32 w .. + 32 (2 row tiles) x the 64 experts (4 tiles): per 4-k step lane l reads A = x[row l % 16][k l / 16] and
// B = w[expert l % 16][k l / 16] from the k-major LDS chunk and holds D rows 4 (l / 16) .. + 4 of expert l % 16.
// A 32-k chunk of x (bf16 -> fp32) and of w is staged in LDS k-major (rows padded by 4 floats); the next chunk's
// global loads are in flight while this chunk computes (two buffers, one barrier per chunk).
constexpr int SM_R = 128, SM_E = 64, SM_XP = SM_R + 4, SM_WP = SM_E + 4;
__global__ void __launch_bounds__(256) router_seg_mfma_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ wt, float* __restrict__ seg, int R, int K, int E)
{
    constexpr int WJ = 2;                                       // w loads (4 floats) per thread per chunk
    __shared__ __attribute__((aligned(16))) float xs[2][RCHUNK][SM_XP];
    __shared__ __attribute__((aligned(16))) float ws[2][RCHUNK][SM_WP];
    const int r0 = blockIdx.x * SM_R, e0 = blockIdx.y * SM_E, s = blockIdx.z;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int segk = K / RSEG, k0 = s * segk, nch = segk / RCHUNK;
    const int sr = t & 127, sh = t >> 7, se = t % SM_E, seh = t / SM_E;
    const bool xin = r0 + sr < R, win = e0 + se < E;
    const uint16_t* xp = x + (size_t) (xin ? r0 + sr : 0) * K + k0;
    const float* wp = wt + (size_t) (win ? e0 + se : 0) * K + k0;
    u32x4 gx[2];
    f32x4 gw[WJ];
    auto load = [&](int c) {
        #pragma unroll
        for (int h = 0; h < 2; ++h) gx[h] = *(const u32x4*) (xp + c * RCHUNK + 8 * (sh + 2 * h));
        #pragma unroll
        for (int j = 0; j < WJ; ++j) gw[j] = *(const f32x4*) (wp + c * RCHUNK + 4 * (seh + 4 * j));
    };
    auto store = [&](int b) {
        #pragma unroll
        for (int h = 0; h < 2; ++h)
            #pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const int k = 8 * (sh + 2 * h) + 2 * q;
                xs[b][k][sr] = xin ? __uint_as_float(gx[h][q] << 16) : 0.f;
                xs[b][k + 1][sr] = xin ? __uint_as_float(gx[h][q] & 0xffff0000u) : 0.f;
            }
        #pragma unroll
        for (int j = 0; j < WJ; ++j)
            #pragma unroll
            for (int q = 0; q < 4; ++q) ws[b][4 * (seh + 4 * j) + q][se] = win ? gw[j][q] : 0.f;
    };
    f32x4 tot[2][4];
    #pragma unroll
    for (int i = 0; i < 2; ++i)
        #pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = (f32x4) {0.f, 0.f, 0.f, 0.f};
    load(0);
    store(0);
    __syncthreads();
    const int ar = 32 * w + (l & 15), kl = l >> 4;
    for (int c = 0; c < nch; ++c)
    {
        const int b = c & 1;
        if (c + 1 < nch) load(c + 1);
        f32x4 d[2][4];
        #pragma unroll
        for (int kk = 0; kk < RCHUNK / 4; ++kk)
        {
            const int k = 4 * kk + kl;
            float a[2], bv[4];
            #pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = xs[b][k][ar + 16 * i];
            #pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = ws[b][k][16 * j + (l & 15)];
            #pragma unroll
            for (int i = 0; i < 2; ++i)
                #pragma unroll
                for (int j = 0; j < 4; ++j)
                    d[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], bv[j],
                                                                   kk == 0 ? (f32x4) {0.f, 0.f, 0.f, 0.f} : d[i][j],
                                                                   0, 0, 0);
        }
        #pragma unroll
        for (int i = 0; i < 2; ++i)
            #pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][j] = tot[i][j] + d[i][j];
        if (c + 1 < nch) store(b ^ 1);
        __syncthreads();
    }
    #pragma unroll
    for (int i = 0; i < 2; ++i)
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const int r = r0 + 32 * w + 16 * i + 4 * (l >> 4) + q;
            if (r >= R) continue;
            #pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const int e = e0 + 16 * j + (l & 15);
                if (e < E) seg[((size_t) s * R + r) * RMAXE + e] = tot[i][j][q];
            }
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

int router_select_small(const float* logits, const float* bias, int R, int E, int topk, float scale, int64_t* sel,
                        uint16_t* rw, hipStream_t st)
{
    router_select_small_kernel<<<1, 1024, 0, st>>>(logits, bias, R, E, topk, scale, sel, rw);
    return HMOE_LAUNCHED("router select");
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
        if (int rc = HMOE_LAUNCHED("router_fused")) return rc;
        return router_select_small(logits, bias, R, E, topk, scale, sel, rw, st);
    }
    // 128 experts per workgroup from 4096 rows (the 8 x 8 tiles are faster at 8192 rows, -115 us); fewer rows take 64
    // experts per workgroup, so that the grid still fills the CUs twice over
    router_seg_mfma_kernel<<<dim3((R + SM_R - 1) / SM_R, (E + SM_E - 1) / SM_E, RSEG), 256, 0, st>>>(
            (const uint16_t*) x, wt, logits, R, K, E);
    router_select_kernel<<<(R + 3) / 4, 256, 0, st>>>(logits, bias, R, E, topk, scale, sel, rw, (const uint16_t*) x,
                                                      (_Float16*) xh, K);
    return HMOE_LAUNCHED("router_fused");
}
