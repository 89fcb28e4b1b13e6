// norm.hip - residual + RMSNorm on gfx950 in the reduction order of the reference's rms_norm_kernel (hmoe_dev.h
// half_wave_sum / rms_factor): the MoE combine fused into the next input norm (runtime/tier/cn.cu:48-103,189-235
// combine_norm), the post-attention norm + router (runtime/core/exl3_normroute.py:16-65, nr4_kernel.cuh:122-381
// norm_route), the decode stack's output launch fused with the next layer's norm, and the plain residual + RMSNorm.
//
// One 1024-thread workgroup per row, thread t owning float4 columns t and t + 1024 (t < 512), as rms_norm_kernel and
// cn.cu:61-66 lay them out, so the 1024 chains, both butterflies and therefore r and xn are the reference's bits up
// to the rsqrt (the reference's is fast math; here 1 / sqrt, correctly rounded).
#include "cputier_dev.h"

namespace hmoe {

// how the row's residual is updated before the norm
enum { CN_COMBINE = 0,   // a = ((f + y) + o) + o2 (f NULL reads as +0, cn.cu:105-110), y zeroed, r = a + r
       CN_ADD = 1,       // r = y + r, y zeroed (y NULL: r as it is)
       CN_ROUTE = 2,     // r = y + r, y read only (nr4_kernel.cuh:176-186: the attention output and the residual)
       CN_PARTS = 3 };   // r = s + r, s = the decode down launch's parts summed in part order (dec_d_kernel's sum)
enum { WT_F32 = HMOE_DT_F32, WT_BF16 = HMOE_DT_BF16, WT_F16 = HMOE_DT_F16 };

struct CnArgs
{
    const float* f; const float* o; float* y; const float* o2;
    const float* y32; const int* nparts;
    float* r; const void* w; void* xn; _Float16* xh;
    float eps, cbias, cscale;
    hmoe_cpu_mailbox* cmb;      // CN_COMBINE: the CPU tier's mailbox (device address) whose partial is o2, or NULL
    long long ticks;            // the bound of the wait for it
};

template <int WDT>
__device__ __forceinline__ f32x4 load_w4(const void* w, int c)
{
    if constexpr (WDT == WT_F32) return *(const f32x4*) ((const float*) w + 4 * c);
    const u32x2 u = *(const u32x2*) ((const uint16_t*) w + 4 * c);
    f32x4 o;
    #pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        const uint16_t b = (uint16_t) (u[e >> 1] >> (16 * (e & 1)));
        o[e] = WDT == WT_BF16 ? bf2f(b) : (float) __builtin_bit_cast(_Float16, b);
    }
    return o;
}

template <int MODE, int WDT, int XDT>
__global__ void __launch_bounds__(1024) cn_kernel(CnArgs p)
{
    __shared__ float gs[32];
    __shared__ int cpu_ok;
    const int t = threadIdx.x, row = blockIdx.x;
    const size_t ro = (size_t) row * H;
    const bool hb = t + 1024 < H / 4;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 x[2] = {z, z};
    int np = 0;
    if (MODE == CN_PARTS) np = min(max(*p.nparts, 0), MAX_PARTS);
    // the norm weights of both column halves, in flight while the residual is formed (a thread with one half reads its
    // first twice)
    f32x4 w4[2];
    #pragma unroll
    for (int k = 0; k < 2; ++k) w4[k] = load_w4<WDT>(p.w, hb ? t + 1024 * k : t);
    // with the CPU tier: its partial is o2, once the job the norm + router posted has finished (cn.cu:114-119 waits for
    // CPU_DONE the same way); when the wait runs out, or no job of this step was posted, nothing is added for it
    const float* o2 = p.o2;
    if (MODE == CN_COMBINE && p.cmb)
    {
        if (t == 0) cpu_ok = collect_ready(p.cmb, p.ticks);
        __syncthreads();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        o2 = cpu_ok ? p.cmb->out : nullptr;
    }
    if constexpr (MODE == CN_PARTS)
    {
        // the parts of both column halves are loaded in one batch of up to 8 once the part count is in (a part past
        // the count moves no bytes: one CU per row reads all of them), then added in part order from 0 (dec_d_kernel's
        // sum); counts past 8 take further batches
        constexpr size_t PS = (size_t) MAXR * H;
        const size_t ih[2] = {ro + 4 * (size_t) t, ro + 4 * (size_t) (t + 1024)};
        f32x4 rr[2] = {z, z}, a[2] = {z, z};
        for (int q0 = 0; q0 < np || q0 == 0; q0 += 8)
        {
            f32x4 pv[2][8];
            #pragma unroll
            for (int k = 0; k < 2; ++k)
            {
                if (k && !hb) break;
                if (q0 == 0) rr[k] = *(const f32x4*) (p.r + ih[k]);
                #pragma unroll
                for (int j = 0; j < 8; ++j)
                    pv[k][j] = q0 + j < np ? *(const f32x4*) (p.y32 + (q0 + j) * PS + ih[k]) : z;
            }
            #pragma unroll
            for (int k = 0; k < 2; ++k)
            {
                if (k && !hb) break;
                #pragma unroll
                for (int j = 0; j < 8; ++j) a[k] = q0 + j < np ? a[k] + pv[k][j] : a[k];
            }
        }
        #pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            if (k && !hb) break;
            x[k] = a[k] + rr[k];
            *(f32x4*) (p.r + ih[k]) = x[k];
        }
    }
    else
    {
        #pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            if (k && !hb) break;
            const size_t i = ro + 4 * (size_t) (t + 1024 * k);
            const f32x4 rr = *(const f32x4*) (p.r + i);
            f32x4 a;
            if (MODE == CN_COMBINE)
            {
                a = p.f ? *(const f32x4*) (p.f + i) : z;
                a += *(const f32x4*) (p.y + i);
                if (p.o) a += *(const f32x4*) (p.o + i);
                if (o2) a += *(const f32x4*) (o2 + i);
                *(f32x4*) (p.y + i) = z;
                x[k] = a + rr;
            }
            else
            {
                if (p.y)
                {
                    x[k] = *(const f32x4*) (p.y + i) + rr;
                    if (MODE == CN_ADD) *(f32x4*) (p.y + i) = z;
                }
                else x[k] = rr;
            }
            *(f32x4*) (p.r + i) = x[k];
        }
    }
    float s = chain4(0.f, x[0]);
    if (hb) s = chain4(s, x[1]);
    s = half_wave_sum(s);
    if ((t & 31) == 0) gs[t >> 5] = s;
    __syncthreads();
    const float rmf = rms_factor(half_wave_sum(gs[t & 31]), p.eps, p.cscale);
    #pragma unroll
    for (int k = 0; k < 2; ++k)
    {
        if (k && !hb) break;
        const int c = t + 1024 * k;
        f32x4 wk = w4[k];
        if (p.cbias != 0.f) wk += p.cbias;
        u32x2 o;
        f16x4 oh;
        #pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            const float v = (x[k][e] * wk[e]) * rmf;
            const uint16_t b = XDT == WT_BF16 ? hmoe_f2bf(v) : hmoe_f2h(v);
            if (e & 1) o[e >> 1] |= (uint32_t) b << 16; else o[e >> 1] = b;
            oh[e] = XDT == WT_BF16 ? (_Float16) bf2f(b) : __builtin_bit_cast(_Float16, b);
        }
        *(u32x2*) ((uint16_t*) p.xn + ro + 4 * c) = o;
        if (p.xh) *(f16x4*) (p.xh + ro + 4 * c) = oh;
    }
}

template <int MODE>
static int launch_cn(const CnArgs& a, int rows, int wdt, int xdt, hipStream_t st)
{
    auto pick = [&](auto wc, auto xc) {
        cn_kernel<MODE, decltype(wc)::value, decltype(xc)::value><<<rows, 1024, 0, st>>>(a);
    };
    const bool xb = xdt == WT_BF16;
    if (wdt == WT_F32) { if (xb) pick(ic<WT_F32>{}, ic<WT_BF16>{}); else pick(ic<WT_F32>{}, ic<WT_F16>{}); }
    else if (wdt == WT_BF16) { if (xb) pick(ic<WT_BF16>{}, ic<WT_BF16>{}); else pick(ic<WT_BF16>{}, ic<WT_F16>{}); }
    else { if (xb) pick(ic<WT_F16>{}, ic<WT_BF16>{}); else pick(ic<WT_F16>{}, ic<WT_F16>{}); }
    return HMOE_LAUNCHED("cn_kernel");
}

static int check_norm(const char* what, const float* r, const void* w, const void* xn, int rows, int maxrows,
                      int wdt, int xdt)
{
    HMOE_REQUIRE(r && w && xn, "%s: null buffer", what);
    HMOE_REQUIRE(rows >= 1 && rows <= maxrows, "%s: rows %d not in [1, %d]", what, rows, maxrows);
    HMOE_REQUIRE(wdt == HMOE_DT_F32 || wdt == HMOE_DT_BF16 || wdt == HMOE_DT_F16, "%s: weight dtype %d", what, wdt);
    HMOE_REQUIRE(xdt == HMOE_DT_BF16 || xdt == HMOE_DT_F16, "%s: output dtype %d (bf16 or f16)", what, xdt);
    HMOE_REQUIRE(((uintptr_t) r & 15) == 0 && ((uintptr_t) w & (wdt == HMOE_DT_F32 ? 15 : 7)) == 0 &&
                 ((uintptr_t) xn & 7) == 0, "%s: alignment", what);
    return HMOE_OK;
}

// the norm + router's router on the normed rows: x2 bf16 or f16, gt fp32 or f16 (pair_logits, two experts per
// workgroup, the router_fused order)
template <bool XF16, bool WF16>
__global__ void __launch_bounds__(512) nr_logits_kernel(const uint16_t* __restrict__ x2, const void* __restrict__ gt,
                                                        float* __restrict__ logits, int R, int E)
{
    pair_logits<false, 2, XF16, WF16>(x2, NormIn{}, (const float*) gt, 2 * blockIdx.x, E, R, logits);
}

// the norm + router's selection with the CPU tier's hand-off folded in (nr4_kernel.cuh:360-378: the last leader writes
// the band slot's rows and routing, then releases ISSUE): one wave per row selects as router_select_small does, then
// the workgroup posts x2 (bf16) and the routing to the mailbox once the pool's previous job is done
__global__ void __launch_bounds__(1024) nr_select_post_kernel(const float* __restrict__ logits,
    const float* __restrict__ bias, int R, int E, int topk, float scale, int64_t* __restrict__ sel,
    uint16_t* __restrict__ rw, const uint16_t* __restrict__ x2, hmoe_cpu_mailbox* mb, int layer, long long ticks)
{
    __shared__ int ready;
    __shared__ uint32_t gen;
    if (threadIdx.x == 0) {
        uint32_t g;
        ready = post_begin(mb, ticks, g);
        gen = g;
    }
    const int r = threadIdx.x >> 6;
    if (r < R) select_row(logits + (size_t) r * RMAXE, bias, E, topk, scale, sel + (size_t) r * topk, rw + (size_t) r * topk);
    // (the rows' selections, stored by their waves, are seen by the whole workgroup past the barrier)
    __syncthreads();
    if (!ready) return;
    post_job(mb, (const uint4*) x2, (const uint4*) sel, (const uint4*) rw, R, layer, gen, 1024);
}

}  // namespace hmoe

using namespace hmoe;

extern "C" int hmoe_combine_norm(const float* f, const float* o, float* y, int rows, const float* o2,
                                 const unsigned* done, float* r, const void* w, void* xn, float eps, float cbias,
                                 float cscale, int w_dtype, int xn_dtype, void* stream)
{
    if (int rc = check_norm("combine_norm", r, w, xn, rows, 64, w_dtype, xn_dtype)) return rc;
    HMOE_REQUIRE(y, "combine_norm: null y");
    HMOE_REQUIRE(!done, "combine_norm: the cross-device DONE flag is not supported (the RTX band is not built)");
    HMOE_REQUIRE(((uintptr_t) f & 15) == 0 && ((uintptr_t) y & 15) == 0 && ((uintptr_t) o & 15) == 0 &&
                 ((uintptr_t) o2 & 15) == 0, "combine_norm: alignment");
    CnArgs a = {f, o, y, o2, nullptr, nullptr, r, w, xn, nullptr, eps, cbias, cscale, nullptr, 0};
    return launch_cn<CN_COMBINE>(a, rows, w_dtype, xn_dtype, (hipStream_t) stream);
}

extern "C" int hmoe_combine_norm_cpu(const float* f, const float* o, float* y, int rows, hmoe_cpu_mailbox* mb,
                                     float* r, const void* w, void* xn, float eps, float cbias, float cscale,
                                     int w_dtype, int xn_dtype, void* stream)
{
    if (int rc = check_norm("combine_norm_cpu", r, w, xn, rows, HMOE_CPU_MAXR, w_dtype, xn_dtype)) return rc;
    HMOE_REQUIRE(y && mb, "combine_norm_cpu: null y or mailbox");
    HMOE_REQUIRE(((uintptr_t) f & 15) == 0 && ((uintptr_t) y & 15) == 0 && ((uintptr_t) o & 15) == 0,
                 "combine_norm_cpu: alignment");
    hmoe_cpu_mailbox* d = nullptr;
    long long ticks = 0;
    if (int rc = cpu_mailbox_device(mb, &d, &ticks)) return rc;
    CnArgs a = {f, o, y, nullptr, nullptr, nullptr, r, w, xn, nullptr, eps, cbias, cscale, d, ticks};
    return launch_cn<CN_COMBINE>(a, rows, w_dtype, xn_dtype, (hipStream_t) stream);
}

extern "C" int hmoe_residual_rmsnorm(float* r, float* a, const float* w, int R, float eps, uint16_t* xn, uint16_t* xh,
                                     void* stream)
{
    if (int rc = check_norm("residual_rmsnorm", r, w, xn, R, 1 << 20, HMOE_DT_F32, HMOE_DT_BF16)) return rc;
    HMOE_REQUIRE(((uintptr_t) a & 15) == 0 && ((uintptr_t) xh & 7) == 0, "residual_rmsnorm: alignment");
    CnArgs c = {nullptr, nullptr, a, nullptr, nullptr, nullptr, r, w, xn, (_Float16*) xh, eps, 0.f, 1.f, nullptr, 0};
    return launch_cn<CN_ADD>(c, R, HMOE_DT_F32, HMOE_DT_BF16, (hipStream_t) stream);
}

extern "C" int hmoe_decode_combine_norm(const float* y32, const int* ctr_a, int R, float* r, const void* w, void* xn,
                                        void* xh, float eps, float cbias, float cscale, int w_dtype, int xn_dtype,
                                        void* stream)
{
    if (int rc = check_norm("decode_combine_norm", r, w, xn, R, MAXR, w_dtype, xn_dtype)) return rc;
    HMOE_REQUIRE(y32 && ctr_a && ((uintptr_t) y32 & 15) == 0 && ((uintptr_t) xh & 7) == 0,
                 "decode_combine_norm: arguments");
    CnArgs a = {nullptr, nullptr, nullptr, nullptr, y32, ctr_a, r, w, xn, (_Float16*) xh, eps, cbias, cscale};
    return launch_cn<CN_PARTS>(a, R, w_dtype, xn_dtype, (hipStream_t) stream);
}

extern "C" size_t hmoe_norm_route_scratch_bytes(int R, int E)
{
    (void) E;
    return (size_t) (R > 0 ? R : 1) * RMAXE * sizeof(float);
}

extern "C" int hmoe_norm_route(const float* y, float* r, const void* w, void* x2, const void* gt, const float* bias,
                               int64_t* sel, uint16_t* rw, float* cand, int* ctr, float scale, float eps, float cbias,
                               float cscale, const int64_t* ho, int n_ho, int R, int E, int w_dtype, int x2_dtype,
                               int gt_dtype, void* stream)
{
    (void) ctr;
    if (int rc = check_norm("norm_route", r, w, x2, R, MAXR, w_dtype, x2_dtype)) return rc;
    HMOE_REQUIRE(y && gt && sel && rw && cand, "norm_route: null buffer");
    HMOE_REQUIRE(E >= TOPK && E <= RMAXE, "norm_route: %d experts", E);
    HMOE_REQUIRE(gt_dtype == HMOE_DT_F32 || gt_dtype == HMOE_DT_F16, "norm_route: gate dtype %d (fp32 or f16)",
                 gt_dtype);
    HMOE_REQUIRE(((uintptr_t) y & 15) == 0 && ((uintptr_t) gt & 15) == 0 && ((uintptr_t) x2 & 15) == 0,
                 "norm_route: alignment");
    // the hand-off: none, or this build's CPU tier {mailbox, layer} (the reference's 10 / 11 words address its RTX and
    // Grace bands' slots, which are not built here)
    HMOE_REQUIRE(n_ho == 0 || (n_ho == 2 && ho), "norm_route: the hand-off ho must be empty or {mailbox, layer} (%d words)", n_ho);
    hmoe_cpu_mailbox* mb = nullptr;
    long long ticks = 0;
    int layer = 0;
    if (n_ho == 2)
    {
        HMOE_REQUIRE(ho[0] != 0 && ho[1] >= 0 && ho[1] <= INT32_MAX, "norm_route: hand-off mailbox / layer");
        HMOE_REQUIRE(x2_dtype == HMOE_DT_BF16 && R <= HMOE_CPU_MAXR, "norm_route: the CPU tier's hand-off takes bf16 x2 "
                     "and at most %d rows (%d)", HMOE_CPU_MAXR, R);
        HMOE_REQUIRE((((uintptr_t) sel | (uintptr_t) rw) & 15) == 0, "norm_route: sel / rw not 16-byte aligned");
        if (int rc = cpu_mailbox_device((hmoe_cpu_mailbox*) (uintptr_t) ho[0], &mb, &ticks)) return rc;
        layer = (int) ho[1];
    }
    hipStream_t st = (hipStream_t) stream;
    CnArgs a = {nullptr, nullptr, (float*) y, nullptr, nullptr, nullptr, r, w, x2, nullptr, eps, cbias, cscale};
    if (int rc = launch_cn<CN_ROUTE>(a, R, w_dtype, x2_dtype, st)) return rc;
    const bool xf16 = x2_dtype == HMOE_DT_F16, wf16 = gt_dtype == HMOE_DT_F16;
    const dim3 g((E + 1) / 2);
    if (xf16 && wf16) nr_logits_kernel<true, true><<<g, 512, 0, st>>>((const uint16_t*) x2, gt, cand, R, E);
    else if (xf16) nr_logits_kernel<true, false><<<g, 512, 0, st>>>((const uint16_t*) x2, gt, cand, R, E);
    else if (wf16) nr_logits_kernel<false, true><<<g, 512, 0, st>>>((const uint16_t*) x2, gt, cand, R, E);
    else nr_logits_kernel<false, false><<<g, 512, 0, st>>>((const uint16_t*) x2, gt, cand, R, E);
    if (int rc = HMOE_LAUNCHED("norm_route logits")) return rc;
    if (!mb) return router_select_small(cand, bias, R, E, TOPK, scale, sel, rw, st);
    nr_select_post_kernel<<<1, 1024, 0, st>>>(cand, bias, R, E, TOPK, scale, sel, rw, (const uint16_t*) x2, mb, layer,
                                              ticks);
    return HMOE_LAUNCHED("norm_route select + hand-off");
}
