// hmoe_dev.h - gfx950 device helpers shared by the kernels of libhecate_moe.so: fragment types, the int4 -> f16
// decode of the I4G128 layout, MFMA wrappers, conversions, error plumbing of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/hecate_moe.h"
#include "../../include/hmoe_rng.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace hmoe {

constexpr int H = HMOE_H, I = HMOE_I, TOPK = HMOE_TOPK, MAXR = HMOE_MAXR, MAXSLOT = HMOE_MAXSLOT;
constexpr int SH_SLOT = MAXSLOT;            // act slot of the shared expert
constexpr int SHP_SLOT = MAXSLOT + 1;       // the shared expert's fp32 gate and up sums [2][MAXR][I] (4 slots' room)
constexpr int REC_SLOT = SHP_SLOT + 4;      // the gate/up launch's routing record for the down launch (int words)
constexpr int ACT_SLOTS = REC_SLOT + 1;
constexpr int MAX_PARTS = 1 + MAXSLOT / 4;  // the decode down launch's part partials: the shared expert's, one per slot quad
constexpr int REC_E = 64;                   // record: word 0 = distinct experts m, words REC_E + j (j < MAXSLOT) = local
                                            // id of slot j (0 past m) | m << 16, so every lane's word carries m

// I4G128 group scales: 128-byte blocks of 16 rows x 4 k groups; the index (in bf16 units) of row n's scale of group g
// (KG = K / 128 groups, a multiple of 4)
__host__ __device__ __forceinline__ size_t sc_index(int n, int g, int KG)
{
    return ((size_t) (n >> 4) * (KG >> 2) + (g >> 2)) * 64 + (n & 15) * 4 + (g & 3);
}

// ---- error state of the C ABI (common.hip) ----
int set_error(int code, const char* fmt, ...);
// the prefill shared expert (shared_gemm.hip), f16 row-major operands: act [T][I] = f16(silu(wg x) (wu x)), and
// out [T][H] = wd act (fp32, written or, with add, added into)
int dense_gate_up(const _Float16* wg, const _Float16* wu, const _Float16* x, int T, _Float16* act, hipStream_t st);
// the shared expert's down projection over T tokens: out rows [T][H] stored as f16 (DG_MODE_F16) or added into fp32
// (DG_MODE_ADD)
enum { DG_MODE_F16 = 0, DG_MODE_ADD = 1 };
int dense_down(const _Float16* wd, const _Float16* act, int T, void* out, int mode, hipStream_t st);
int hip_check(hipError_t e, const char* what);
// the router's select launch for R <= MAXR rows of finished logits [R][RMAXE] (router.hip): one wave per row
int router_select_small(const float* logits, const float* bias, int R, int E, int topk, float scale, int64_t* sel,
                        uint16_t* rw, hipStream_t st);
#define HMOE_REQUIRE(cond, ...) do { if (!(cond)) return ::hmoe::set_error(HMOE_ERR_ARG, __VA_ARGS__); } while (0)
#define HMOE_LAUNCHED(what) ::hmoe::hip_check(hipGetLastError(), what)

// ---- compile-time loop: f(ic<0>{}), ..., f(ic<N-1>{}) (register arrays indexed by a constant stay in registers) ----
template <int V> struct ic { static constexpr int value = V; };
template <int N, int K = 0, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (K < N) { f(ic<K>{}); static_for<N, K + 1>(f); }
}

// ---- conversions ----
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t) b << 16); }

// 8 codes of one I4G128 dword -> 8 exact f16 values q = code - 8, element e of the MFMA operand at nibble bit
// 4(e/2) + 16(e%2): (code | 0x6400) is the f16 1024 + code (0x6400 = 1024, one unit per mantissa step), minus 1032;
// the odd nibble of each byte lands 4 bits up, 1024 + 16 code, scaled by 1/16 and offset by -72 (all exact).
// The two masks and the exponent live in registers made once per kernel (dq_consts): (w & mask) | 0x6400.. is then
// one v_and_or_b32 (a VOP3 of gfx9 takes no 32-bit literal; with literals it costs two instructions).
struct DqConsts { uint32_t m0, m1, mg; };
__device__ __forceinline__ DqConsts dq_consts()
{
    DqConsts c = {0x000f000fu, 0x00f000f0u, 0x64006400u};
    asm volatile("" : "+v"(c.m0), "+v"(c.m1), "+v"(c.mg));
    return c;
}

__device__ __forceinline__ f16x8 dq8(uint32_t w, const DqConsts& c)
{
    const uint32_t top = w >> 8;
    const f16x2 m1032 = {(_Float16) -1032.0f, (_Float16) -1032.0f};
    const f16x2 s16 = {(_Float16) 0.0625f, (_Float16) 0.0625f};
    const f16x2 m72 = {(_Float16) -72.0f, (_Float16) -72.0f};
    const f16x2 a0 = __builtin_bit_cast(f16x2, (w & c.m0) | c.mg) + m1032;
    const f16x2 a1 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w & c.m1) | c.mg), s16, m72);
    const f16x2 a2 = __builtin_bit_cast(f16x2, (top & c.m0) | c.mg) + m1032;
    const f16x2 a3 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (top & c.m1) | c.mg), s16, m72);
    f16x8 r;
    r[0] = a0[0]; r[1] = a0[1]; r[2] = a1[0]; r[3] = a1[1];
    r[4] = a2[0]; r[5] = a2[1]; r[6] = a3[0]; r[7] = a3[1];
    return r;
}

// dq8 times a per-row f16 scale pair {s, s}: f16((code - 8) * s) (exact codes, one rounding)
__device__ __forceinline__ f16x8 dq8s(uint32_t w, f16x2 ss, const DqConsts& c)
{
    const uint32_t top = w >> 8;
    const f16x2 m1032 = {(_Float16) -1032.0f, (_Float16) -1032.0f};
    const f16x2 s16 = {(_Float16) 0.0625f, (_Float16) 0.0625f};
    const f16x2 m72 = {(_Float16) -72.0f, (_Float16) -72.0f};
    const f16x2 a0 = (__builtin_bit_cast(f16x2, (w & c.m0) | c.mg) + m1032) * ss;
    const f16x2 a1 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (w & c.m1) | c.mg), s16, m72) * ss;
    const f16x2 a2 = (__builtin_bit_cast(f16x2, (top & c.m0) | c.mg) + m1032) * ss;
    const f16x2 a3 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (top & c.m1) | c.mg), s16, m72) * ss;
    f16x8 r;
    r[0] = a0[0]; r[1] = a0[1]; r[2] = a1[0]; r[3] = a1[1];
    r[4] = a2[0]; r[5] = a2[1]; r[6] = a3[0]; r[7] = a3[1];
    return r;
}

// D = A(16 x 32) * B(32 x 16) + C, f16 operands, fp32 accumulation. Lane l: A row l%16 (k slice 8(l/16)..+8),
// B column l%16 (same k slice), D rows 4(l/16)..+4 of column l%16.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// Loads from global memory through pointers the compiler cannot trace to a kernel argument (expert addresses read from
// a table): the explicit global address space makes them global_load. A generic pointer would give flat_load, which
// also counts against the LDS wait counter, so every LDS wait would drain the weight loads in flight. The pointer must
// address global memory: a generic pointer into LDS read this way is an illegal access.
#define HMOE_GLOBAL __attribute__((address_space(1)))
template <typename T> __device__ __forceinline__ T ldg(const void* p) { return *(const HMOE_GLOBAL T*) p; }
// weights read once: nontemporal (not kept in the caches)
__device__ __forceinline__ u32x4 ldw16(const void* p) { return __builtin_nontemporal_load((const HMOE_GLOBAL u32x4*) p); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return ldg<u32x4>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return ldg<u32x2>(p); }

// silu(g) = g / (1 + e^-g) with the hardware reciprocal (1 ulp) in place of a correctly rounded division: the result
// is rounded to f16 next, and the division's refinement sequence is ten VALU instructions per element
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// the inputs of one row's selection held by a lane: logits and bias of experts lane + 64 i (i < 4)
struct RowIn { float lg[4], b[4]; };

// from global memory, every load unconditional (index clamped to E - 1, the logits standing in for a NULL bias), so
// a kernel can issue them ahead of other loads and select later: the logits of a row, and the bias (raw: a select on
// the loaded value here would wait for it, and for every load issued before it, where it stands; bias_or_zero()
// applies the NULL bias where the selection needs the values anyway)
__device__ __forceinline__ void load_logits_global(const float* __restrict__ lg, int E, float (&out)[4])
{
    const int lane = threadIdx.x & 63;
    #pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = ldg<float>(lg + min(lane + 64 * i, E - 1));
}
__device__ __forceinline__ void load_bias_global(const float* __restrict__ bias, const float* __restrict__ lg, int E,
                                                 float (&out)[4])
{
    const int lane = threadIdx.x & 63;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = min(lane + 64 * i, E - 1);
        out[i] = ldg<float>(bias ? bias + e : lg + e);
    }
}
__device__ __forceinline__ void bias_or_zero(float (&b)[4], bool has_bias)
{
    #pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = has_bias ? b[i] : 0.0f;
}

// the wave's maximum (MAX) or minimum of a 32-bit value, returned from lane 63: quad, 8-lane and 16-lane butterflies,
// then the row broadcasts into rows 1, 3 and 2, 3 (gfx9 DPP: each step is one max / min whose first operand is read
// across lanes; a lane of a masked row keeps its value). Two wait states before each DPP read of a VGPR the previous
// VALU instruction wrote (the s_nop 1).
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext_u32(uint32_t v)
{
#define HMOE_DPP_STEPS(OP)                                                                                            \
    "s_nop 1\n\t" OP " %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"                                 \
    "s_nop 1\n\t" OP " %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"                                 \
    "s_nop 1\n\t" OP " %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"                                     \
    "s_nop 1\n\t" OP " %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf\n\t"                                          \
    "s_nop 1\n\t" OP " %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"                                        \
    "s_nop 1\n\t" OP " %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"                                        \
    "s_nop 1"
    if (MAX) asm volatile(HMOE_DPP_STEPS("v_max_u32_dpp") : "+v"(v));
    else asm volatile(HMOE_DPP_STEPS("v_min_u32_dpp") : "+v"(v));
#undef HMOE_DPP_STEPS
    return (uint32_t) __builtin_amdgcn_readlane((int) v, 63);
}

// top-k of one row by a wave (all 64 lanes active): keys of experts lane + 64 i; the selection is the one of taking
// the largest (key, -index) pair topk times, so ties go to the lowest index and sel is in descending key order
// (exl3_router.py:106-121); the sum runs over the selected unbiased activations in that order. Done as exactly that:
// each lane sorts its 4 (key, id) pairs (key descending, then id ascending), and each of topk rounds takes the wave's
// largest lane head (a DPP reduction; on an exact tie of keys the lowest id among the tied heads, by a second one)
// and pops it from its lane.
__device__ inline void select_from(const RowIn& in, int E, int topk, float scale, int64_t* __restrict__ sel,
                                   uint16_t* __restrict__ rw)
{
    const int lane = threadIdx.x & 63;
    uint32_t k[4], id[4];
    float a[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = lane + 64 * i;
        const bool ok = e < E;
        a[i] = ok ? hmoe_sigmoid(in.lg[i]) : 0.f;
        k[i] = ok ? hmoe_okey(a[i] + in.b[i]) : 0u;          // (a finite float's key is never 0)
        id[i] = (uint32_t) e;
    }
    // the lane's 4 pairs in selection order (a 5-comparator network; ids start ascending)
    auto cas = [&](int p, int q) {
        const bool sw = k[q] > k[p] || (k[q] == k[p] && id[q] < id[p]);
        const uint32_t tk = k[p], ti = id[p];
        const float ta = a[p];
        k[p] = sw ? k[q] : k[p]; id[p] = sw ? id[q] : id[p]; a[p] = sw ? a[q] : a[p];
        k[q] = sw ? tk : k[q]; id[q] = sw ? ti : id[q]; a[q] = sw ? ta : a[q];
    };
    cas(0, 1); cas(2, 3); cas(0, 2); cas(1, 3); cas(1, 2);
    // topk rounds; lane r of es / as receives the r-th pick's id and activation
    int es = 0;
    float as = 0.f;
    for (int r = 0; r < topk; ++r)
    {
        const uint32_t mk = wave_ext_u32<true>(k[0]);
        const uint64_t tie = __ballot(k[0] == mk);
        int wl = __builtin_ctzll(tie);                          // the lane of the winning head
        if (__popcll(tie) > 1)                                  // equal keys: the lowest id among the tied heads
            wl = (int) (wave_ext_u32<false>(k[0] == mk ? id[0] : 0xffffffffu) & 63u);
        const int ex = __builtin_amdgcn_readlane((int) id[0], wl);
        const float aw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[0]), wl));
        es = lane == r ? ex : es;
        as = lane == r ? aw : as;
        const bool win = lane == wl;
        k[0] = win ? k[1] : k[0]; id[0] = win ? id[1] : id[0]; a[0] = win ? a[1] : a[0];
        k[1] = win ? k[2] : k[1]; id[1] = win ? id[2] : id[1]; a[1] = win ? a[2] : a[1];
        k[2] = win ? k[3] : k[2]; id[2] = win ? id[3] : id[2]; a[2] = win ? a[3] : a[2];
        k[3] = win ? 0u : k[3];
    }
    // the unbiased sigmoids summed in selection order, from 0
    float sum = 0.f;
    for (int kk = 0; kk < topk; ++kk) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(as), kk));
    if (lane < topk)
    {
        sel[lane] = es;
        rw[lane] = hmoe_f2h((as * scale) / (sum + 1e-20f));
    }
}

// select_from on a row in LDS or global memory (generic loads)
__device__ inline void select_row(const float* __restrict__ lg, const float* __restrict__ bias, int E, int topk,
                                  float scale, int64_t* __restrict__ sel, uint16_t* __restrict__ rw)
{
    const int lane = threadIdx.x & 63;
    RowIn r;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = lane + 64 * i;
        r.lg[i] = e < E ? lg[e] : 0.f;
        r.b[i] = (e < E && bias) ? bias[e] : 0.0f;
    }
    select_from(r, E, topk, scale, sel, rw);
}


// ---- router logits, fixed order (see hecate_moe.h) ----
constexpr int RCHUNK = 32, RSEG = 8, RMAXE = 256;

// logits of expert e for R <= 16 rows by 256 threads (tid in [0, 256)): thread c computes the fmaf chain of chunk c
// for every row into sums[c][r]; after the workgroup barrier threads r < R fold the chunk sums in segment order and
// write logits[r * RMAXE + e]. Every thread of the workgroup must call it (it contains a barrier). e >= E: no-op.
__device__ inline void expert_logits(const uint16_t* __restrict__ x, const float* __restrict__ wt, int e, int E, int R,
                                     int K, int tid, float (*sums)[MAXR + 1], float* __restrict__ logits)
{
    const int nch = K / RCHUNK;
    if (e < E && tid < nch)
    {
        const float* w = wt + (size_t) e * K + tid * RCHUNK;
        float wv[RCHUNK];
        #pragma unroll
        for (int i = 0; i < RCHUNK; i += 4)
        {
            const f32x4 v = *(const f32x4*) (w + i);
            wv[i] = v[0]; wv[i + 1] = v[1]; wv[i + 2] = v[2]; wv[i + 3] = v[3];
        }
        for (int r = 0; r < R; ++r)
        {
            const uint16_t* xr = x + (size_t) r * K + tid * RCHUNK;
            u32x4 xv[4];
            #pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = *(const u32x4*) (xr + 8 * i);
            float acc = 0.f;
            #pragma unroll
            for (int i = 0; i < 4; ++i)
                #pragma unroll
                for (int k = 0; k < 4; ++k)
                {
                    acc = __builtin_fmaf(__uint_as_float(xv[i][k] << 16), wv[8 * i + 2 * k], acc);
                    acc = __builtin_fmaf(__uint_as_float(xv[i][k] & 0xffff0000u), wv[8 * i + 2 * k + 1], acc);
                }
            sums[tid][r] = acc;
        }
    }
    __syncthreads();
    if (e < E && tid < R)
    {
        const int cps = nch / RSEG;
        float t = 0.f;
        for (int s = 0; s < RSEG; ++s)
        {
            float seg = 0.f;
            for (int q = s * cps; q < (s + 1) * cps; ++q) seg = seg + sums[q][tid];
            t = t + seg;
        }
        logits[(size_t) tid * RMAXE + e] = t;
    }
}

// ---- RMSNorm in the reduction order of the reference's rms_norm_kernel (runtime/tier/cn.cu:21-31,80-103), which its
// fused kernels keep bit for bit (nr4_kernel.cuh:4-9): a row of H = 6144 is 1536 float4 columns; chain t (t < 1024)
// is one fmaf chain from 0 over columns t and t + 1024 (the latter for t < 512), element by element; reduce_1024:
// an xor butterfly within each group of 32 chains (offsets 16 .. 1), then the same butterfly over the 32 group sums.
// On gfx950 a group of 32 is a half-wave, so both butterflies run in registers; every lane of a half-wave ends with its
// group's sum (fp32 addition commutes, so the two partners of each step compute the same value).
__device__ __forceinline__ float half_wave_sum(float v)
{
    #pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float chain4(float p, f32x4 v)
{
    p = __builtin_fmaf(v[0], v[0], p); p = __builtin_fmaf(v[1], v[1], p);
    p = __builtin_fmaf(v[2], v[2], p); p = __builtin_fmaf(v[3], v[3], p);
    return p;
}
// rmf = 1 / sqrt(sum / H + eps) * cscale (the reference's rsqrtf, fast math there, as the correctly rounded 1 / sqrt)
__device__ __forceinline__ float rms_factor(float sum, float eps, float cscale)
{
    return (1.0f / __builtin_sqrtf(sum / (float) H + eps)) * cscale;
}

// The fused input path of the router (nr4_kernel.cuh:122-381: RMSNorm + router in one launch): the residual h fp32
// [R][H] and the norm weight w; xn = bf16((h * w) * rmf), rmf from the rms_norm_kernel order above, so xn is
// bit-identical to the residual + RMSNorm kernel's. Each workgroup writes its slice of xn (and of xh, the f16 copy,
// when not NULL).
struct NormIn
{
    const float* h;
    const float* w;
    float eps;
    uint16_t* xn;
    _Float16* xh;
};

// logits of experts e0 .. e0 + EPW - 1 (those < E) for R <= MAXR rows over K = H, by a workgroup of EPW x 256 threads
// (EPW 1 or 2: more experts per workgroup share its x staging, fewer spread the weight rows over more CUs), in the order of
// expert_logits with every global load coalesced: the two weight rows, then each group of 4 rows of x, are staged in
// LDS (consecutive threads on consecutive 16-byte pieces) in a chunk-major layout padded to 144 B (weights) and 80 B
// (x) per chunk, so a thread's 16-byte reads of its own chunk are free of bank conflicts (8 lanes cover the 32 banks);
// thread c < 192 of half h runs the fmaf chain of chunk c for expert e0 + h. (Read straight from global memory, a lane
// takes its chunk's 64 or 128 contiguous bytes in 16-byte steps, and each load instruction touches 64 cache lines.)
// NORM: x is formed from the residual (NormIn) instead of read as bf16. Every thread of the workgroup must call it
// (it contains barriers).
constexpr int LCH = H / RCHUNK;             // 192 chunks
constexpr int WST = RCHUNK + 4;             // weight chunk stride, floats
constexpr int XST = RCHUNK / 2 + 4;         // x chunk stride, u32 words (two bf16 each)
// XF16: x holds f16 values (bf16 otherwise); WF16: the weight rows are f16 (fp32 otherwise), widened exactly when staged.
template <bool XF16> __device__ __forceinline__ float x_lo(uint32_t v)
{
    return XF16 ? (float) __builtin_bit_cast(_Float16, (uint16_t) (v & 0xffffu)) : __uint_as_float(v << 16);
}
template <bool XF16> __device__ __forceinline__ float x_hi(uint32_t v)
{
    return XF16 ? (float) __builtin_bit_cast(_Float16, (uint16_t) (v >> 16)) : __uint_as_float(v & 0xffff0000u);
}

template <bool NORM, int EPW = 2, bool XF16 = false, bool WF16 = false>
__device__ inline void pair_logits(const uint16_t* __restrict__ x, const NormIn& nin, const float* __restrict__ wt,
                                   int e0, int E, int R, float* __restrict__ logits)
{
    static_assert(EPW == 1 || EPW == 2, "one or two experts per workgroup");
    static_assert(!NORM || EPW == 2, "the RMSNorm input path splits rows over two halves of 256 threads");
    static_assert(!(NORM && XF16), "the RMSNorm input path forms bf16 rows");
    constexpr int NTH = 256 * EPW, XP = 3072 / NTH;             // threads; x pieces per thread and group of 4 rows
    __shared__ __attribute__((aligned(16))) float ws[EPW][LCH * WST];
    __shared__ __attribute__((aligned(16))) uint32_t xs[4][LCH * XST];
    __shared__ __attribute__((aligned(16))) float sums[EPW][LCH][MAXR + 1];
    __shared__ float segs[EPW][MAXR][RSEG];
    __shared__ float rmfs[MAXR];
    __shared__ float gsum[MAXR][32];
    const int t = threadIdx.x, half = t >> 8, c = t & 255;
    // the weight rows: EPW x 1536 pieces of 4 floats, 6 per thread (a row past E re-reads row E - 1)
    #pragma unroll
    for (int i = 0; i < 6; ++i)
    {
        const int p = t + NTH * i, h = p / 1536, q = p - h * 1536;
        const size_t wo = (size_t) min(e0 + h, E - 1) * H + 4 * q;
        f32x4 v;
        if (WF16)
        {
            const u32x2 u = *(const u32x2*) ((const uint16_t*) wt + wo);
            v = (f32x4) {x_lo<true>(u[0]), x_hi<true>(u[0]), x_lo<true>(u[1]), x_hi<true>(u[1])};
        }
        else v = *(const f32x4*) (wt + wo);
        *(f32x4*) &ws[h][(q >> 3) * WST + 4 * (q & 7)] = v;
    }
    if constexpr (NORM)
    {
        // rmf of every row in the rms_norm_kernel order: thread t (of 512) runs chains t (columns t and t + 1024) and
        // t + 512 (column t + 512); half-wave g sums groups g and g + 16 in registers, the 32 group sums of a row go
        // to gsum, and half-wave r < R sums row r's
        static_assert(NTH == 512, "the norm's chains are laid out for 512 threads");
        for (int r = 0; r < R; ++r)
        {
            const f32x4* v = (const f32x4*) (nin.h + (size_t) r * H);
            const f32x4 a = v[t], b2 = v[t + 1024], m = v[t + 512];
            const float c0 = half_wave_sum(chain4(chain4(0.f, a), b2)), c1 = half_wave_sum(chain4(0.f, m));
            if ((t & 31) == 0) { gsum[r][t >> 5] = c0; gsum[r][16 + (t >> 5)] = c1; }
        }
        __syncthreads();
        if ((t >> 5) < R)
        {
            const float tot = half_wave_sum(gsum[t >> 5][t & 31]);
            if ((t & 31) == 0) rmfs[t >> 5] = rms_factor(tot, nin.eps, 1.0f);
        }
        __syncthreads();
    }
    // rows r0 .. r0 + 3 of x: 4 x 768 pieces of 8 bf16, XP per thread (rows past R re-read row R - 1); the next
    // group's loads are in flight while the current group computes (NORM: formed at the start of each group, and
    // piece q of a live row also stored to xn by workgroup q * G / 768)
    u32x4 nx[XP];
    auto load_x = [&](int r0) {
        #pragma unroll
        for (int i = 0; i < XP; ++i)
        {
            const int p = t + NTH * i, j = p / 768, q = p - j * 768;
            nx[i] = *(const u32x4*) (x + (size_t) min(r0 + j, R - 1) * H + 8 * q);
        }
    };
    auto store_x = [&]() {
        #pragma unroll
        for (int i = 0; i < XP; ++i)
        {
            const int p = t + NTH * i, j = p / 768, q = p - j * 768;
            *(u32x4*) &xs[j][(q >> 2) * XST + 4 * (q & 3)] = nx[i];
        }
    };
    auto form_x = [&](int r0) {
        #pragma unroll
        for (int i = 0; i < XP; ++i)
        {
            const int p = t + NTH * i, j = p / 768, q = p - j * 768, row = min(r0 + j, R - 1);
            const float* hp = nin.h + (size_t) row * H + 8 * q;
            const f32x4 h0 = *(const f32x4*) hp, h1 = *(const f32x4*) (hp + 4);
            const f32x4 w0 = *(const f32x4*) (nin.w + 8 * q), w1 = *(const f32x4*) (nin.w + 8 * q + 4);
            const float rf = rmfs[row];
            u32x4 v;
            #pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const float a0 = e < 2 ? h0[2 * e] : h1[2 * e - 4], a1 = e < 2 ? h0[2 * e + 1] : h1[2 * e - 3];
                const float b0 = e < 2 ? w0[2 * e] : w1[2 * e - 4], b1 = e < 2 ? w0[2 * e + 1] : w1[2 * e - 3];
                v[e] = (uint32_t) hmoe_f2bf((a0 * b0) * rf) | ((uint32_t) hmoe_f2bf((a1 * b1) * rf) << 16);
            }
            *(u32x4*) &xs[j][(q >> 2) * XST + 4 * (q & 3)] = v;
            if (r0 + j < R && (int) ((q * ((E + EPW - 1) / EPW)) / 768) == (int) blockIdx.x)
            {
                *(u32x4*) (nin.xn + (size_t) row * H + 8 * q) = v;
                if (nin.xh)
                {
                    f16x8 o;
                    #pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        o[2 * e] = (_Float16) __uint_as_float(v[e] << 16);
                        o[2 * e + 1] = (_Float16) __uint_as_float(v[e] & 0xffff0000u);
                    }
                    *(f16x8*) (nin.xh + (size_t) row * H + 8 * q) = o;
                }
            }
        }
    };
    if (!NORM)
    {
        load_x(0);
        store_x();
    }
    float wv[RCHUNK];
    for (int r0 = 0; r0 < R; r0 += 4)
    {
        if (NORM) form_x(r0);
        __syncthreads();                                        // group r0 in xs
        if (!NORM) load_x(r0 + 4);
        if (c < LCH)
        {
            if (r0 == 0)
            {
                #pragma unroll
                for (int i = 0; i < RCHUNK; i += 4)
                {
                    const f32x4 v = *(const f32x4*) &ws[half][c * WST + i];
                    wv[i] = v[0]; wv[i + 1] = v[1]; wv[i + 2] = v[2]; wv[i + 3] = v[3];
                }
            }
            #pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                if (r0 + j >= R) break;
                u32x4 xv[4];
                #pragma unroll
                for (int i = 0; i < 4; ++i) xv[i] = *(const u32x4*) &xs[j][c * XST + 4 * i];
                float acc = 0.f;
                #pragma unroll
                for (int i = 0; i < 4; ++i)
                    #pragma unroll
                    for (int k = 0; k < 4; ++k)
                    {
                        acc = __builtin_fmaf(x_lo<XF16>(xv[i][k]), wv[8 * i + 2 * k], acc);
                        acc = __builtin_fmaf(x_hi<XF16>(xv[i][k]), wv[8 * i + 2 * k + 1], acc);
                    }
                sums[half][c][r0 + j] = acc;
            }
        }
        __syncthreads();                                        // every read of xs done
        if (!NORM) store_x();
    }
    // the fold: segment sums (chunks in order) by one thread per (expert, row, segment), then the segments in order
    constexpr int cps = LCH / RSEG;
    if (t < EPW * R * RSEG)
    {
        const int h = t / (R * RSEG), rem = t - h * R * RSEG, r = rem / RSEG, sg = rem - r * RSEG;
        float seg = 0.f;
        #pragma unroll
        for (int q = 0; q < cps; ++q) seg = seg + sums[h][sg * cps + q][r];
        segs[h][r][sg] = seg;
    }
    __syncthreads();
    if (e0 + half < E && c < R)
    {
        float tot = 0.f;
        #pragma unroll
        for (int sg = 0; sg < RSEG; ++sg) tot = tot + segs[half][c][sg];
        logits[(size_t) c * RMAXE + e0 + half] = tot;
    }
}

// bf16 -> f16 of n elements [b0, b1) by the calling threads (stride nthr from tid)
__device__ inline void to_f16_range(const uint16_t* __restrict__ x, _Float16* __restrict__ xh, int b0, int b1, int tid,
                                    int nthr)
{
    for (int i = b0 + tid; i < b1; i += nthr) xh[i] = (_Float16) bf2f(x[i]);
}
}  // namespace hmoe
