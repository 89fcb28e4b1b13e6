// shared_gemm.hip - the prefill shared expert's projections as hand-written dense MFMA GEMMs (f16 operands, fp32
// accumulation). The shared expert is a dense bf16 MLP (its weights are exact in f16), run over every token of the
// chunk; the reference keeps it outside its routed op at prefill (runtime/tier/tier_split.py:548-560, the model's own
// shared-expert forward). gate and up run as one GEMM whose epilogue writes act = f16(silu(g) u); down writes f16
// rows (the ordered combine adds them) or adds them into fp32 out.
//
// dgemm_kernel: D[n][m] = sum_k X[n][k] W[m][k] over row-major W [M][K] (one matrix, or gate and up as two) and X
// [N][K]. Workgroup = WM x WN waves (WM along the weight rows, WN along the tokens) = 16 WM TM / NMAT output rows x
// 16 WN TN tokens; wave (wm, wn) holds TM weight tiles (TM / NMAT of each matrix) x TN token tiles of 16 x 16 in its
// accumulators. K runs in stages of 64:
// both operands of a stage go to LDS by direct global-to-LDS loads, in a ring of 3 stages issued two ahead, so the
// one wait and barrier per stage find the stage long arrived; each 32-k step's fragments are read one step ahead of
// its MFMAs. A stage holds each 8 rows' 128 bytes as a 1 KB block:
// one load per block, lane l taking row l / 8's 16-byte chunk (l % 8) ^ (l / 8) (whole 128-byte lines from memory),
// stored at 16 l; the swizzle puts the 16 rows x 16 bytes of an MFMA fragment read (row l % 16, chunk 4 ks + l / 16)
// on distinct banks. Each 32-k step reads the wave's TM + TN fragments and runs TM TN MFMAs. A token past N reads
// row N - 1 and is not stored.
#include "hmoe_dev.h"

namespace hmoe {

enum { DG_ACT = 0, DG_D16 = 1, DG_ADD = 2 };

template <int NMAT, int TM, int TN, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WM * WN / 4, WM * WN / 4)))
dgemm_kernel(
    const _Float16* __restrict__ w0, const _Float16* __restrict__ w1, const _Float16* __restrict__ x, int N, int K,
    void* __restrict__ out, int ldo)
{
    static_assert((NMAT == 2) == (EPI == DG_ACT), "the SwiGLU epilogue pairs gate and up");
    constexpr int NST = 3;                              // LDS stages, issued NST - 1 ahead
    constexpr int TMO = TM / NMAT;                      // tiles per matrix per wave
    constexpr int NW = WM * WN;                         // waves: WM along the weight rows, WN along the tokens
    constexpr int AT = WM * TM, BT = WN * TN;           // weight and token tiles of the workgroup
    constexpr int NB = (AT + BT) * 2;                   // 1 KB blocks (8 rows x 64 k) per stage
    constexpr int SL = NB / NW;                         // blocks staged per wave per stage
    static_assert(NB % NW == 0 && TM % NMAT == 0 && TM * TN <= 64, "the waves share the staging; 256 accumulators");
    __shared__ __attribute__((aligned(16))) u32x4 lds[NST][NB * 64];
    const int t = threadIdx.x, l = t & 63, row = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6), wm = w % WM, wn = w / WM;
    const int m0 = blockIdx.x * WM * 16 * TMO;          // first output row of each matrix
    const int n0 = blockIdx.y * WN * 16 * TN;           // first token
    const int KS = K / 64;
    // the blocks this wave stages (b = w + NW i): block b holds rows 8 b .. + 8 of the stage's tiles (weight tiles
    // first: tile a = matrix a / (WM TMO), rows 16 (a % (WM TMO)) .., then token tiles); a scalar base per block and
    // the lane's byte offset from it
    const _Float16* sb[SL];
    uint32_t vo[SL];
    const uint32_t chunk = 16u * (uint32_t) ((l & 7) ^ (l >> 3));
    #pragma unroll
    for (int i = 0; i < SL; ++i)
    {
        const int b = w + NW * i, tile = b >> 1, r = 8 * (b & 1) + (l >> 3);
        if (tile < AT)
        {
            const int mat = tile / (WM * TMO), tr = tile % (WM * TMO);
            sb[i] = (mat == 0 ? w0 : w1) + (size_t) (m0 + 16 * tr) * K;
            vo[i] = (uint32_t) r * (K * 2) + chunk;
        }
        else
        {
            const int tk = min(n0 + 16 * (tile - AT) + r, N - 1);
            sb[i] = x;
            vo[i] = (uint32_t) tk * (K * 2) + chunk;
        }
    }
    // stage s into LDS buffer s % NST; a stage past the last (kept so every stage issues the same loads, which the
    // wait counts) reads one fixed 16 bytes
    auto stage = [&](int s) {
        const bool live = s < KS;
        u32x4* buf = lds[s % NST];
        #pragma unroll
        for (int i = 0; i < SL; ++i)
        {
            const _Float16* base = sb[i] + (live ? 64 * s : 0);
            const uint32_t v = live ? vo[i] : 0u;
            const uint32_t la = __builtin_amdgcn_readfirstlane(
                (uint32_t) (uintptr_t) (__attribute__((address_space(3))) void*) (buf + (w + NW * i) * 64));
    #pragma clang diagnostic push
    #pragma clang diagnostic ignored "-Winline-asm"
            // (an SALU write of M0 needs one wait state before an LDS-DMA load reads it: the s_nop)
            asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(v), "s"(base), "s"(la)
                         : "memory", "m0");
    #pragma clang diagnostic pop
        }
    };
    // a fragment's lane l: row l % 16 of the tile (block 2 tile + (l % 16) / 8, row (l % 8) in it), chunk 4 ks + l / 16
    int fo[2];
    #pragma unroll
    for (int ks = 0; ks < 2; ++ks) fo[ks] = 64 * (row >> 3) + 8 * (l & 7) + (((4 * ks + (l >> 4)) ^ (l & 7)));
    f32x4 acc[TM][TN];
    #pragma unroll
    for (int i = 0; i < TM; ++i)
        #pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (f32x4) {0.f, 0.f, 0.f, 0.f};
    // the wave's fragments of one 32-k step of a stage
    f16x8 a[2][TM], bv[2][TN];
    auto read = [&](const u32x4* cur, int ks) {
        #pragma unroll
        for (int i = 0; i < TM; ++i)
        {
            const int tile = (i / TMO) * WM * TMO + wm * TMO + i % TMO;
            a[ks][i] = as_f16x8(cur[tile * 128 + fo[ks]]);
        }
        #pragma unroll
        for (int j = 0; j < TN; ++j) bv[ks][j] = as_f16x8(cur[(AT + wn * TN + j) * 128 + fo[ks]]);
    };
    // stage s is complete when at most the NST - 2 stages issued after it are outstanding
    auto arrive = [&]() {
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"((NST - 2) * SL) : "memory");
        __syncthreads();
    };
    #pragma unroll
    for (int s = 0; s < NST - 1; ++s) stage(s);
    arrive();
    read(lds[0], 0);
    // each step's fragments are read one step ahead of its MFMAs, so no wave waits out an LDS latency: a stage's
    // second step is read before its first step's MFMAs, the next stage's first step (after its wait and barrier)
    // before this stage's second step's MFMAs; the next stage's loads go out between the two steps
    for (int s = 0; s < KS; ++s)
    {
        read(lds[s % NST], 1);
        #pragma unroll
        for (int i = 0; i < TM; ++i)
            #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(a[0][i], bv[0][j], acc[i][j]);
        __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);       // the second step's LDS reads
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);       // then the first step's MFMAs
        stage(s + NST - 1);
        arrive();                                                      // stage s + 1 (past the last: the stand-in)
        read(lds[(s + 1) % NST], 0);
        #pragma unroll
        for (int i = 0; i < TM; ++i)
            #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma16(a[1][i], bv[1][j], acc[i][j]);
        __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);       // the next stage's first-step reads
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);       // then the second step's MFMAs
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // lane l holds output rows 4 (l / 16) .. + 4 of each weight tile for token 16 j + l % 16 of its token tiles
    #pragma unroll
    for (int j = 0; j < TN; ++j)
    {
        const int n = n0 + 16 * (wn * TN + j) + row;
        if (n >= N) continue;
        #pragma unroll
        for (int i = 0; i < TMO; ++i)
        {
            const int m = m0 + 16 * (wm * TMO + i) + 4 * (l >> 4);
            if (EPI == DG_ACT)
            {
                _Float16 o[4];
                #pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = (_Float16) (silu(acc[i][j][q]) * acc[TMO + i][j][q]);
                *(uint2*) ((_Float16*) out + (size_t) n * ldo + m) = *(const uint2*) o;
            }
            else if (EPI == DG_D16)
            {
                _Float16 o[4];
                #pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = (_Float16) acc[i][j][q];
                *(uint2*) ((_Float16*) out + (size_t) n * ldo + m) = *(const uint2*) o;
            }
            else
            {
                f32x4* o = (f32x4*) ((float*) out + (size_t) n * ldo + m);
                *o = *o + acc[i][j];
            }
        }
    }
}

// 8 waves, two per SIMD (measured against 2 x 2 waves of twice the tiles and 2 x 4: -1 % and -0.5 % of the prefill
// chunk): gate and up, workgroups of 128 act columns x 128 tokens (TM 4 = 2 gate + 2 up tiles, TN 4: I / 128 x T / 128,
// 256 workgroups at 2048 tokens, one per CU); down, 192 output rows x 128 tokens (TM 3, TN 4: 512 at 2048)
constexpr int GU_TM = 4, GU_TN = 4, GU_WM = 4, GU_WN = 2;
constexpr int DN_TM = 3, DN_TN = 4, DN_WM = 4, DN_WN = 2;

}  // namespace hmoe

using namespace hmoe;

int hmoe::dense_gate_up(const _Float16* wg, const _Float16* wu, const _Float16* x, int T, _Float16* act, hipStream_t st)
{
    constexpr int BM = 16 * GU_WM * GU_TM / 2, BN = 16 * GU_WN * GU_TN;
    static_assert(I % BM == 0 && H % 64 == 0, "gate/up tiling");
    HMOE_REQUIRE(T >= 1 && ((uintptr_t) wg & 15) == 0 && ((uintptr_t) wu & 15) == 0 && ((uintptr_t) x & 15) == 0 &&
                 ((uintptr_t) act & 7) == 0, "shared gate/up: T %d or alignment", T);
    dgemm_kernel<2, GU_TM, GU_TN, GU_WM, GU_WN, DG_ACT><<<dim3(I / BM, (T + BN - 1) / BN), 64 * GU_WM * GU_WN, 0, st>>>(
        wg, wu, x, T, H, act, I);
    return HMOE_LAUNCHED("shared gate/up");
}

int hmoe::dense_down(const _Float16* wd, const _Float16* act, int T, void* out, int mode, hipStream_t st)
{
    constexpr int BM = 16 * DN_WM * DN_TM, BN = 16 * DN_WN * DN_TN;
    static_assert(H % BM == 0 && I % 64 == 0, "down tiling");
    HMOE_REQUIRE(T >= 1 && ((uintptr_t) wd & 15) == 0 && ((uintptr_t) act & 15) == 0 && ((uintptr_t) out & 15) == 0,
                 "shared down: T %d or alignment", T);
    const dim3 g(H / BM, (T + BN - 1) / BN);
    constexpr int NT = 64 * DN_WM * DN_WN;
    if (mode == DG_MODE_ADD) dgemm_kernel<1, DN_TM, DN_TN, DN_WM, DN_WN, DG_ADD><<<g, NT, 0, st>>>(wd, nullptr, act, T, I, out, H);
    else dgemm_kernel<1, DN_TM, DN_TN, DN_WM, DN_WN, DG_D16><<<g, NT, 0, st>>>(wd, nullptr, act, T, I, out, H);
    return HMOE_LAUNCHED("shared down");
}
