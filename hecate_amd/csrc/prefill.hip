// prefill.hip - prefill MoE on gfx950: device-side dispatch plan (runtime/tier/tier_split.py:400-420 +
// runtime/tier/rtx_split.py:236-255, no host sync) and the grouped expert GEMMs (runtime/tier/moe4/moe4p.cu:217-245).
//
// Dispatch: picks sorted by (expert, flat index) by a counting sort with per-block histograms and in-block ranks, so
// the order equals a stable argsort of the selection; row blocks {expert, first pick, picks, 0} of at most bm picks.
// GEMMs: workgroup = (row block of <= 128 picks of one expert, 128 gate/up or 256 down output columns); see
// pgemm_kernel. gu fuses act = silu(g) * u * w (f16), down writes d = W_d act (fp32), fin adds each
// token's picks into out in top-k order (or with atomics, as p4_fin_kernel, when no inverse map is given). The shared
// expert's projections run on the dense MFMA GEMMs of shared_gemm.hip.
#include "hmoe_dev.h"

namespace hmoe {

constexpr int PB = 128;                     // picks per row block (dispatch bm <= 128)
constexpr int PT = 256;                     // threads
constexpr int DBLK = 256;                   // picks per dispatch block

// ---------------------------------------------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(DBLK) disp_count_kernel(const int64_t* __restrict__ sel, int F, int lo, int n,
                                                          int* __restrict__ hist, int* __restrict__ rank)
{
    __shared__ int es[DBLK];
    __shared__ int h[256];
    const int t = threadIdx.x, i = blockIdx.x * DBLK + t;
    h[t] = 0;
    int e = -1;
    if (i < F) { const int64_t v = sel[i] - lo; if (v >= 0 && v < n) e = (int) v; }
    es[t] = e;
    __syncthreads();
    if (e >= 0)
    {
        atomicAdd(&h[e], 1);
        int rk = 0;
        for (int j = 0; j < t; ++j) rk += es[j] == e;
        rank[i] = rk;
    }
    __syncthreads();
    if (t < n) hist[(size_t) blockIdx.x * n + t] = h[t];
}

// the per-block histograms -> each block's first position per expert (hist rewritten in place), the expert counts,
// the row-block table and meta. Thread (q, e) of 4 x 256 covers a quarter of the blocks for expert e, its loads
// issued 8 at a time so that they are in flight together (a load-add-store chain over the blocks waits out one load
// latency per block: 92 us at 8192 tokens).
__global__ void __launch_bounds__(1024) disp_scan_kernel(int* __restrict__ hist, int nblk, int n, int bm, int balance,
                                                         int* __restrict__ counts, int* __restrict__ rbt, int nrb_max,
                                                         int* __restrict__ meta)
{
    constexpr int NQ = 4, BT = 8;
    __shared__ int part[NQ][256], sc[256], sr[256];
    const int e = threadIdx.x & 255, q = threadIdx.x >> 8;
    const int b_lo = nblk * q / NQ, b_hi = nblk * (q + 1) / NQ;
    const bool live = e < n;
    auto batch = [&](int b0, int (&v)[BT]) {
        #pragma unroll
        for (int j = 0; j < BT; ++j) v[j] = b0 + j < b_hi ? hist[(size_t) (b0 + j) * n + e] : 0;
    };
    int cq = 0;                                                 // expert e's picks in this quarter's blocks
    if (live)
        for (int b0 = b_lo; b0 < b_hi; b0 += BT)
        {
            int v[BT];
            batch(b0, v);
            #pragma unroll
            for (int j = 0; j < BT; ++j) cq += v[j];
        }
    part[q][e] = cq;
    __syncthreads();
    int c = 0, qoff = 0;                                        // expert e's count; picks in the quarters before q
    #pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
    {
        qoff += qq < q ? part[qq][e] : 0;
        c += part[qq][e];
    }
    const int nb = live ? (c + bm - 1) / bm : 0;
    if (q == 0) { sc[e] = live ? c : 0; sr[e] = nb; }
    __syncthreads();
    // inclusive scans of counts and row blocks over the experts (Hillis-Steele over 256, by the first 256 threads)
    for (int off = 1; off < 256; off <<= 1)
    {
        const int a = q == 0 && e >= off ? sc[e - off] : 0, b = q == 0 && e >= off ? sr[e - off] : 0;
        __syncthreads();
        if (q == 0) { sc[e] += a; sr[e] += b; }
        __syncthreads();
    }
    const int off_e = sc[e] - (live ? c : 0), rb0 = sr[e] - nb;
    if (live)
    {
        // each block's first position: the expert's offset, the quarters before, the blocks before in this quarter
        int run = off_e + qoff;
        for (int b0 = b_lo; b0 < b_hi; b0 += BT)
        {
            int v[BT];
            batch(b0, v);
            #pragma unroll
            for (int j = 0; j < BT; ++j)
                if (b0 + j < b_hi) { hist[(size_t) (b0 + j) * n + e] = run; run += v[j]; }
        }
    }
    if (q == 0 && live)
    {
        counts[e] = c;
        for (int k = 0; k < nb; ++k)
        {
            int rows, start;
            if (balance) { const int bs = c / nb, ex = c % nb; rows = bs + (k < ex ? 1 : 0); start = k * bs + (k < ex ? k : ex); }
            else { rows = min(bm, c - bm * k); start = bm * k; }
            const int r = rb0 + k;
            if (r < nrb_max) { rbt[4 * r + 0] = e; rbt[4 * r + 1] = off_e + start; rbt[4 * r + 2] = rows; rbt[4 * r + 3] = 0; }
        }
    }
    if (threadIdx.x == 255) { meta[0] = sc[255]; meta[1] = min(sr[255], nrb_max); meta[2] = sr[255]; meta[3] = 0; }
}

__global__ void __launch_bounds__(DBLK) disp_place_kernel(const int64_t* __restrict__ sel, const uint16_t* __restrict__ rw,
    int F, int topk, int lo, int n, const int* __restrict__ hist, const int* __restrict__ rank, int* __restrict__ tok,
    int* __restrict__ eid, float* __restrict__ wt, int* __restrict__ inv)
{
    const int i = blockIdx.x * DBLK + threadIdx.x;
    if (i >= F) return;
    const int64_t v = sel[i] - lo;
    if (v < 0 || v >= n) { inv[i] = -1; return; }
    const int e = (int) v;
    const int p = hist[(size_t) blockIdx.x * n + e] + rank[i];
    tok[p] = i / topk; eid[p] = e; wt[p] = (float) __builtin_bit_cast(_Float16, rw[i]); inv[i] = p;
}

// ---------------------------------------------------------------------------------------------------------------
// grouped GEMMs
// ---------------------------------------------------------------------------------------------------------------
struct Block { int e, p0, rows; };

// The workgroup's row block and column block. The dispatcher deals a launch's workgroups round-robin over the 8
// XCDs (workgroup i runs on XCD i % 8), each with its own L2: the column blocks of one row block go to consecutive
// workgroups of one XCD, so they run together and read the block's input rows from that XCD's L2 (one fetch from
// memory instead of one per column block). The grid's x extent is a multiple of 8 (pgemm_grid).
// (the grid's extents come from the launch's own arguments: gridDim reads the dispatch packet, a round trip to the
// queue's memory at every workgroup start)
__device__ __forceinline__ void xcd_tile(int& rb, int& cb, int gx, int ny)
{
    const int i = blockIdx.x + gx * blockIdx.y, j = i >> 3;
    rb = (j / ny) * 8 + (i & 7);
    cb = j % ny;
}

static dim3 pgemm_grid(int nrb, int ny) { return dim3((nrb + 7) & ~7, ny); }

// row block rb of the plan: up to 2 PB picks (the dispatch's bm <= 256), run as halves of <= PB picks; a block
// whose expert or picks fall outside the tables (np picks) is skipped, so a caller's malformed plan reads nothing
// out of bounds
__device__ __forceinline__ bool get_block(const int* rbt, int nrb, const int* meta, int n_tab, int np, int rb, Block& b)
{
    if (rb >= nrb || (meta && rb >= meta[1])) return false;
    b.e = rbt[4 * rb]; b.p0 = rbt[4 * rb + 1]; b.rows = min(rbt[4 * rb + 2], 2 * PB);
    return b.e >= 0 && b.e < n_tab && b.rows > 0 && b.p0 >= 0 && b.p0 <= np - b.rows;
}

// A pipelined grouped GEMM for both projections. Workgroup = (row block of <= 128 picks of one expert, 64 NS output
// columns); wave w of column block cb owns output strips nb0 = NWV NS cb + NS w .. + NS (16 rows each) of NMAT
// matrices (gate and up: NS = 2, or down: NS = 4), so every wave holds 4 weight fragments per k step and reads each
// 16-pick input fragment from LDS once for 4 MFMAs. Per 128-k group kg:
//   * the block's input rows are staged in LDS as f16 by direct global-to-LDS loads (double-buffered, one barrier
//     per group): the next group's rows load while this group computes;
//   * the weight tiles come from a ring of D groups of unconditional 16-byte loads, issued D - 1 groups ahead, so HBM
//     latency hides behind that many groups of MFMA work; each tile is loaded once per workgroup; the lane's row
//     scales come 4 groups at a time (one 8-byte load per fragment every fourth group);
//   * each k step dequantises the 4 weight fragments (exact f16 codes times the f16 group scale) and runs the
//     16x16x32 MFMA against the block's 16-pick tiles (up to 8).
// Every vector-memory instruction costs issue time on the SIMD beside the MFMA and dequantisation work, so the loads
// are few and their addresses cheap: uniform bases in scalar registers with 32-bit lane offsets.
template <int NMAT, int NS>
struct PFetch
{
    u32x4 q[NS][NMAT];
};

// epilogues: gate/up -> act f16 (EPI_ACT) or the raw gate and up sums (EPI_RAW, fp32 [2][ps][I], the test entry of
// moe4t); down -> d f16 rows for the ordered combine (EPI_D16), d fp32 rows (EPI_D, the moe4t.gemm test entry) or
// added into out[tok] with fp32 atomics (EPI_FIN, moe4t.cu's down epilogue)
enum { EPI_ACT = 0, EPI_RAW = 1, EPI_D = 2, EPI_FIN = 3, EPI_D16 = 4 };

// NTT: 16-pick tiles per pass (8: 128 picks, 4 waves; 16: 256 picks, 8 waves, one pass for the long prefill's 256-pick
// blocks, each dequantised weight fragment feeding twice the MFMAs); NWV waves, each staging two tiles
template <int NMAT, int NS, int D, int EPI = NMAT == 2 ? EPI_ACT : EPI_D, int NTT = 8, int NWV = 4>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2))) pgemm_kernel(
    const _Float16* __restrict__ xin, const int* __restrict__ tok, const float* __restrict__ wt,
    const int* __restrict__ rbt, int nrb, const int* __restrict__ meta, int n_tab,
    const int64_t* __restrict__ w0, const int64_t* __restrict__ w1, const int64_t* __restrict__ s0,
    const int64_t* __restrict__ s1, _Float16* __restrict__ ar, float* __restrict__ dout, int T, int off, int np,
    float* __restrict__ fout = nullptr, int ps = 0)
{
    static_assert((NMAT == 2) == (EPI == EPI_ACT || EPI == EPI_RAW), "gate/up epilogues need both matrices");
    constexpr int K = NMAT == 2 ? H : I;                 // gate/up: x [T][H] -> act; down: act [.][I] -> d
    constexpr int NOUT = NMAT == 2 ? I : H;
    constexpr int KG = K / 128;
    static_assert(KG % D == 0, "the ring depth divides the k groups");
    static_assert(NS * NMAT * NTT == 32, "32 accumulator tiles per wave (4 fragments x 8 tiles or 2 x 16)");
    static_assert(NTT == 2 * NWV, "each wave stages two tiles");
    constexpr int PBX = 16 * NTT;                        // picks per pass
    // the staged input of a 128-k group (four 1 KB blocks per 16-pick tile, below); two buffers, the next group loads
    // while one computes
    __shared__ __attribute__((aligned(16))) u32x4 xs0[NTT * 4 * 64];
    __shared__ __attribute__((aligned(16))) u32x4 xs1[NTT * 4 * 64];
    int rbi, cbi;
    xcd_tile(rbi, cbi, (nrb + 7) & ~7, NOUT / (16 * NS * NWV));
    Block rb;
    if (!get_block(rbt, nrb, meta, n_tab, np, rbi, rb)) return;
    // a block of more than PBX picks runs as passes of PBX, one after the other (a later pass reads the weights
    // again, mostly from the caches); the barrier between them keeps one pass's last LDS reads ahead of the next
    // pass's first staging
    for (int h0 = 0; h0 < rb.rows; h0 += PBX)
    {
        if (h0) __syncthreads();
        const Block b = {rb.e, rb.p0 + h0, min(PBX, rb.rows - h0)};
        const int t = threadIdx.x, l = t & 63, row = l & 15;
        const int w = __builtin_amdgcn_readfirstlane(t >> 6);   // wave index, kept in a scalar register
        const int nb0 = (cbi * NWV + w) * NS;
        const uint8_t* wp[NMAT];
        const uint8_t* sp[NMAT];
        #pragma unroll
        for (int m = 0; m < NMAT; ++m)
        {
            wp[m] = (const uint8_t*) (m == 0 ? w0 : w1)[b.e];
            sp[m] = (const uint8_t*) (m == 0 ? s0 : s1)[b.e];
        }
        const int ntt = (b.rows + 15) >> 4;
        const DqConsts dq = dq_consts();
        // The staged input of a 128-k group: per 16-pick tile, four 1 KB blocks (k half kh, row half rh) of 8 rows x 64
        // k; lane l of a block takes row l / 8's 16-byte chunk (l % 8) ^ (l / 8) (whole 128-byte lines from memory) and
        // stores it at 16 l, so a fragment read (row l % 16, chunk 4 (k % 2) + l / 16 of k half k / 2) meets distinct
        // banks. Wave w stages tiles 2w and 2w + 1: lane l's source row in each row half; a pick past the block re-reads
        // a valid row (its output columns are never stored), a whole tile past the block reads one fixed 16 bytes.
        uint32_t src[2][2];                                     // byte offsets from xin
        #pragma unroll
        for (int h = 0; h < 2; ++h)
            #pragma unroll
            for (int rh = 0; rh < 2; ++rh)
            {
                const int tt = 2 * w + h, pk = tt * 16 + 8 * rh + (l >> 3);
                const bool in = pk < b.rows, tin = tt < ntt;
                int srow;
                if (NMAT == 2)
                {
                    // (no token map: the picks' inputs are rows p0 .. of xin, as the moe4t test entry passes them)
                    const int tk = !tok ? b.p0 + (in ? pk : 0) : tok[b.p0 + (in ? pk : 0)];
                    srow = (unsigned) tk < (unsigned) T ? tk : 0;
                }
                else srow = off + b.p0 + (in ? pk : 0);
                src[h][rh] = (uint32_t) (((size_t) srow * K + (tin ? 8 * ((l & 7) ^ (l >> 3)) : 0)) * 2);
            }
        int fo[4];
        #pragma unroll
        for (int k = 0; k < 4; ++k)
            fo[k] = ((k >> 1) * 2 + (row >> 3)) * 64 + 8 * (l & 7) + ((4 * (k & 1) + (l >> 4)) ^ (l & 7));
        // Direct global-to-LDS loads (16 bytes per lane, lane l at LDS base + 16 l), issued from inline assembly: the
        // compiler then does not count them, so its own waits for the weight ring stay exact, and the wait that makes a
        // staged group visible is placed by hand before the barrier (the loads issued after a stage are exactly those
        // of one ring refill). M0 holds the LDS base of each load; nothing else in this kernel uses M0.
        auto stage = [&](int kg, u32x4* buf) {
            #pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                const int tt = 2 * w + h;
                const bool tin = tt < ntt;
                #pragma unroll
                for (int kh = 0; kh < 2; ++kh)
                    #pragma unroll
                    for (int rh = 0; rh < 2; ++rh)
                    {
                        const uint32_t gp = src[h][rh] + (tin ? (kg * 128 + 64 * kh) * 2 : 0);
                        const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t)
                            (__attribute__((address_space(3))) void*) (buf + (tt * 4 + kh * 2 + rh) * 64));
    #pragma clang diagnostic push
    #pragma clang diagnostic ignored "-Winline-asm"
                        // (an SALU write of M0 needs one wait state before an LDS-DMA load reads it: the s_nop)
                        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(gp), "s"(xin),
                                     "s"(lds) : "memory", "m0");
    #pragma clang diagnostic pop
                    }
            }
        };
        PFetch<NMAT, NS> ring[D];
        // the row scales of two blocks of 4 groups (a block's 4 bf16 of one row are 8 contiguous bytes of I4G128)
        u32x2 sc4[2][NS][NMAT];
        // the weights of group kg into ring slot SL; when kg starts a block of 4, the block's scales too, into sc4[SC]
        // (SC = -1: none). Offsets are 32-bit (an expert's matrix is 6.3 MB), so the loads take the base from scalar
        // registers.
        auto fetch = [&](int kg, auto sl, auto sc) {
            constexpr int SL = decltype(sl)::value, SC = decltype(sc)::value;
            #pragma unroll
            for (int st = 0; st < NS; ++st)
                #pragma unroll
                for (int m = 0; m < NMAT; ++m)
                {
                    const int nb = nb0 + st;
                    ring[SL].q[st][m] = ldw16(wp[m] + (uint32_t) (((nb * KG + kg) * 64 + l) * 16));
                    if constexpr (SC >= 0)
                        sc4[SC][st][m] = ld8(sp[m] + (uint32_t) (sc_index(nb * 16 + row, kg & ~3, KG) * 2));
                }
        };
        f32x4 acc[NS][NMAT][NTT];
        #pragma unroll
        for (int st = 0; st < NS; ++st)
            #pragma unroll
            for (int m = 0; m < NMAT; ++m)
                #pragma unroll
                for (int tt = 0; tt < NTT; ++tt) acc[st][m][tt] = (f32x4) {0.f, 0.f, 0.f, 0.f};
        // the prologue stages group 0 and fills D - 1 ring slots; group kg then issues its loads (the next stage and
        // the refill of the slot group kg - 1 used, D - 1 groups ahead) only after its own operands are in hand, so
        // that no wait for them counts the new loads: a weight refill has D - 1 groups to arrive
        stage(0, xs0);
        static_for<D - 1>([&](auto sc) {
            constexpr int g = decltype(sc)::value;
            fetch(g, sc, std::integral_constant<int, g % 4 == 0 ? (g / 4) % 2 : -1>{});
            __builtin_amdgcn_sched_barrier(0);                  // keep the ring's issue order (waits count in order)
        });
        // the group loop runs in steps of 8, so that the ring slot (kg % D), the scale block (kg / 4 % 2) and whether a
        // refill starts a block are compile-time constants
        static_assert(KG % 8 == 0 && 8 % D == 0, "the group loop runs in steps of 8");
        for (int kg0 = 0; kg0 < KG; kg0 += 8)
        {
            static_for<8>([&](auto sc8) {
                constexpr int s8 = decltype(sc8)::value, s = s8 % D;
                const int kg = kg0 + s8;
                const bool even = (kg & 1) == 0;
                u32x4* cur = even ? xs0 : xs1;
                // this wave's staged loads of group kg are older than the loads of the refill issued with them in group
                // kg - 1 (its NS NMAT weight loads and, when that refill started a block of 4, as many scale loads); for
                // kg = 0 every load is waited for. The barrier then makes every wave's group kg visible.
                constexpr int gp = (s8 + 7) % 8 + D - 1;            // the group refilled in group kg - 1, mod 8
                constexpr int after = NS * NMAT * (gp % 4 == 0 ? 2 : 1);
                if (kg == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(%0)" :: "n"(after) : "memory");
                __syncthreads();
                // the slot's scales and first k step: the compiler's wait for the slot falls here, before the loads
                // below (its count of later loads is then the D - 2 refills it knows of, and the stage, which has
                // arrived, is the only load it does not count)
                f16x2 sh[NS][NMAT];
                f16x8 a0[NS][NMAT];
                #pragma unroll
                for (int st = 0; st < NS; ++st)
                    #pragma unroll
                    for (int m = 0; m < NMAT; ++m)
                    {
                        const uint32_t sw = sc4[s8 / 4][st][m][(s8 % 4) / 2];     // bf16 of group kg: half s8 % 2
                        const _Float16 h = (_Float16) __uint_as_float(s8 % 2 == 0 ? sw << 16 : sw & 0xffff0000u);
                        sh[st][m] = (f16x2) {h, h};
                        a0[st][m] = dq8s(ring[s].q[st][m][0], sh[st][m], dq);
                    }
                __builtin_amdgcn_sched_barrier(0);
                if (kg + 1 < KG) stage(kg + 1, even ? xs1 : xs0);
                // the refill: group kg + D - 1, clamped to the last group; it starts a block of 4 when (s8 + D - 1) % 4
                // == 0, whose scales go to sc4[(s8 + D - 1) / 4 % 2] (kg0 is a multiple of 8). Past the last group the
                // clamped group's block is loaded again into the buffer that no remaining group reads.
                constexpr int gn = s8 + D - 1;
                fetch(min(kg + D - 1, KG - 1), std::integral_constant<int, (s + D - 1) % D>{},
                      std::integral_constant<int, gn % 4 == 0 ? (gn / 4) % 2 : -1>{});
                __builtin_amdgcn_sched_barrier(0);
                #pragma unroll
                for (int k = 0; k < 4; ++k)
                {
                    f16x8 a[NS][NMAT];
                    #pragma unroll
                    for (int st = 0; st < NS; ++st)
                        #pragma unroll
                        for (int m = 0; m < NMAT; ++m)
                            a[st][m] = k == 0 ? a0[st][m] : dq8s(ring[s].q[st][m][k], sh[st][m], dq);
                    // The pick tiles are read PD tiles ahead of their MFMAs (a tile past the block reads stale LDS
                    // data, never used). Each read is consumed by an empty asm after the MFMAs of the tile before it,
                    // which keeps the read ahead of the branch that ends the block's tiles: the compiler would
                    // otherwise sink it behind that branch, next to its MFMAs, and wait out its latency there. With
                    // four MFMAs per tile one tile ahead is enough and the consuming asm is pinned behind all four
                    // (measured: -1 %); with two, two tiles ahead and the asm left to the scheduler (-8 % at 8192
                    // tokens, pinning it cost 1.5 %).
                    constexpr int PD = NS * NMAT >= 4 ? 1 : 2;
                    f16x8 bq[PD + 1];
                    #pragma unroll
                    for (int i = 0; i < PD; ++i) bq[i] = as_f16x8(cur[i * 256 + fo[k]]);
                    #pragma unroll
                    for (int tt = 0; tt < NTT; ++tt)
                    {
                        if (tt >= ntt) break;
                        if (tt + PD < NTT) bq[PD] = as_f16x8(cur[(tt + PD) * 256 + fo[k]]);
                        #pragma unroll
                        for (int st = 0; st < NS; ++st)
                            #pragma unroll
                            for (int m = 0; m < NMAT; ++m) acc[st][m][tt] = mfma16(a[st][m], bq[0], acc[st][m][tt]);
                        if constexpr (PD == 1) __builtin_amdgcn_sched_barrier(0);
                        if (tt + 1 < NTT) asm volatile("" :: "v"(bq[1]));
                        #pragma unroll
                        for (int i = 0; i < PD; ++i) bq[i] = bq[i + 1];
                    }
                }
            });
        }
        // epilogue: lane holds output rows 4(l/16)..+4 of pick tt*16 + l%16
        #pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
        {
            const int pk = tt * 16 + row;
            if (pk >= b.rows) continue;
            #pragma unroll
            for (int st = 0; st < NS; ++st)
            {
                const int n = (nb0 + st) * 16 + 4 * (l >> 4);
                if (EPI == EPI_RAW)
                {
                    #pragma unroll
                    for (int m = 0; m < NMAT; ++m)
                        *(f32x4*) (dout + ((size_t) m * ps + b.p0 + pk) * NOUT + n) = acc[st][m][tt];
                }
                else if (EPI == EPI_ACT)
                {
                    const float wv = wt[b.p0 + pk];
                    _Float16 o[4];
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = (_Float16) (silu(acc[st][0][tt][i]) * acc[st][NMAT - 1][tt][i] * wv);
                    *(uint2*) (ar + (size_t) (off + b.p0 + pk) * NOUT + n) = *(const uint2*) o;
                }
                else if (EPI == EPI_FIN)
                {
                    // out[tok] += acc (the combine in the epilogue, fp32 atomics as moe4t.cu's down GEMM: no d buffer)
                    const int tk = tok[b.p0 + pk];
                    if ((unsigned) tk < (unsigned) T)
                    {
                        float* o = fout + (size_t) tk * NOUT + n;
                        #pragma unroll
                        for (int i = 0; i < 4; ++i) unsafeAtomicAdd(o + i, acc[st][0][tt][i]);
                    }
                }
                else if (EPI == EPI_D16)
                {
                    // (a pick's down row rounded to f16: half the bytes written here and read by the combine)
                    _Float16 o[4];
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = (_Float16) acc[st][0][tt][i];
                    *(uint2*) ((_Float16*) dout + (size_t) (off + b.p0 + pk) * NOUT + n) = *(const uint2*) o;
                }
                else *(f32x4*) (dout + (size_t) (off + b.p0 + pk) * NOUT + n) = acc[st][0][tt];
            }
        }
    }
}

// x bf16 -> f16 (the GEMM input when the caller has no f16 copy), on a grid of TF16_GRID workgroups
constexpr int TF16_GRID = 1024;
__global__ void __launch_bounds__(256) to_f16_kernel(const uint16_t* __restrict__ x, size_t n, _Float16* __restrict__ xh)
{
    for (size_t i = (blockIdx.x * (size_t) 256 + threadIdx.x) * 8; i < n; i += (size_t) TF16_GRID * 256 * 8)
    {
        const u32x4 v = ld16(x + i);
        f16x8 o;
        #pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            o[2 * k] = (_Float16) __uint_as_float(v[k] << 16);
            o[2 * k + 1] = (_Float16) __uint_as_float(v[k] & 0xffff0000u);
        }
        *(f16x8*) (xh + i) = o;
    }
}

// fin, deterministic: out[t] += (sum over k in top-k order of d[inv[t][k]]) (+ the shared expert's row), the d rows f16,
// summed in fp32. Every row's load is unconditional (an absent pick or shared row reads row 0 and is dropped by a
// select at its add), so all of them are in flight together: under a branch each load was followed by a wait for it.
// MODE PF_ADD: out += the sum; PF_BF16: the sum goes to ob as bf16 (the partial out taken as zero and left untouched),
// as PF_ADD into a zeroed out followed by finish_bf16 (0 + s is s, and s is never -0: it starts at +0); PF_FIN: ob =
// bf16(out + sum) and out zeroed, as PF_ADD followed by finish_bf16
enum { PF_ADD = 0, PF_BF16 = 1, PF_FIN = 2 };
template <int MODE>
__global__ void __launch_bounds__(256) pfin_kernel(const _Float16* __restrict__ d, const int* __restrict__ inv, int topk,
                                                   int np, int sh_off, float* __restrict__ out, uint16_t* __restrict__ ob)
{
    constexpr int NR = HMOE_TOPK + 1;
    const int t = blockIdx.x;
    int pos[NR];
    bool use[NR];
    #pragma unroll
    for (int k = 0; k < HMOE_TOPK; ++k)
    {
        const int p = k < topk ? inv[(size_t) t * topk + min(k, topk - 1)] : -1;
        use[k] = (unsigned) p < (unsigned) np;                      // -1: a pick outside the window
        pos[k] = use[k] ? p : 0;
    }
    use[HMOE_TOPK] = sh_off >= 0;
    pos[HMOE_TOPK] = sh_off >= 0 ? sh_off + t : 0;
    for (int n = threadIdx.x * 4; n < H; n += 256 * 4)
    {
        f16x4 v[NR];
        #pragma unroll
        for (int k = 0; k < NR; ++k) v[k] = *(const f16x4*) (d + (size_t) pos[k] * H + n);
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        #pragma unroll
        for (int k = 0; k < NR; ++k)
        {
            f32x4 vk;
            #pragma unroll
            for (int i = 0; i < 4; ++i) vk[i] = (float) v[k][i];
            s = use[k] ? s + vk : s;
        }
        if constexpr (MODE != PF_ADD)
        {
            if constexpr (MODE == PF_FIN)
            {
                f32x4* o = (f32x4*) (out + (size_t) t * H + n);
                s = *o + s;
                *o = (f32x4) {0.f, 0.f, 0.f, 0.f};
            }
            uint32_t w[2];
            #pragma unroll
            for (int i = 0; i < 2; ++i) w[i] = (uint32_t) hmoe_f2bf(s[2 * i]) | ((uint32_t) hmoe_f2bf(s[2 * i + 1]) << 16);
            *(uint2*) (ob + (size_t) t * H + n) = *(const uint2*) w;
        }
        else
        {
            f32x4* o = (f32x4*) (out + (size_t) t * H + n);
            *o = *o + s;
        }
    }
}

}  // namespace hmoe

using namespace hmoe;

extern "C" size_t hmoe_dispatch_work_bytes(int T, int topk, int n)
{
    const size_t F = (size_t) T * topk, nblk = (F + DBLK - 1) / DBLK;
    return (nblk * (size_t) n + F) * sizeof(int);
}

extern "C" int hmoe_dispatch_nrb_max(int npos_max, int n, int bm)
{
    if (bm <= 0) return 0;
    return n + npos_max / bm;
}

extern "C" int hmoe_dispatch(const int64_t* sel, const uint16_t* rw, int T, int topk, int lo, int n, int bm,
                             int balance, int* counts, int* tok, int* eid, float* wt, int* inv, int* rbt, int nrb_max,
                             int* meta, void* work, void* stream)
{
    HMOE_REQUIRE(sel && rw && counts && tok && eid && wt && inv && rbt && meta && work, "dispatch: null buffer");
    HMOE_REQUIRE(T >= 1 && topk >= 1 && topk <= TOPK && n >= 1 && n <= 256 && lo >= 0 && bm >= 1 && bm <= 2 * PB &&
                 nrb_max >= 1,
                 "dispatch: T %d topk %d n %d bm %d", T, topk, n, bm);
    const int F = T * topk, nblk = (F + DBLK - 1) / DBLK;
    int* hist = (int*) work;
    int* rank = hist + (size_t) nblk * n;
    hipStream_t st = (hipStream_t) stream;
    disp_count_kernel<<<nblk, DBLK, 0, st>>>(sel, F, lo, n, hist, rank);
    disp_scan_kernel<<<1, 1024, 0, st>>>(hist, nblk, n, bm, balance, counts, rbt, nrb_max, meta);
    disp_place_kernel<<<nblk, DBLK, 0, st>>>(sel, rw, F, topk, lo, n, hist, rank, tok, eid, wt, inv);
    return HMOE_LAUNCHED("dispatch");
}

namespace hmoe {

// the gu scratch: the f16 copy of x ([T][H], when xf = 0)
#define SH_X_BYTES(T) (((size_t) (T) * H * 2 + 255) & ~(size_t) 255)

}  // namespace hmoe

extern "C" size_t hmoe_moe4p_scratch_bytes(int which, int ps, int T)
{
    switch (which)
    {
        case 0: return SH_X_BYTES(T);                                   // gu: the f16 copy of x
        case 1: return (size_t) (ps + T) * I * 2;                       // ar f16 [ps + T][I]
        case 2: return (size_t) (ps + T) * H * 4;                       // d [ps + T][H]: f16 rows (fp32-sized, as the reference)
        default: return 0;
    }
}

// moe4p forward; ob (with inv): the combine writes bf16 rows to ob and out is neither read nor written
static int moe4p_run(const void* x, const int* tok, const float* wt, const int* rbt, int npos, int nrb, int n_tab,
                     const int64_t* gw, const int64_t* uw, const int64_t* dw, const int64_t* gs, const int64_t* us,
                     const int64_t* ds, float* gu, uint16_t* ar, float* d, float* out, int ps, const int* meta,
                     const int* inv, int T, int topk, const void* sh_gw, const void* sh_uw, const void* sh_dw, int xf,
                     uint16_t* ob, void* stream)
{
    // an empty chunk is a no-op, as the reference returns when no pick reaches the tier (moe4p.cu:229)
    if (T == 0 && npos == 0) return HMOE_OK;
    HMOE_REQUIRE(x && tok && wt && rbt && ar && d && (out || ob), "moe4p_forward: null buffer");
    HMOE_REQUIRE(!ob || (inv && ((uintptr_t) ob & 7) == 0), "moe4p_forward_bf16: needs the inverse map and an 8-byte "
                 "aligned bf16 output");
    HMOE_REQUIRE(npos >= 0 && nrb >= 0 && npos <= ps && T >= 1 && topk >= 1 && topk <= TOPK,
                 "moe4p_forward: npos %d nrb %d ps %d T %d topk %d", npos, nrb, ps, T, topk);
    // (the grouped GEMMs address their input rows by 32-bit byte offsets)
    HMOE_REQUIRE((size_t) T * H * 2 <= UINT32_MAX && (size_t) (ps + T) * I * 2 <= UINT32_MAX,
                 "moe4p_forward: T %d ps %d past the 4 GB input offsets", T, ps);
    HMOE_REQUIRE(n_tab >= 0 && n_tab <= HMOE_MAXE && (n_tab == 0 || (gw && uw && dw && gs && us && ds)),
                 "moe4p_forward: tables");
    HMOE_REQUIRE((!sh_gw && !sh_uw && !sh_dw) || (sh_gw && sh_uw && sh_dw && inv),
                 "moe4p_forward: the shared expert needs all three matrices and the inverse map");
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) ar & 15) == 0 && ((uintptr_t) d & 15) == 0 &&
                 ((uintptr_t) out & 15) == 0, "moe4p_forward: alignment");
    HMOE_REQUIRE(xf == HMOE_XF_BF16 || xf == HMOE_XF_F16, "moe4p_forward: xf must be HMOE_XF_BF16 (0) or HMOE_XF_F16 "
                 "(2); the reference's fragment-order x (xf = 1) is not supported");
    hipStream_t st = (hipStream_t) stream;
    const uint16_t* xb = (const uint16_t*) x;
    if (xf == HMOE_XF_BF16)
    {
        HMOE_REQUIRE(gu && ((uintptr_t) gu & 15) == 0, "moe4p_forward: xf = 0 needs the gu scratch (the f16 copy of x)");
        to_f16_kernel<<<TF16_GRID, 256, 0, st>>>(xb, (size_t) T * H, (_Float16*) gu);
        xb = (const uint16_t*) gu;
    }
    _Float16* a = (_Float16*) ar;
    // gate/up: 64 x 2 output columns per workgroup (NS 2); down: 64 x 4 (NS 4), into d rows for the ordered combine
    // (inv given) or added into out[tok] by its epilogue (no inverse map: the atomic combine of p4_fin_kernel)
    if (nrb > 0)
    {
        pgemm_kernel<2, 2, 2><<<pgemm_grid(nrb, I / 128), PT, 0, st>>>((const _Float16*) xb, tok, wt, rbt, nrb, meta,
            n_tab, gw, uw, gs, us, a, nullptr, T, 0, npos);
        if (inv)
            pgemm_kernel<1, 4, 2, EPI_D16><<<pgemm_grid(nrb, H / 256), PT, 0, st>>>(a, nullptr, nullptr, rbt, nrb, meta,
                n_tab, dw, nullptr, ds, nullptr, nullptr, d, T, 0, npos);
        else
            pgemm_kernel<1, 4, 2, EPI_FIN><<<pgemm_grid(nrb, H / 256), PT, 0, st>>>(a, tok, nullptr, rbt, nrb, meta, n_tab,
                dw, nullptr, ds, nullptr, nullptr, nullptr, T, 0, npos, out);
    }
    const bool sh = sh_gw != nullptr;
    if (sh)
    {
        // the shared expert on every token: act rows ps.. = f16(silu(gate x) up x), then down into d rows ps.. (f16),
        // which the ordered combine adds after each token's picks
        if (int rc = dense_gate_up((const _Float16*) sh_gw, (const _Float16*) sh_uw, (const _Float16*) xb, T,
                                   a + (size_t) ps * I, st))
            return rc;
        if (int rc = dense_down((const _Float16*) sh_dw, a + (size_t) ps * I, T, (_Float16*) d + (size_t) ps * H,
                                DG_MODE_F16, st))
            return rc;
    }
    if (inv && ob) pfin_kernel<PF_BF16><<<T, 256, 0, st>>>((const _Float16*) d, inv, topk, npos, sh ? ps : -1, nullptr, ob);
    else if (inv) pfin_kernel<PF_ADD><<<T, 256, 0, st>>>((const _Float16*) d, inv, topk, npos, sh ? ps : -1, out, nullptr);
    return HMOE_LAUNCHED("moe4p_forward");
}

extern "C" int hmoe_moe4p_forward(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt,
                                  int npos, int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw,
                                  const int64_t* gs, const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar,
                                  float* d, float* out, int ps, const int* meta, const int* inv, int T, int topk,
                                  const void* sh_gw, const void* sh_uw, const void* sh_dw, int xf, void* stream)
{
    (void) eid;
    HMOE_REQUIRE(out || (T == 0 && npos == 0), "moe4p_forward: null buffer");
    return moe4p_run(x, tok, wt, rbt, npos, nrb, n_tab, gw, uw, dw, gs, us, ds, gu, ar, d, out, ps, meta, inv, T, topk,
                     sh_gw, sh_uw, sh_dw, xf, nullptr, stream);
}

extern "C" int hmoe_moe4p_forward_bf16(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt,
                                       int npos, int nrb, int n_tab, const int64_t* gw, const int64_t* uw,
                                       const int64_t* dw, const int64_t* gs, const int64_t* us, const int64_t* ds,
                                       float* gu, uint16_t* ar, float* d, int ps, const int* meta, const int* inv, int T,
                                       int topk, const void* sh_gw, const void* sh_uw, const void* sh_dw, int xf,
                                       uint16_t* out_bf16, void* stream)
{
    (void) eid;
    HMOE_REQUIRE(out_bf16 || (T == 0 && npos == 0), "moe4p_forward_bf16: null buffer");
    return moe4p_run(x, tok, wt, rbt, npos, nrb, n_tab, gw, uw, dw, gs, us, ds, gu, ar, d, nullptr, ps, meta, inv, T,
                     topk, sh_gw, sh_uw, sh_dw, xf, out_bf16, stream);
}

// ---------------------------------------------------------------------------------------------------------------
// the shared expert alone over a chunk (the reference runs it through the model's own shared-expert MLP at prefill,
// runtime/tier/tier_split.py:548-560): out += down(silu(gate x) * up x)
// ---------------------------------------------------------------------------------------------------------------
namespace hmoe {

// work layout: x f16 copy [T][H] | act f16 [T][I]
static size_t shw_act(int T) { return SH_X_BYTES(T); }
static size_t shw_end(int T) { return shw_act(T) + (((size_t) T * I * 2 + 255) & ~(size_t) 255); }

}  // namespace hmoe

extern "C" size_t hmoe_shared_work_bytes(int T) { return shw_end(T > 0 ? T : 1); }

extern "C" int hmoe_shared_forward(const void* x, int T, const void* sh_gw, const void* sh_uw, const void* sh_dw,
                                   void* work, float* out, int xf, void* stream)
{
    if (T == 0) return HMOE_OK;
    HMOE_REQUIRE(x && sh_gw && sh_uw && sh_dw && work && out && T > 0, "shared_forward: arguments");
    HMOE_REQUIRE(xf == HMOE_XF_BF16 || xf == HMOE_XF_F16, "shared_forward: xf must be HMOE_XF_BF16 (0) or HMOE_XF_F16 (2)");
    // (the dense GEMMs address their input rows by 32-bit byte offsets)
    HMOE_REQUIRE((size_t) T * H * 2 <= UINT32_MAX, "shared_forward: T %d past the 4 GB input offsets", T);
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) work & 255) == 0 && ((uintptr_t) out & 15) == 0,
                 "shared_forward: alignment (x, out 16 bytes, work 256)");
    hipStream_t st = (hipStream_t) stream;
    uint8_t* wk = (uint8_t*) work;
    const _Float16* xs = (const _Float16*) x;
    if (xf == HMOE_XF_BF16)
    {
        to_f16_kernel<<<TF16_GRID, 256, 0, st>>>((const uint16_t*) x, (size_t) T * H, (_Float16*) wk);
        xs = (const _Float16*) wk;
    }
    _Float16* a = (_Float16*) (wk + shw_act(T));
    if (int rc = dense_gate_up((const _Float16*) sh_gw, (const _Float16*) sh_uw, xs, T, a, st)) return rc;
    // (out += each product element once, in the GEMM's epilogue)
    if (int rc = dense_down((const _Float16*) sh_dw, a, T, out, DG_MODE_ADD, st)) return rc;
    return HMOE_LAUNCHED("shared_forward");
}

// ---------------------------------------------------------------------------------------------------------------
// long prefill: runtime/tier/moe4/moe4t.cu:476-524 (moe4t.gemm / scratch / forward)
// ---------------------------------------------------------------------------------------------------------------
extern "C" size_t hmoe_moe4t_scratch_bytes(int which, int npos)
{
    const size_t n = npos > 0 ? (size_t) npos : 1;
    switch (which)
    {
        case 0: return 2 * n * I * 4;                                   // gu fp32 [2][npos][I] (unused)
        case 1: return n * I * 2;                                       // ar f16 [npos][I]
        case 2: return n * H * 4;                                       // d fp32 [1][npos][H]: the f16 copy of bf16 x
        default: return 0;
    }
}

// moe4t forward; ob (with inv): the combine writes bf16(out + picks) to ob and zeroes out
static int moe4t_run(const void* x, const int* tok, const float* wt, const int* rbt, int npos, int nrb, int n_tab,
                     const int64_t* gw, const int64_t* uw, const int64_t* dw, const int64_t* gs, const int64_t* us,
                     const int64_t* ds, uint16_t* ar, float* d, float* out, int ps, const int* meta, int T, int xf,
                     const int* inv, int topk, uint16_t* ob, void* stream)
{
    if (npos == 0) return HMOE_OK;                                      // moe4t.cu:508: no pick, no work
    HMOE_REQUIRE(x && tok && wt && rbt && ar && out, "moe4t_forward: null buffer");
    HMOE_REQUIRE(npos > 0 && nrb >= 0 && npos <= ps && T >= 1, "moe4t_forward: npos %d nrb %d ps %d T %d", npos, nrb, ps,
                 T);
    HMOE_REQUIRE((size_t) T * H * 2 <= UINT32_MAX && (size_t) ps * I * 2 <= UINT32_MAX,
                 "moe4t_forward: T %d ps %d past the 4 GB input offsets", T, ps);
    HMOE_REQUIRE(n_tab >= 1 && n_tab <= HMOE_MAXE && gw && uw && dw && gs && us && ds, "moe4t_forward: tables");
    HMOE_REQUIRE(xf == HMOE_XF_BF16 || xf == HMOE_XF_F16, "moe4t_forward: xf must be HMOE_XF_BF16 (0) or HMOE_XF_F16 (2)");
    HMOE_REQUIRE(((uintptr_t) x & 15) == 0 && ((uintptr_t) ar & 15) == 0 && ((uintptr_t) out & 15) == 0 &&
                 ((uintptr_t) d & 15) == 0, "moe4t_forward: alignment");
    HMOE_REQUIRE(!inv || (d && topk >= 1 && topk <= TOPK), "moe4t_forward: the ordered combine needs d and topk");
    hipStream_t st = (hipStream_t) stream;
    const _Float16* xh = (const _Float16*) x;
    if (xf == HMOE_XF_BF16)
    {
        // the f16 copy of x in d (the reference gathers the picks' rows into d; T rows fit: T * H * 2 <= npos * H * 4
        // whenever every token has a pick, and the check below holds it in general)
        HMOE_REQUIRE(d && (size_t) T * H * 2 <= (size_t) ps * H * 4, "moe4t_forward: bf16 x needs d for its f16 copy");
        to_f16_kernel<<<TF16_GRID, 256, 0, st>>>((const uint16_t*) x, (size_t) T * H, (_Float16*) d);
        xh = (const _Float16*) d;
    }
    if (nrb > 0)
    {
        // 256-pick blocks in one pass: 8 waves, each one 16-row strip of gate and of up (or two of down) against the
        // block's 16 pick tiles
        pgemm_kernel<2, 1, 4, EPI_ACT, 16, 8><<<pgemm_grid(nrb, I / 128), 512, 0, st>>>(xh, tok, wt, rbt, nrb, meta, n_tab,
            gw, uw, gs, us, (_Float16*) ar, nullptr, T, 0, npos);
        // (d held the f16 copy of x, which the gate/up GEMM has consumed by now: the down rows may overwrite it)
        if (inv)
            pgemm_kernel<1, 2, 4, EPI_D16, 16, 8><<<pgemm_grid(nrb, H / 256), 512, 0, st>>>((const _Float16*) ar,
                nullptr, nullptr, rbt, nrb, meta, n_tab, dw, nullptr, ds, nullptr, nullptr, d, T, 0, npos);
        else
            pgemm_kernel<1, 2, 4, EPI_FIN, 16, 8><<<pgemm_grid(nrb, H / 256), 512, 0, st>>>((const _Float16*) ar, tok,
                nullptr, rbt, nrb, meta, n_tab, dw, nullptr, ds, nullptr, nullptr, nullptr, T, 0, npos, out);
    }
    if (inv && ob) pfin_kernel<PF_FIN><<<T, 256, 0, st>>>((const _Float16*) d, inv, topk, npos, -1, out, ob);
    else if (inv) pfin_kernel<PF_ADD><<<T, 256, 0, st>>>((const _Float16*) d, inv, topk, npos, -1, out, nullptr);
    return HMOE_LAUNCHED("moe4t_forward");
}

extern "C" int hmoe_moe4t_forward(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt,
                                  int npos, int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw,
                                  const int64_t* gs, const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar,
                                  float* d, float* out, int ps, const int* meta, int T, int xf, const int* inv,
                                  int topk, void* stream)
{
    (void) eid; (void) gu;
    return moe4t_run(x, tok, wt, rbt, npos, nrb, n_tab, gw, uw, dw, gs, us, ds, ar, d, out, ps, meta, T, xf, inv, topk,
                     nullptr, stream);
}

extern "C" int hmoe_moe4t_forward_bf16(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt,
                                       int npos, int nrb, int n_tab, const int64_t* gw, const int64_t* uw,
                                       const int64_t* dw, const int64_t* gs, const int64_t* us, const int64_t* ds,
                                       float* gu, uint16_t* ar, float* d, float* out, int ps, const int* meta, int T,
                                       int xf, const int* inv, int topk, uint16_t* out_bf16, void* stream)
{
    (void) eid; (void) gu;
    HMOE_REQUIRE(out && out_bf16 && inv && T >= 1 && ((uintptr_t) out_bf16 & 7) == 0,
                 "moe4t_forward_bf16: needs out, the inverse map and an 8-byte aligned bf16 output");
    // no pick: the output is the partial alone (finish_bf16 rounds it and zeroes it)
    if (npos == 0) return hmoe_finish_bf16(out, T, out_bf16, stream);
    return moe4t_run(x, tok, wt, rbt, npos, nrb, n_tab, gw, uw, dw, gs, us, ds, ar, d, out, ps, meta, T, xf, inv, topk,
                     out_bf16, stream);
}

extern "C" int hmoe_moe4t_gemm(const void* xs, int rows, const int* rbt, int nrb, int n_tab, const int64_t* w0,
                               const int64_t* w1, const int64_t* s0, const int64_t* s1, float* out, int ps, int down,
                               void* stream)
{
    HMOE_REQUIRE(xs && rbt && out && w0 && s0 && (down || (w1 && s1)), "moe4t_gemm: null buffer");
    HMOE_REQUIRE(rows >= 1 && nrb >= 0 && ps >= rows && n_tab >= 1 && n_tab <= HMOE_MAXE,
                 "moe4t_gemm: rows %d nrb %d ps %d n_tab %d", rows, nrb, ps, n_tab);
    HMOE_REQUIRE((size_t) rows * (down ? I : H) * 2 <= UINT32_MAX, "moe4t_gemm: rows %d past the 4 GB input offsets",
                 rows);
    HMOE_REQUIRE(((uintptr_t) xs & 15) == 0 && ((uintptr_t) out & 15) == 0, "moe4t_gemm: alignment");
    if (nrb == 0) return HMOE_OK;
    hipStream_t st = (hipStream_t) stream;
    if (down)
        pgemm_kernel<1, 4, 2><<<pgemm_grid(nrb, H / 256), PT, 0, st>>>((const _Float16*) xs, nullptr, nullptr, rbt, nrb,
            nullptr, n_tab, w0, nullptr, s0, nullptr, nullptr, out, rows, 0, rows);
    else
        pgemm_kernel<2, 2, 2, EPI_RAW><<<pgemm_grid(nrb, I / 128), PT, 0, st>>>((const _Float16*) xs, nullptr, nullptr,
            rbt, nrb, nullptr, n_tab, w0, w1, s0, s1, nullptr, out, rows, 0, rows, nullptr, ps);
    return HMOE_LAUNCHED("moe4t_gemm");
}
