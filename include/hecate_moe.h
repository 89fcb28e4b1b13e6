/* hecate_moe.h - C ABI of the MI355X (gfx950) routed int4 MoE hot path: the drop-in for chronarion/hecate's GPU-tier
 * MoE operators (runtime/tier/moe4/moe4.cu, moe4p.cu, runtime/core/exl3_router.py).
 *
 * Conventions (kept from the reference's pybind ops, runtime/tier/moe4/moe4.cu:826-843):
 *   - every pointer is a device address unless the argument name ends in _host; sizes are plain ints;
 *   - expert weights are passed as int64 device tables of raw device addresses, one table per matrix and per scale
 *     (runtime/tier/tier_split.py:206-214, 246); the caller owns every buffer, the library never frees;
 *   - work is queued on `stream` (a hipStream_t; NULL = default stream), asynchronously, with a static launch shape
 *     and no allocation, host synchronisation or hipMemset, so the launches are hipGraph-capturable;
 *   - scratch buffers are workspace: no launch reads scratch it has not written in the same call, so any contents
 *     work (nothing needs zeroing) and calls that share one scratch must not overlap;
 *   - every entry point returns HMOE_OK or an error code; hmoe_last_error() gives the thread's last message.
 *
 * Formats (this build's gfx950 layouts, hmoe_pack_* produce them from the canonical row-major ones):
 *   I4G128 int4 matrix [N][K] (N % 16 == 0, K % 512 == 0): codes in 1 KB tiles of 16 rows x 128 k, tile (nb, kg) at
 *          byte (nb * K/128 + kg) * 1024; lane l (0..63) of a tile holds 16 bytes = 4 dwords, dword j packs the 8 codes
 *          (q + 8) of row nb*16 + l%16 at k = kg*128 + 32j + 8(l/16) + e, e = 0..7, code e at bit 4(e/2) + 16(e%2).
 *          Scales bf16, N x K/128 of them in 128-byte blocks of 16 rows x 4 k groups: the scale of row n, group g at
 *          byte ((n/16) * K/512 + g/4) * 128 + (n%16) * 8 + (g%4) * 2, so the 16 rows of a tile read their scales of
 *          one to four groups from one 128-byte line.
 *   F16T   dense matrix [N][K] (K % 32 == 0) as f16 in 1 KB tiles of 16 rows x 32 k, tile (nb, ks) at byte
 *          (nb * K/32 + ks) * 1024, lane l holds the 8 f16 of row nb*16 + l%16 at k = ks*32 + 8(l/16) + e.
 *   x      bf16 [R][H] (the MoE input); xh its f16 copy (exact for the reference's fp16 activation range).
 */
#ifndef HECATE_MOE_H
#define HECATE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HMOE_H 6144            /* hidden size (runtime/tier/moe4/moe4.cu:33) */
#define HMOE_I 2048            /* expert intermediate size */
#define HMOE_TOPK 8
#define HMOE_MAXR 16           /* decode rows per call (the reference's MAXR is 8; 8 requests + 8 draft rows need 16) */
#define HMOE_MAXE 256          /* expert ids per residency window */
#define HMOE_MAXSLOT 128       /* distinct experts per decode call (MAXR * TOPK) */

enum { HMOE_OK = 0, HMOE_ERR_ARG = 1, HMOE_ERR_HIP = 2 };

/* the x format flag `xf` of the decode and prefill ops. The reference's moe4.forward takes fp16 row-major x with xf = 0
 * and x in mma B-fragment order (as its fused norm kernel writes it) with xf = 1 (runtime/tier/moe4/moe4.cu:826); a C
 * ABI cannot see a dtype, so this build names each format: bf16 row-major (BASELINE's activation type), the
 * reference's fragment order (refused with HMOE_ERR_ARG: an NVIDIA mma layout, never produced on gfx950), and fp16
 * row-major (the reference's xf = 0 data; the Python mirror maps an fp16 tensor with xf = 0 to it) */
enum { HMOE_XF_BF16 = 0, HMOE_XF_FRAG = 1, HMOE_XF_F16 = 2 };

/* last error message of the calling thread ("" if none) */
const char* hmoe_last_error(void);
/* ABI version of this library */
int hmoe_version(void);

/* ---- formats (host) ------------------------------------------------------------------------------------------ */
/* canonical int4 (codes uint8 [N][K/2], code = q + 8, low nibble = even k, as runtime/tier/cpuband.cpp:3-4 and
 * tier_split.py:104-106; scales bf16 [N][K/128] row-major) -> I4G128. Replaces the reference's pack_u4
 * (tools/quant/gptq_int4.py:74-77) for this build's layout. */
int hmoe_pack_i4(const uint8_t* codes_host, const uint16_t* scales_host, int N, int K, void* q_host, void* s_host);
/* inverse of hmoe_pack_i4 (tier_split.py:98-101 _unpack_moe4 is the reference's inverse of its own packing) */
int hmoe_unpack_i4(const void* q_host, const void* s_host, int N, int K, uint8_t* codes_host, uint16_t* scales_host);
/* dense bf16 [N][K] -> F16T (the shared expert; bf16 -> f16 is exact for |w| in [2^-14, 65504]) */
int hmoe_pack_dense(const uint16_t* w_bf16_host, int N, int K, uint16_t* f16t_host);
/* the reference's moe4 weights (fragment-order int4, tools/quant/gptq_int4.py:74-77, with fp32 row scales,
 * tier_split.py:207-214) -> I4G128 with the row scale rounded to bf16 in every group */
int hmoe_repack_moe4(const uint8_t* frag_q_host, const float* row_scale_host, int N, int K, void* q_host, void* s_host);

/* ---- synthetic data on the device (include/hmoe_rng.h; no reference counterpart: seeded benchmark weights) ---- */
int hmoe_gen_i4(uint64_t key_q, uint64_t key_s, float sigma_s, int N, int K, void* q, void* s, void* stream);
int hmoe_gen_dense(uint64_t key, float sigma, int N, int K, void* f16t, void* stream);
/* out[i] = mean + sigma * z(key, i); dtype 0 = fp32, 1 = bf16 */
int hmoe_gen_normal(uint64_t key, int64_t n, float mean, float sigma, int dtype, void* out, void* stream);

/* ---- router: runtime/core/exl3_router.py:134-146 router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale) ----
 * x bf16 [R][K]; wt fp32 [E][K] (the transposed gate); bias fp32 [E] or NULL (selection only); logits fp32 scratch
 * of hmoe_router_scratch_bytes(R, E) bytes; ctr unused (kept for the argument position); sel int64 [R][topk]; rw f16
 * [R][topk] = f16(a * scale / (sum a + 1e-20)); xh optional f16 [R][K] copy of x for hmoe_moe4_forward(xf =
 * HMOE_XF_F16). Logits in fp32 with one fixed summation order (bit-reproducible): 8 segments of K/8, each the in-order
 * sum from 0 of 32-element fmaf chains (k ascending, from 0), the segment sums added in order from 0. Sigmoid, keys and
 * weights follow exl3_router.py:94-127 with the exp of include/hmoe_rng.h. R >= 1, E <= 256, topk <= 8, K % 256 == 0.
 * Scratch: R <= 16 rows use R x 256 fp32 (the reference's [8, 256] logits buffer, exl3_router.py:180, serves R <= 8),
 * more rows 8 x R x 256 (one plane per segment). */
size_t hmoe_router_scratch_bytes(int R, int E);
int hmoe_router_fused(const void* x, const float* wt, const float* bias, float* logits, int* ctr, int64_t* sel,
                      uint16_t* rw, int R, int K, int E, int topk, float scale, void* xh, void* stream);

/* ---- decode: runtime/tier/moe4/moe4.cu:828-895 moe4_forward ----
 * x [R][H] bf16 (xf = HMOE_XF_BF16) or fp16 (xf = HMOE_XF_F16, e.g. the router's copy); xf = HMOE_XF_FRAG (the
 * reference's fragment-order x) returns HMOE_ERR_ARG; sel int64 [R][8]; rw f16 [R][8];
 * picks with sel - lo in [0, n_hot) run, tables indexed by sel - lo hold I4G128 codes (gate/up [I][H], down [H][I])
 * and their scales; y fp32 [R][H] is accumulated into. sh_gw / sh_uw / sh_dw: the shared expert as F16T (gate/up
 * [I][H], down [H][I]) or NULL; sh_gs / sh_us / sh_ds must be NULL (the reference's int8 row scales; F16T has none).
 * Scratch (act, gu32, ctr_a, y32, ctr_b) from hmoe_moe4_scratch_bytes (gu32 and ctr_b unused, kept for the argument
 * positions). blocks: grid size of the gate/up and down kernels (0 = one workgroup per CU; with the shared expert
 * the gate/up grid is fixed at 256, and the down grid is kept in [192, 384]), blocks_a: unused. The shared expert
 * runs inside the routed launches, ahead of the routed items. R in [1, 16]. */
size_t hmoe_moe4_scratch_bytes(int which);      /* which: 0 act, 1 gu32, 2 ctr_a, 3 y32, 4 ctr_b */
int hmoe_moe4_forward(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                      const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                      const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s,
                      void* act, float* gu32, int* ctr_a, float* y32, int* ctr_b, float* y, int blocks, int blocks_a,
                      int lo, const void* sh_gw, const void* sh_uw, const void* sh_dw, const void* sh_gs,
                      const void* sh_us, const void* sh_ds, int xf, void* stream);
/* hmoe_moe4_forward without workspace arguments: no counterpart in the reference. For callers that cannot allocate
 * (code under hipGraph capture, serving loops or harnesses that forbid hipMalloc): act, the part count and the part
 * partials live in one static device array of hmoe_moe4_noalloc_bytes() bytes (21,762,048: sized for R <= 16 rows;
 * more rows return HMOE_ERR_ARG), which each GPU the library runs on holds until the process ends. The call allocates
 * nothing and frees nothing. Every call on a GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams, other threads) race; nothing in it needs clearing (each launch reads only what the call wrote). The
 * other arguments are those of hmoe_moe4_forward, with blocks = 0. */
size_t hmoe_moe4_noalloc_bytes(void);
int hmoe_moe4_forward_noalloc(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                              const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                              const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s, float* y, int lo,
                              const void* sh_gw, const void* sh_uw, const void* sh_dw, int xf, void* stream);
/* the two phases of hmoe_moe4_forward, for callers that time or schedule them apart (this build's addition):
 * gate_up writes act (with the shared expert: also its fp32 gate and up sums, in act) and, in act, the step's routing
 * record (distinct expert count and the local expert of each act slot); down adds into y (above one row ctr_b
 * carries its part count to the ordered sum), taking the slots from that record, so it must follow a gate_up of the
 * same step on the same act (sel, rw and lo are accepted for the argument positions); same arguments and rules as
 * forward otherwise */
int hmoe_moe4_gate_up(const void* x, const int64_t* sel, const uint16_t* rw, int R, int n_hot,
                      const int64_t* gate_w, const int64_t* up_w, const int64_t* gate_s, const int64_t* up_s,
                      void* act, float* gu32, int* ctr_a, int blocks, int lo, const void* sh_gw, const void* sh_uw,
                      int xf, void* stream);
int hmoe_moe4_down(const int64_t* sel, const uint16_t* rw, int R, int n_hot, const int64_t* down_w,
                   const int64_t* down_s, const void* act, float* y32, int* ctr_b, float* y, int blocks, int lo,
                   const void* sh_dw, void* stream);
/* the whole decode layer in the four launches of forward (this build's addition; tier_split.py:520-574 runs the
 * router, the shared expert and moe4 apart): router logits (wt fp32 [E][H], bias) with the router_fused rules, the
 * selection written to sel / rw (int64 / f16 [R][8]), routed experts of the picks in [lo, lo + n_hot) and the shared
 * expert (F16T or NULL); y fp32 [R][H] accumulated into and / or out bf16 [R][H] written (either may be NULL, not
 * both). x bf16 [R][H]. phases: bit mask of the four launches (1 router logits, 2 selection + shared and routed
 * gate/up, 4 shared and routed down, 8 output), 15 = the whole layer. At one row the down launch owns its output
 * rows and writes y / out itself (the layer is three launches; bit 8 then launches nothing); bit 16 takes the
 * part-sum form (down partials, then the ordered output launch) at any row count, with the same bits. topk must
 * be 8. */
int hmoe_moe_decode_layer(const void* x, const float* wt, const float* bias, int E, int topk, float scale,
                          float* logits, int64_t* sel, uint16_t* rw, int R, int n_hot, int lo,
                          const int64_t* gate_w, const int64_t* up_w, const int64_t* down_w,
                          const int64_t* gate_s, const int64_t* up_s, const int64_t* down_s,
                          const void* sh_gw, const void* sh_uw, const void* sh_dw, void* act, float* gu32,
                          int* ctr_a, float* y32, float* y, uint16_t* out, int blocks, int phases, void* stream);
/* moe4.cu:700-717,817-824: f[r] += y[r] (+ o[r]) (+ o2[r]) in that order, y zeroed; o, o2 may be NULL. done must be
 * NULL (the cross-device DONE flag is out of scope). f, y fp32 [rows][H]. */
int hmoe_moe4_combine(float* f, const float* o, float* y, int rows, const float* o2, const unsigned* done, void* stream);
/* moe4.cu:678-698,904-911: I4G128 codes + scales -> f16 [N][K] (value (q) * scale, rounded to f16) */
int hmoe_moe4_dequant(const void* q, const void* s, int N, int K, uint16_t* out, void* stream);
/* y fp32 [rows][H] -> bf16 out (the layer output), y zeroed (the combine's self-cleaning, this build's addition) */
int hmoe_finish_bf16(float* y, int rows, uint16_t* out, void* stream);

/* ---- prefill dispatch: runtime/tier/tier_split.py:400-420 (argsort, bincount, tok/eid/wt) and
 * runtime/tier/rtx_split.py:236-255 (pick_groups) on the device, with no host sync ----
 * sel int64 [T][topk], rw f16 [T][topk]; window [lo, lo + n). Outputs: counts int32 [n], tok/eid int32 [T*topk],
 * wt fp32 [T*topk], inv int32 [T*topk] (position of each flat pick, -1 outside the window), rbt int32 [nrb_max][4]
 * rows {expert, first pick, picks, 0} with bm rows per block (balance as pick_groups), meta int32 [4] = {npos, nrb,
 * 0, 0}. work: scratch of hmoe_dispatch_work_bytes(T, topk, n) bytes. nrb_max = hmoe_dispatch_nrb_max(T*topk, n, bm).
 * bm in [1, 256] (the reference uses 64 for moe4p and 256, balanced, for moe4t: tier_split.py:417,449,457). */
size_t hmoe_dispatch_work_bytes(int T, int topk, int n);
int hmoe_dispatch_nrb_max(int npos_max, int n, int bm);
int hmoe_dispatch(const int64_t* sel, const uint16_t* rw, int T, int topk, int lo, int n, int bm, int balance,
                  int* counts, int* tok, int* eid, float* wt, int* inv, int* rbt, int nrb_max, int* meta, void* work,
                  void* stream);

/* ---- prefill: runtime/tier/moe4/moe4p.cu:217-245 moe4p_forward(x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar,
 * d, out) ----
 * x bf16 [T][H] (xf = HMOE_XF_BF16) or fp16 (xf = HMOE_XF_F16, e.g. router_fused's copy; HMOE_XF_FRAG is refused);
 * tok int32 [npos] (token of each pick),
 * eid int32 [npos] (not read: the expert of a row block is in
 * rbt), wt fp32 [npos]; rbt int32 [nrb][4] rows {expert (relative to the tables), first pick, picks <= 256, 0} (a
 * block of more than 128 picks runs as two halves in one workgroup; the dispatch's bm is at most 256);
 * tables (n_tab entries) as in hmoe_moe4_forward; ar f16 [ps + T][I] and d fp32 [ps + T][H] scratch
 * (hmoe_moe4p_scratch_bytes); gu (16-byte aligned, hmoe_moe4p_scratch_bytes(0) bytes): the f16 copy of x [T][H]
 * when x is bf16 (NULL allowed for fp16 x); out fp32 [T][H] accumulated into. meta: NULL, or the device
 * {npos, nrb} written by hmoe_dispatch (then npos / nrb are the static maxima the grids are sized for). inv: NULL
 * (picks added with atomics, as p4_fin_kernel) or the dispatch's inverse map (each token's picks added in top-k
 * order: deterministic). sh_*: the shared expert as row-major f16 (gate [I][H], up [I][H], down [H][I]) or NULL
 * (needs inv); it runs on every token with weight 1 on dense MFMA GEMMs (fp32 accumulation; act rows ps.. and d
 * rows ps.. hold its SwiGLU and down output, added after each token's picks). T = 0 with npos = 0 is a no-op. */
size_t hmoe_moe4p_scratch_bytes(int which, int ps, int T);     /* which: 0 gu, 1 ar, 2 d */
int hmoe_moe4p_forward(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt, int npos,
                       int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw, const int64_t* gs,
                       const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar, float* d, float* out, int ps,
                       const int* meta, const int* inv, int T, int topk, const void* sh_gw, const void* sh_uw,
                       const void* sh_dw, int xf, void* stream);
/* No counterpart in the reference: hmoe_moe4p_forward into a zero partial followed by hmoe_finish_bf16, in one
 * combine pass, for callers with no partial to add (the layer's own prefill). Arguments as hmoe_moe4p_forward without out; inv is required; out_bf16 bf16 [T][H] (8-byte aligned)
 * gets bf16(sum of each token's picks in top-k order + shared row), bit-identical to the two-op form. */
int hmoe_moe4p_forward_bf16(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt, int npos,
                            int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw,
                            const int64_t* gs, const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar, float* d,
                            int ps, const int* meta, const int* inv, int T, int topk, const void* sh_gw,
                            const void* sh_uw, const void* sh_dw, int xf, uint16_t* out_bf16, void* stream);

/* ---- long prefill: runtime/tier/moe4/moe4t.cu:490-524 moe4t_scratch(device, npos) / moe4t_forward(x, tok, eid, wt,
 * rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out) ----
 * As hmoe_moe4p_forward for the chunks the reference sends to moe4t (more than 2048 rows, tier_split.py:427-462,543):
 * row blocks of up to 256 picks (hmoe_dispatch with bm = 256 and balance, as pick_groups(..., 256, True)). inv NULL:
 * the down GEMM adds its rows into out[tok] itself (fp32 atomics, the reference's fused epilogue, moe4t.cu:514-516),
 * so the order of the adds into out varies run to run; inv = the dispatch's inverse map (this build's addition, with
 * topk): the down rows go to d and each token adds its picks in top-k order (deterministic, and cheaper on gfx950
 * than scattered fp32 atomics). Scratch
 * (hmoe_moe4t_scratch_bytes(which, npos)): gu fp32 [2][npos][I] (unused, kept for the argument), ar f16 [npos][I],
 * d fp32 [1][npos][H] (the reference's size; the kernels write f16 rows into it, the copy of x when x is bf16 and with
 * inv each pick's down row, so npos * H * 2 bytes suffice; the reference gathers the picks' rows into it).
 * T: rows of x and out; meta as in moe4p (the device plan's {npos, nrb}, or NULL); no shared expert (the reference
 * runs it apart at prefill: hmoe_shared_forward). npos = 0 is a no-op (moe4t.cu:508). */
size_t hmoe_moe4t_scratch_bytes(int which, int npos);      /* which: 0 gu, 1 ar, 2 d */
int hmoe_moe4t_forward(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt, int npos,
                       int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw, const int64_t* gs,
                       const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar, float* d, float* out, int ps,
                       const int* meta, int T, int xf, const int* inv, int topk, void* stream);
/* No counterpart in the reference: hmoe_moe4t_forward (with inv) followed by hmoe_finish_bf16, in one combine pass:
 * out_bf16 bf16 [T][H] (8-byte aligned) = bf16(out + each token's picks in top-k order) and out zeroed, bit-identical
 * to the two-op form; npos = 0 gives finish_bf16 of out alone. For the layer's long prefill (the shared expert added
 * into out first). */
int hmoe_moe4t_forward_bf16(const void* x, const int* tok, const int* eid, const float* wt, const int* rbt, int npos,
                            int nrb, int n_tab, const int64_t* gw, const int64_t* uw, const int64_t* dw,
                            const int64_t* gs, const int64_t* us, const int64_t* ds, float* gu, uint16_t* ar, float* d,
                            float* out, int ps, const int* meta, int T, int xf, const int* inv, int topk,
                            uint16_t* out_bf16, void* stream);
/* runtime/tier/moe4/moe4t.cu:476-488 moe4t_gemm(xs, rbt, w0, w1, out, down), the test entry: one grouped GEMM over
 * row blocks of <= 256 picks whose inputs are rows p of xs f16 [rows][K]. Gate/up shape (down = 0, K = H): out fp32
 * [2][ps][I] = the gate (w0, s0) and up (w1, s1) sums; down shape (down = 1, K = I): out fp32 [ps][H] (w0, s0). The
 * reference writes raw sums and applies its per-row scale later; with group-128 scales there is no row factor, so
 * the sums here include the group scales. */
int hmoe_moe4t_gemm(const void* xs, int rows, const int* rbt, int nrb, int n_tab, const int64_t* w0, const int64_t* w1,
                    const int64_t* s0, const int64_t* s1, float* out, int ps, int down, void* stream);

/* ---- the shared expert alone over a chunk (this build's addition: the reference runs it through the model's own
 * shared-expert MLP at prefill, runtime/tier/tier_split.py:548-560, next to moe4t): out fp32 [T][H] += down(silu(gate
 * x) * up x), x bf16 / fp16 [T][H] (xf as above), the weights row-major f16 (gate [I][H], up [I][H], down [H][I]);
 * work: hmoe_shared_work_bytes(T) bytes, 256-byte aligned (the f16 copy of x, act f16 [T][I]). Every output
 * element is added once, by the down GEMM's epilogue: deterministic. */
size_t hmoe_shared_work_bytes(int T);
int hmoe_shared_forward(const void* x, int T, const void* sh_gw, const void* sh_uw, const void* sh_dw, void* work,
                        float* out, int xf, void* stream);

/* ---- residual + RMSNorm: runtime/tier/cn.cu and runtime/core/nr4_kernel.cuh ----
 * Every RMSNorm here uses the reduction order of the reference's rms_norm_kernel, which its fused kernels reproduce
 * bit for bit (cn.cu:1-6,21-31,80-103; nr4_kernel.cuh:4-9): a row is H / 4 = 1536 float4 columns, chain t of 1024
 * is one fmaf chain from 0 over the elements of columns t and t + 1024 (t < 512), the chains of each group of 32 are
 * summed by an xor butterfly (offsets 16, 8, 4, 2, 1), the 32 group sums by the same butterfly;
 * rmf = 1 / sqrt(sum / H + eps) * cscale (the reference's rsqrtf, fast math there, as the correctly rounded 1 / sqrt
 * here), xn = (r * (w + cbias)) * rmf with cbias added only when nonzero, rounded to the output type. w: fp32, bf16 or
 * f16 [H] (w_dtype); xn: bf16 or f16 [rows][H] (xn_dtype). Rows are 16-byte aligned fp32, xn 8-byte aligned. */
enum { HMOE_DT_F32 = 0, HMOE_DT_BF16 = 1, HMOE_DT_F16 = 2 };
/* runtime/tier/cn.cu:189-235 combine_norm(f, o_ptr, y, rows, o2_ptr, done_ptr, r, w, xn, eps, cbias, cscale): the MoE
 * combine of a layer fused into the next input norm, one workgroup per row: a = ((f + y) + o) + o2 (f may be NULL, read
 * as +0 as combine_norm_pdl does, cn.cu:105-110; o, o2 may be NULL), y zeroed, r = a + r, xn = RMSNorm(r). f, y, o, o2,
 * r fp32 [rows][H]; rows in [1, 64]. done must be NULL (the RTX band's DONE flag: that band is not built). */
int hmoe_combine_norm(const float* f, const float* o, float* y, int rows, const float* o2, const unsigned* done,
                      float* r, const void* w, void* xn, float eps, float cbias, float cscale, int w_dtype,
                      int xn_dtype, void* stream);
/* runtime/core/exl3_normroute.py:16-65 norm_route(y, r, w, x2, gt, bias, sel, rw, cand, ctr, scale, eps, cbias, cscale,
 * ho) (nr4_kernel.cuh:122-381): the post-attention residual add and RMSNorm, then the router on the normed rows:
 * r = y + r (y fp32 [R][H], read only), x2 = RMSNorm(r) (bf16 or f16, x2_dtype), logits of x2 against gt ([E][H],
 * fp32 or the reference's f16, gt_dtype) in router_fused's fixed order, sel int64 / rw f16 [R][8] by router_fused's
 * rules (sigmoid + bias keys, ties to the lowest index, rw = f16(a * scale / (sum a + 1e-20))). cand: logits scratch of
 * hmoe_norm_route_scratch_bytes(R, E) bytes (the reference's candidate buffer has the same role); ctr unused (kept for
 * the argument position). ho (n_ho words, host memory): the band hand-off. The reference's 10 / 11 words address its RTX
 * and Grace bands' slots and flags (exl3_normroute.py:38-47), which this build does not have; here n_ho is 0 (no
 * hand-off) or 2, {mailbox, layer}: the selection launch also posts the CPU tier's job as hmoe_cpu_submit does (waits
 * for the pool's previous job, copies x2 and the routing into the mailbox, releases issue), which nr4_kernel.cuh:
 * 360-378 does for the reference's Grace band; it needs bf16 x2, R <= HMOE_CPU_MAXR and 16-byte aligned sel / rw.
 * R in [1, 16] (the reference: 2..8), E in [8, 256]. Three launches: the norm (one workgroup per row), the logits (two
 * experts per workgroup), the selection (with the post); r and x2 are those of hmoe_combine_norm's norm, the routing
 * that of hmoe_router_fused on x2. */
size_t hmoe_norm_route_scratch_bytes(int R, int E);
int hmoe_norm_route(const float* y, float* r, const void* w, void* x2, const void* gt, const float* bias, int64_t* sel,
                    uint16_t* rw, float* cand, int* ctr, float scale, float eps, float cbias, float cscale,
                    const int64_t* ho, int n_ho, int R, int E, int w_dtype, int x2_dtype, int gt_dtype, void* stream);
/* the decode layer's output launch fused with the next layer's input norm (this build's addition: cn.cu:48-103's
 * combine-into-norm for the part-sum decode form): s = the down launch's part partials (y32, their count in ctr_a, as
 * hmoe_moe_decode_layer left them with phases 2 | 4 at R > 1, or with bit 16 at any R) summed in part order, r = s + r
 * (the bits of that layer's output launch adding into r), xn = RMSNorm(r) as above, xh optional f16 copy of xn. R in
 * [1, 16]. */
int hmoe_decode_combine_norm(const float* y32, const int* ctr_a, int R, float* r, const void* w, void* xn, void* xh,
                             float eps, float cbias, float cscale, int w_dtype, int xn_dtype, void* stream);
/* residual + RMSNorm between layers (cn.cu:80-103 with the layer output as a): r = a + r (a fp32 [R][H] or NULL; a is
 * zeroed after use), xn = bf16 RMSNorm(r) with fp32 w, cbias 0, cscale 1; xh optional f16 copy of xn. */
int hmoe_residual_rmsnorm(float* r, float* a, const float* w, int R, float eps, uint16_t* xn, uint16_t* xh,
                          void* stream);
/* ---- RMSNorm + router logits in one launch: runtime/tier/nr4_kernel.cuh:122-381 (nr4_kernel: norm, router scores) --
 * h fp32 [R][H] (the residual, read only; R <= 16), norm_w fp32 [H]: xn = bf16 RMSNorm(h) (bit-identical to
 * hmoe_residual_rmsnorm with a = NULL), xh optional f16 copy of xn, and the router logits of xn into logits, as phase 1
 * of hmoe_moe_decode_layer computes them; run hmoe_moe_decode_layer on xn with the same logits and phases 14 to finish
 * the layer. Passing y = h to that call adds the layer's output into the residual (the combine of cn.cu:48-103), so a
 * decode stack at one row needs three launches per layer. */
int hmoe_norm_router(const float* h, const float* norm_w, float eps, int R, const float* wt, int E, float* logits,
                     uint16_t* xn, void* xh, void* stream);

/* ---- host-CPU expert tier: runtime/tier/cpuband.cpp (cb_start :241, cb_add_layer :228, cb_stats :254, cb_stop :256,
 * the job of worker :113-223) for x86 hosts ----
 * A pool of host threads serves decode jobs of <= HMOE_CPU_MAXR rows from a mailbox: the cold experts of the job's
 * layer (ids in [lo, lo + n)) with q8_0 activations and int4 x int8 dot products (the arithmetic of cpuband.cpp with
 * bf16 group-128 scales), the fp32 partial into out. The mailbox is any host memory the pool can read; for the GPU
 * hand-off it must be pinned and device-mapped (hipHostMalloc, mapped + coherent).
 * Protocol (generation numbers, as cpuband.cpp:117-136,221 with ISSUE gen / CPU_DONE = gen): a poster may post when
 * done == issue (the last job finished); it fills rows, layer, sel, rw and x, then stores issue = issue + 1 (release;
 * 0 is skipped on wrap-around). Each pool thread remembers the last generation it served and runs a job when issue
 * differs from it; after the job's last barrier the pool writes out and err (0; 1 for a row count outside [1, 8], 2
 * for a layer it does not hold, with out zero) and stores done = the job's generation (release). A waiter waits for
 * done == the generation it posted: a stale value of done (an older job, or any other number) never satisfies it.
 * With HMOE_CPU_SKIP=1 in the environment at pool start, jobs are acknowledged with a zero partial (the timing
 * diagnostic of cpuband.cpp:40,249). */
#define HMOE_CPU_MAXR 8        /* rows per CPU job (cpuband.cpp:7, 154: MAXR = 8) */
typedef struct hmoe_cpu_mailbox
{
    uint32_t issue;                               /* generation of the last posted job (own 128-byte line) */
    uint32_t pad0[31];
    uint32_t done;                                /* generation of the last finished job (own 128-byte line) */
    uint32_t pad1[31];
    int32_t rows, layer, err;                     /* job header, written before issue */
    int32_t gpu_err;                              /* sticky, set by the GPU side: 1 a collect's wait ran out (partial
                                                     not added), 2 a hand-off found the pool busy (job not posted;
                                                     later collects add nothing while it is set); the host reads and
                                                     clears it */
    int32_t pad2[28];
    int64_t sel[HMOE_CPU_MAXR * HMOE_TOPK];       /* global expert ids [rows][8] */
    uint16_t rw[HMOE_CPU_MAXR * HMOE_TOPK];       /* f16 routing weights [rows][8] */
    uint16_t x[HMOE_CPU_MAXR * HMOE_H];           /* bf16 rows */
    float out[HMOE_CPU_MAXR * HMOE_H];            /* fp32 partial [rows][H] */
} hmoe_cpu_mailbox;
/* start the pool (threads >= 1, pinned to cores first_core + t when first_core >= 0) on a mailbox; one pool per process.
 * The pool serves the jobs posted after it starts (it takes the mailbox's issue as already served). A test hook:
 * HMOE_CPU_HOLD="t,usec" in the environment at start makes pool thread t sleep usec after each job before it looks
 * for the next (the window in which a fast poster re-posts), in steps that watch for hmoe_cpu_stop. */
int hmoe_cpu_start(hmoe_cpu_mailbox* mb, int threads, int first_core);
/* the cold experts of a layer, host memory: q[3 e + {0, 1, 2}] the row-major int4 codes (cpuband.cpp:3-4: [N][K/2],
 * low nibble first) of gate [I][H], up [I][H], down [H][I] of cold expert e (id lo + e), s[...] their bf16 [N][K/128]
 * scales; the pool keeps the pointers (the caller keeps the memory alive). Every pointer is checked before the layer
 * changes, so a refused call leaves the pool's layers as they were. Only while no job is in flight. */
int hmoe_cpu_add_layer(int layer, int lo, int n, const uint8_t* const* q, const uint16_t* const* s);
int hmoe_cpu_stats(long long* jobs, long long* picks);
int hmoe_cpu_stop(void);
/* the GPU side of a job, one kernel each, capturable in a hipGraph. hmoe_cpu_submit: waits for done == issue (the
 * previous job finished), copies x bf16 [R][H], sel, rw (device, 16-byte aligned) into the mailbox, writes rows /
 * layer / err, then issue + 1 with a system-scope release (runtime/tier/moe4/moe4.cu:719-738 moe4_handoff_kernel).
 * hmoe_cpu_collect: waits for done == issue (the generation the submit before it posted, read from the mailbox) and
 * adds out into y fp32 [R][H] (runtime/tier/tier_split.py:577-644 tier_combine, the graph form's spinning combine).
 * Both waits are bounded (2 s of wall clock); past the bound the kernel sets gpu_err and returns; a collect adds
 * nothing while gpu_err is set. The mailbox must come from hmoe_cpu_mailbox_alloc (or be otherwise device-mapped). */
int hmoe_cpu_submit(hmoe_cpu_mailbox* mb, const void* x, const int64_t* sel, const uint16_t* rw, int R, int layer,
                    void* stream);
int hmoe_cpu_collect(hmoe_cpu_mailbox* mb, float* y, int R, void* stream);
/* runtime/tier/cn.cu:108-142 combine_norm_pdl's CPU_DONE form for this build's CPU tier: hmoe_combine_norm with the
 * pool's partial (the mailbox's out) in the o2 position, added once the job the last post (hmoe_norm_route with a
 * hand-off, or hmoe_cpu_submit) issued has finished: a = ((f + y) + o) + out, y zeroed, r = a + r, xn = RMSNorm(r).
 * The wait is bounded as hmoe_cpu_collect's; past it, or with gpu_err already set, out is not added and gpu_err says
 * so. rows in [1, HMOE_CPU_MAXR] (the job's rows). With the post folded into the norm + router and the collect into
 * this combine, a tiered layer needs no launch of its own for the hand-off. */
int hmoe_combine_norm_cpu(const float* f, const float* o, float* y, int rows, hmoe_cpu_mailbox* mb, float* r,
                          const void* w, void* xn, float eps, float cbias, float cscale, int w_dtype, int xn_dtype,
                          void* stream);
/* a mapped, coherent pinned mailbox (hipHostMalloc) and its release */
int hmoe_cpu_mailbox_alloc(hmoe_cpu_mailbox** mb);
int hmoe_cpu_mailbox_free(hmoe_cpu_mailbox* mb);

#ifdef __cplusplus
}
#endif
#endif
