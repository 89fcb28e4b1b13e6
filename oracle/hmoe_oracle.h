/* hmoe_oracle.h - CPU restatement of chronarion/hecate's routed int4 MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the CPU baseline: only tests/, the smoke() of
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it. The product path (hecate_amd/) never calls it.
 *
 * Formats (host, canonical):
 *   x        bf16 [R][H]
 *   codes    uint8 [N][K/2], row-major, code = q + 8, low nibble = even k (runtime/tier/cpuband.cpp:3-4)
 *   scales   bf16 [N][K/128] group-128 scales (the benchmark format; the reference keeps fp32 per row)
 *   shared   bf16 [N][K] dense
 *   sel      int64 [R][topk], rw f16 [R][topk]
 * Every function cites the reference lines it restates.
 */
#ifndef HMOE_ORACLE_H
#define HMOE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fixed summation order of the router logits: SEGMENTS folds of (K / SEGMENTS / CHUNK) sequential fmaf chains of
 * CHUNK elements each */
#define ORC_ROUTER_CHUNK 32
#define ORC_ROUTER_SEGMENTS 8

/* ---- synthetic data (include/hmoe_rng.h) ---- */
void orc_gen_normal_f32(uint64_t key, int64_t n, float mean, float sigma, float* out);
void orc_gen_normal_bf16(uint64_t key, int64_t n, float sigma, uint16_t* out);
void orc_gen_codes(uint64_t key, int N, int K, uint8_t* out);
void orc_gen_scales(uint64_t key, int N, int K, float sigma, uint16_t* out);
uint64_t orc_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t expert);
void orc_f32_to_bf16(const float* in, int64_t n, uint16_t* out);
void orc_f32_to_f16(const float* in, int64_t n, uint16_t* out);
void orc_f16_to_f32(const uint16_t* in, int64_t n, float* out);
float orc_expf(float x);

/* ---- router: exl3_router.py:86-131, nr4_kernel.cuh:307-366 ---- */
/* the same order on fp32 rows (x widened exactly from bf16 or f16 by the caller) */
void orc_router_logits_f32(const float* x, const float* w, int R, int K, int E, float* logits);
void orc_router_logits(const uint16_t* x, const float* w, int R, int K, int E, float* logits);
void orc_router_select(const float* logits, const float* bias, int R, int E, int topk, float scale,
                       int64_t* sel, uint16_t* rw);

/* ---- dispatch: tier_split.py:400-420 (stable order, counts, tok/eid/wt) ---- */
int orc_dispatch(const int64_t* sel, const uint16_t* rw, int T, int topk, int lo, int n, int64_t* counts,
                 int32_t* tok, int32_t* eid, float* wt, int32_t* inv);
/* rtx_split.py:236-255 pick_groups for one group covering every pick (npos >= total): rbt int32 [nrb][4] */
int orc_pick_groups(const int64_t* counts, int n, int bm, int balance, int32_t* rbt, int cap);

/* ---- expert layer: cpuband.cpp:137-221 ----
 * picks are taken in first appearance over rows then top-k (cpuband.cpp:163-170); tables hold host addresses indexed
 * by local id (sel - lo), [0, n_hot). mode 0 = exact (fp32 activations, fp64 accumulation), 1 = q8_0 (faithful int8
 * activations and integer dot products). out [R][H] fp32: out = (accumulate ? out : 0) + routed (+ shared). */
int orc_moe(int mode, int R, int H, int I, const uint16_t* x, const int64_t* sel, const uint16_t* rw, int topk,
            int lo, int n_hot, const uint64_t* gq, const uint64_t* gs, const uint64_t* uq, const uint64_t* us,
            const uint64_t* dq, const uint64_t* ds, const uint16_t* sh_g, const uint16_t* sh_u, const uint16_t* sh_d,
            int accumulate, float* out, int threads);
/* the picks of a job in cpuband order: returns P, fills pick[P], wgt[P][R] */
int orc_picks(const int64_t* sel, const uint16_t* rw, int R, int topk, int lo, int n_hot, int32_t* pick, float* wgt);

/* ---- dequant (moe4.cu:679-698 restated for g128): codes + scales -> fp32 [N][K] ---- */
void orc_dequant(const uint8_t* codes, const uint16_t* scales, int N, int K, float* out);

/* ---- RMSNorm in the reference's rms_norm_kernel order (cn.cu:21-31,80-103; nr4_kernel.cuh:176-243) ---- */
float orc_rms_sum(const float* v, int H);
void orc_rmsnorm_cn(const float* v, const float* w, int R, int H, float eps, float cbias, float cscale, int xn_bf16,
                    uint16_t* xn);
/* r = a + r (a may be NULL), then orc_rmsnorm_cn (cbias 0, cscale 1, bf16 out) */
void orc_residual_rmsnorm(float* r, const float* a, const float* w, int R, int H, float eps, uint16_t* xn_bf16);

#ifdef __cplusplus
}
#endif
#endif
