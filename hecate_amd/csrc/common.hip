// common.hip - error state of the C ABI, host packers of the gfx950 layouts, device generators of the seeded
// synthetic layer, dequant, combine and bf16 finish (the residual + RMSNorm kernels are in norm.hip).
#include "hmoe_dev.h"
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

namespace hmoe {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_check(hipError_t e, const char* what)
{
    if (e == hipSuccess) return HMOE_OK;
    return set_error(HMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ---------------------------------------------------------------------------------------------------------------
// I4G128 / F16T packing (host). Nibble position of element e of a dword: 4(e/2) + 16(e%2), matching dq8().
// ---------------------------------------------------------------------------------------------------------------
static inline int nib_shift(int e) { return 4 * (e >> 1) + 16 * (e & 1); }

static inline uint32_t canon_code(const uint8_t* codes, int K, int n, int k)
{
    const uint8_t b = codes[(size_t) n * (K / 2) + k / 2];
    return (k & 1) ? (b >> 4) : (b & 15u);
}

// ---------------------------------------------------------------------------------------------------------------
// device generators (include/hmoe_rng.h)
// ---------------------------------------------------------------------------------------------------------------
__global__ void gen_i4_kernel(uint64_t key_q, uint64_t key_s, float sigma_s, int N, int K, u32x4* __restrict__ q,
                              uint16_t* __restrict__ s)
{
    const int KG = K / 128;
    const size_t lanes = (size_t) (N / 16) * KG * 64;
    for (size_t i = blockIdx.x * (size_t) blockDim.x + threadIdx.x; i < lanes; i += (size_t) gridDim.x * blockDim.x)
    {
        const int l = (int) (i & 63);
        const size_t tile = i >> 6;
        const int kg = (int) (tile % KG), nb = (int) (tile / KG);
        const int row = nb * 16 + (l & 15);
        u32x4 v;
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int k0 = kg * 128 + 32 * j + 8 * (l >> 4);
            const uint64_t flat = (uint64_t) row * (uint64_t) K + (uint64_t) k0;
            const uint64_t h = hmoe_bits(key_q, flat >> 4) >> (4u * (uint32_t) (flat & 15u));
            uint32_t word = 0u;
            #pragma unroll
            for (int e = 0; e < 8; ++e) word |= (uint32_t) ((h >> (4 * e)) & 15u) << (4 * (e >> 1) + 16 * (e & 1));
            v[j] = word;
        }
        q[i] = v;
        if (l < 16)
        {
            const int r = nb * 16 + l;
            s[sc_index(r, kg, KG)] = hmoe_f2bf(fabsf(sigma_s * hmoe_normal(key_s, (uint64_t) r * KG + kg)));
        }
    }
}

__global__ void gen_dense_kernel(uint64_t key, float sigma, int N, int K, f16x8* __restrict__ out)
{
    const int KS = K / 32;
    const size_t lanes = (size_t) (N / 16) * KS * 64;
    for (size_t i = blockIdx.x * (size_t) blockDim.x + threadIdx.x; i < lanes; i += (size_t) gridDim.x * blockDim.x)
    {
        const int l = (int) (i & 63);
        const size_t tile = i >> 6;
        const int ks = (int) (tile % KS), nb = (int) (tile / KS);
        const int row = nb * 16 + (l & 15);
        const int k0 = ks * 32 + 8 * (l >> 4);
        f16x8 v;
        #pragma unroll
        for (int e = 0; e < 8; ++e)
        {
            const uint16_t b = hmoe_f2bf(sigma * hmoe_normal(key, (uint64_t) row * K + k0 + e));
            v[e] = (_Float16) bf2f(b);
        }
        out[i] = v;
    }
}

__global__ void gen_normal_kernel(uint64_t key, int64_t n, float mean, float sigma, int dtype, void* out)
{
    for (int64_t i = blockIdx.x * (int64_t) blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x)
    {
        const float z = hmoe_normal(key, (uint64_t) i);
        if (dtype == 0) ((float*) out)[i] = mean + sigma * z;
        else ((uint16_t*) out)[i] = hmoe_f2bf(sigma * z);
    }
}

// I4G128 -> f16 [N][K] = f16(q * s)
__global__ void dequant_kernel(const u32x4* __restrict__ q, const uint16_t* __restrict__ s, int N, int K,
                               _Float16* __restrict__ out)
{
    const int KG = K / 128;
    const size_t lanes = (size_t) (N / 16) * KG * 64;
    for (size_t i = blockIdx.x * (size_t) blockDim.x + threadIdx.x; i < lanes; i += (size_t) gridDim.x * blockDim.x)
    {
        const int l = (int) (i & 63);
        const size_t tile = i >> 6;
        const int kg = (int) (tile % KG), nb = (int) (tile / KG);
        const int row = nb * 16 + (l & 15);
        const float sc = bf2f(s[sc_index(row, kg, KG)]);
        const u32x4 v = q[i];
        const DqConsts dq = dq_consts();
        #pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const f16x8 d = dq8(v[j], dq);
            const int k0 = kg * 128 + 32 * j + 8 * (l >> 4);
            #pragma unroll
            for (int e = 0; e < 8; ++e) out[(size_t) row * K + k0 + e] = (_Float16) ((float) d[e] * sc);
        }
    }
}

// moe4.cu:702-717: f += y (+ o) (+ o2), y = 0
__global__ void combine_kernel(float* __restrict__ f, const float* __restrict__ o, float* __restrict__ y, int n,
                               const float* __restrict__ o2)
{
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= n) return;
    f32x4 a = *(f32x4*) (f + i);
    const f32x4 c = *(const f32x4*) (y + i);
    a += c;
    if (o) a += *(const f32x4*) (o + i);
    if (o2) a += *(const f32x4*) (o2 + i);
    *(f32x4*) (f + i) = a;
    *(f32x4*) (y + i) = (f32x4) {0.f, 0.f, 0.f, 0.f};
}

__global__ void finish_kernel(float* __restrict__ y, int n, uint16_t* __restrict__ out)
{
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= n) return;
    const f32x4 a = *(const f32x4*) (y + i);
    #pragma unroll
    for (int k = 0; k < 4; ++k) out[i + k] = hmoe_f2bf(a[k]);
    *(f32x4*) (y + i) = (f32x4) {0.f, 0.f, 0.f, 0.f};
}

static int grid_for(size_t n, int threads, int cap = 65536)
{
    size_t g = (n + threads - 1) / threads;
    if (g < 1) g = 1;
    if (g > (size_t) cap) g = cap;
    return (int) g;
}

}  // namespace hmoe

using namespace hmoe;

extern "C" const char* hmoe_last_error(void) { return g_err.c_str(); }
extern "C" int hmoe_version(void) { return 1; }

extern "C" int hmoe_pack_i4(const uint8_t* codes, const uint16_t* scales, int N, int K, void* q_host, void* s_host)
{
    HMOE_REQUIRE(codes && scales && q_host && s_host, "pack_i4: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 512 == 0, "pack_i4: shape %d x %d", N, K);
    const int KG = K / 128;
    uint32_t* q = (uint32_t*) q_host;
    uint16_t* s = (uint16_t*) s_host;
    for (int nb = 0; nb < N / 16; ++nb)
        for (int kg = 0; kg < KG; ++kg)
        {
            const size_t tile = (size_t) nb * KG + kg;
            for (int l = 0; l < 64; ++l)
                for (int j = 0; j < 4; ++j)
                {
                    const int row = nb * 16 + (l & 15), k0 = kg * 128 + 32 * j + 8 * (l >> 4);
                    uint32_t word = 0u;
                    for (int e = 0; e < 8; ++e) word |= canon_code(codes, K, row, k0 + e) << nib_shift(e);
                    q[(tile * 64 + l) * 4 + j] = word;
                }
        }
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < KG; ++g) s[sc_index(n, g, KG)] = scales[(size_t) n * KG + g];
    return HMOE_OK;
}

extern "C" int hmoe_unpack_i4(const void* q_host, const void* s_host, int N, int K, uint8_t* codes, uint16_t* scales)
{
    HMOE_REQUIRE(codes && scales && q_host && s_host, "unpack_i4: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 512 == 0, "unpack_i4: shape %d x %d", N, K);
    const int KG = K / 128;
    const uint32_t* q = (const uint32_t*) q_host;
    const uint16_t* s = (const uint16_t*) s_host;
    memset(codes, 0, (size_t) N * K / 2);
    for (int nb = 0; nb < N / 16; ++nb)
        for (int kg = 0; kg < KG; ++kg)
        {
            const size_t tile = (size_t) nb * KG + kg;
            for (int l = 0; l < 64; ++l)
                for (int j = 0; j < 4; ++j)
                {
                    const int row = nb * 16 + (l & 15), k0 = kg * 128 + 32 * j + 8 * (l >> 4);
                    const uint32_t word = q[(tile * 64 + l) * 4 + j];
                    for (int e = 0; e < 8; ++e)
                    {
                        const uint32_t c = (word >> nib_shift(e)) & 15u;
                        const int k = k0 + e;
                        codes[(size_t) row * (K / 2) + k / 2] |= (uint8_t) ((k & 1) ? (c << 4) : c);
                    }
                }
        }
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < KG; ++g) scales[(size_t) n * KG + g] = s[sc_index(n, g, KG)];
    return HMOE_OK;
}

extern "C" int hmoe_pack_dense(const uint16_t* w, int N, int K, uint16_t* out)
{
    HMOE_REQUIRE(w && out, "pack_dense: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0, "pack_dense: shape %d x %d", N, K);
    const int KS = K / 32;
    for (int nb = 0; nb < N / 16; ++nb)
        for (int ks = 0; ks < KS; ++ks)
            for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 8; ++e)
                {
                    const int row = nb * 16 + (l & 15), k = ks * 32 + 8 * (l >> 4) + e;
                    out[(((size_t) nb * KS + ks) * 64 + l) * 8 + e] = hmoe_f2h(hmoe_bf2f(w[(size_t) row * K + k]));
                }
    return HMOE_OK;
}

// reference fragment order (tools/quant/gptq_int4.py:74-77; inverse at runtime/tier/tier_split.py:98-101): uint4
// u = ((gr * K/64 + kb) * 4 + s) * 32 + lane, word t, nibble c*4 + h*2 + rh holds row (gr*4 + s)*16 + lane/4 + 8 rh,
// col kb*64 + t*16 + h*8 + (lane%4)*2 + c
extern "C" int hmoe_repack_moe4(const uint8_t* frag, const float* row_scale, int N, int K, void* q_host, void* s_host)
{
    HMOE_REQUIRE(frag && row_scale && q_host && s_host, "repack_moe4: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 64 == 0 && K % 512 == 0, "repack_moe4: shape %d x %d", N, K);
    const int KB = K / 64, KG = K / 128;
    uint8_t* codes = (uint8_t*) calloc((size_t) N * K / 2, 1);
    uint16_t* sc = (uint16_t*) malloc(sizeof(uint16_t) * (size_t) N * KG);
    if (!codes || !sc) { free(codes); free(sc); return set_error(HMOE_ERR_ARG, "repack_moe4: out of host memory"); }
    const uint32_t* w32 = (const uint32_t*) frag;
    for (int gr = 0; gr < N / 64; ++gr)
        for (int kb = 0; kb < KB; ++kb)
            for (int s = 0; s < 4; ++s)
                for (int lane = 0; lane < 32; ++lane)
                {
                    const size_t u = ((size_t) (gr * KB + kb) * 4 + s) * 32 + lane;
                    for (int t = 0; t < 4; ++t)
                    {
                        const uint32_t word = w32[u * 4 + t];
                        for (int nib = 0; nib < 8; ++nib)
                        {
                            const int c = nib >> 2, h = (nib >> 1) & 1, rh = nib & 1;
                            const int row = (gr * 4 + s) * 16 + lane / 4 + 8 * rh;
                            const int col = kb * 64 + t * 16 + h * 8 + (lane % 4) * 2 + c;
                            const uint8_t code = (uint8_t) ((word >> (4 * nib)) & 15u);
                            codes[(size_t) row * (K / 2) + col / 2] |= (uint8_t) ((col & 1) ? (code << 4) : code);
                        }
                    }
                }
    for (int n = 0; n < N; ++n)
    {
        const uint16_t b = hmoe_f2bf(row_scale[n]);
        for (int g = 0; g < KG; ++g) sc[(size_t) n * KG + g] = b;
    }
    const int rc = hmoe_pack_i4(codes, sc, N, K, q_host, s_host);
    free(codes); free(sc);
    return rc;
}

extern "C" int hmoe_gen_i4(uint64_t key_q, uint64_t key_s, float sigma_s, int N, int K, void* q, void* s, void* stream)
{
    HMOE_REQUIRE(q && s, "gen_i4: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 512 == 0, "gen_i4: shape %d x %d", N, K);
    const size_t lanes = (size_t) (N / 16) * (K / 128) * 64;
    gen_i4_kernel<<<grid_for(lanes, 256), 256, 0, (hipStream_t) stream>>>(key_q, key_s, sigma_s, N, K, (u32x4*) q,
                                                                           (uint16_t*) s);
    return HMOE_LAUNCHED("gen_i4");
}

extern "C" int hmoe_gen_dense(uint64_t key, float sigma, int N, int K, void* out, void* stream)
{
    HMOE_REQUIRE(out, "gen_dense: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0, "gen_dense: shape %d x %d", N, K);
    const size_t lanes = (size_t) (N / 16) * (K / 32) * 64;
    gen_dense_kernel<<<grid_for(lanes, 256), 256, 0, (hipStream_t) stream>>>(key, sigma, N, K, (f16x8*) out);
    return HMOE_LAUNCHED("gen_dense");
}

extern "C" int hmoe_gen_normal(uint64_t key, int64_t n, float mean, float sigma, int dtype, void* out, void* stream)
{
    HMOE_REQUIRE(out && n >= 0 && (dtype == 0 || dtype == 1), "gen_normal: arguments");
    if (n == 0) return HMOE_OK;
    gen_normal_kernel<<<grid_for((size_t) n, 256), 256, 0, (hipStream_t) stream>>>(key, n, mean, sigma, dtype, out);
    return HMOE_LAUNCHED("gen_normal");
}

extern "C" int hmoe_moe4_dequant(const void* q, const void* s, int N, int K, uint16_t* out, void* stream)
{
    HMOE_REQUIRE(q && s && out, "moe4_dequant: null buffer");
    HMOE_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 512 == 0, "moe4_dequant: shape %d x %d", N, K);
    const size_t lanes = (size_t) (N / 16) * (K / 128) * 64;
    dequant_kernel<<<grid_for(lanes, 256), 256, 0, (hipStream_t) stream>>>((const u32x4*) q, (const uint16_t*) s, N, K,
                                                                           (_Float16*) out);
    return HMOE_LAUNCHED("moe4_dequant");
}

extern "C" int hmoe_moe4_combine(float* f, const float* o, float* y, int rows, const float* o2, const unsigned* done,
                                 void* stream)
{
    HMOE_REQUIRE(f && y && rows >= 0, "moe4_combine: arguments");
    HMOE_REQUIRE(!done, "moe4_combine: the cross-device DONE flag is not supported");
    HMOE_REQUIRE(((uintptr_t) f & 15) == 0 && ((uintptr_t) y & 15) == 0, "moe4_combine: alignment");
    const int n = rows * H;
    if (n == 0) return HMOE_OK;
    combine_kernel<<<(n / 4 + 255) / 256, 256, 0, (hipStream_t) stream>>>(f, o, y, n, o2);
    return HMOE_LAUNCHED("moe4_combine");
}

extern "C" int hmoe_finish_bf16(float* y, int rows, uint16_t* out, void* stream)
{
    HMOE_REQUIRE(y && out && rows >= 0, "finish_bf16: arguments");
    const int n = rows * H;
    if (n == 0) return HMOE_OK;
    finish_kernel<<<(n / 4 + 255) / 256, 256, 0, (hipStream_t) stream>>>(y, n, out);
    return HMOE_LAUNCHED("finish_bf16");
}

