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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace hmoe {

constexpr int H = HMOE_H, I = HMOE_I, TOPK = HMOE_TOPK, MAXR = HMOE_MAXR, MAXSLOT = HMOE_MAXSLOT;
constexpr int SH_SLOT = MAXSLOT;            // act slot of the shared expert
constexpr int ACT_SLOTS = MAXSLOT + 1 + 3;  // + the f16 copy of x ([16][H] = 3 slots of [16][I]) after the shared slot

// ---- error state of the C ABI (common.hip) ----
int set_error(int code, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
#define HMOE_REQUIRE(cond, ...) do { if (!(cond)) return ::hmoe::set_error(HMOE_ERR_ARG, __VA_ARGS__); } while (0)
#define HMOE_LAUNCHED(what) ::hmoe::hip_check(hipGetLastError(), what)

// ---- conversions ----
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t) b << 16); }

// 8 codes of one I4G128 dword -> 8 exact f16 values q = code - 8, element e of the MFMA operand at nibble bit
// 4(e/2) + 16(e%2): (code | 0x6400) is the f16 1024 + code (0x6400 = 1024, one unit per mantissa step), minus 1032;
// the odd nibble of each byte lands 4 bits up, 1024 + 16 code, scaled by 1/16 and offset by -72 (all exact).
__device__ __forceinline__ f16x8 dq8(uint32_t w)
{
    const uint32_t top = w >> 8;
    const uint32_t h0 = (w & 0x000f000fu) | 0x64006400u;
    const uint32_t h1 = (w & 0x00f000f0u) | 0x64006400u;
    const uint32_t h2 = (top & 0x000f000fu) | 0x64006400u;
    const uint32_t h3 = (top & 0x00f000f0u) | 0x64006400u;
    const f16x2 m1032 = {(_Float16) -1032.0f, (_Float16) -1032.0f};
    const f16x2 s16 = {(_Float16) 0.0625f, (_Float16) 0.0625f};
    const f16x2 m72 = {(_Float16) -72.0f, (_Float16) -72.0f};
    const f16x2 a0 = __builtin_bit_cast(f16x2, h0) + m1032;
    const f16x2 a1 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, h1), s16, m72);
    const f16x2 a2 = __builtin_bit_cast(f16x2, h2) + m1032;
    const f16x2 a3 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, h3), s16, m72);
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

// global loads of weights that are read once (nontemporal: do not keep them in the caches)
__device__ __forceinline__ u32x4 ldw16(const void* p) { return __builtin_nontemporal_load((const u32x4*) p); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*) p; }

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

}  // namespace hmoe
