// device_common.h -- CDNA4 (gfx950) device helpers shared by the k4 decode kernels.
//
// All translation units of libmantle_hip.so are compiled with
// -ffp-contract=off: a*b+c is never fused unless __builtin_fmaf is written.
// That is what makes the "CPU-parity" kernels reproduce Mantle's CPU path
// bit for bit (Go at GOAMD64=v1 never fuses; archsimd MulAdd always does).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mantle {

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Mantle's fp16 -> fp32 (internal/backend/core/float16.go:42-64): subnormal
// inputs flush to zero, inf/NaN keep their payload.
__device__ __forceinline__ float mantle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) return u2f(sign);
    if (exp == 0x1F) return u2f(sign | 0x7F800000u | (mant << 13));
    return u2f(sign | ((exp + 112u) << 23) | (mant << 13));
}

// Mantle's fp32 -> fp16 for the f16 KV cache (internal/backend/simd/float16.go:7-46,
// via StoreKV's Float32ToFloat16Slice): the mantissa is truncated, values too
// small for a normal fp16 become signed zero, too large ones infinity, NaN a
// quiet NaN with payload 0x200.
__device__ __forceinline__ uint16_t mantle_f32_to_f16_trunc(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xFFu);
    const uint32_t m = b & 0x7FFFFFu;
    if (e == 0) return (uint16_t)sign;
    if (e == 0xFF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    const int ne = e - 112;  // e - 127 + 15
    if (ne >= 31) return (uint16_t)(sign | 0x7C00u);
    if (ne <= 0) return (uint16_t)sign;
    return (uint16_t)(sign | ((uint32_t)ne << 10) | (m >> 13));
}

// mantle_f16_to_f32 for f16 KV-cache values, on the hardware conversion
// (v_cvt_f32_f16 is exact for normals, zero and infinity; Mantle flushes
// subnormals to a signed zero).  NaNs come back quiet: the same bits as Mantle's
// for every NaN mantle_f32_to_f16_trunc writes (payload 0x200).
__device__ __forceinline__ float f16_cache_value(uint16_t h) {
    const float f = __half2float(__ushort_as_half(h));
    return fabsf(f) < 6.103515625e-05f ? __uint_as_float(__float_as_uint(f) & 0x80000000u) : f;
}

// The value an f16 cache slot holds for x (store, then Mantle's load).
__device__ __forceinline__ float f16_cache_round(float x) { return mantle_f16_to_f32(mantle_f32_to_f16_trunc(x)); }

// k4 block scale (internal/backend/core/quant_cache.go:77-100):
// super * (float(u6)/32), zero when either factor is zero.
__device__ __forceinline__ float k4_scale(uint16_t super_bits, uint8_t sub) {
    float sup = mantle_f16_to_f32(super_bits);
    uint32_t u6 = sub & 0x3Fu;
    if (sup == 0.0f || u6 == 0) return 0.0f;
    return sup * ((float)u6 * 0.03125f);  // u6/32 is exact
}

// Exact int dot of one 32-element k4 block with 32 int8 activations.
// w: the block's 16 bytes (nibble i = byte i/2, low nibble first).
// xe/xo: the activations re-ordered so dword j of xe holds x[8j+0,2,4,6] and
// dword j of xo holds x[8j+1,3,5,7] -- the lanes the nibble masks produce.
// (w << 4) & 0xF0F0F0F0 turns every even nibble into the signed byte 16*q,
// w & 0xF0F0F0F0 does the same for the odd ones, so v_dot4_i32_i8 yields
// 16*dot exactly; the final >>4 is exact because the sum is a multiple of 16.
__device__ __forceinline__ int k4_block_dot(uint4 w, uint4 xe, uint4 xo) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4((int)((w.x << 4) & 0xF0F0F0F0u), (int)xe.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.x & 0xF0F0F0F0u), (int)xo.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.y << 4) & 0xF0F0F0F0u), (int)xe.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.y & 0xF0F0F0F0u), (int)xo.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.z << 4) & 0xF0F0F0F0u), (int)xe.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.z & 0xF0F0F0F0u), (int)xo.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)((w.w << 4) & 0xF0F0F0F0u), (int)xe.w, acc, false);
    acc = __builtin_amdgcn_sdot4((int)(w.w & 0xF0F0F0F0u), (int)xo.w, acc, false);
    return acc >> 4;
}

// Signed value of nibble `nib` (two's complement, internal/backend/core/quant_cache.go:26-29).
__device__ __forceinline__ int k4_nib(uint32_t word, int i) {
    return ((int)(word << (28 - 4 * i))) >> 28;
}

// Scalar fastExp (internal/backend/simd/ops.go:108-150), the Softmax exponent.
__device__ __forceinline__ float fast_exp_scalar(float x) {
    if (x > 88.0f) return 3.4028235e38f;
    if (x < -88.0f) return 0.0f;
    const float ln2 = 0.693147180559945309417f;
    const float ln2inv = 1.44269504088896340736f;
    int32_t k = (int32_t)(x * ln2inv + 0.5f);
    if (x < 0) k = (int32_t)(x * ln2inv - 0.5f);
    float r = x - (float)k * ln2;
    float r2 = r * r;
    float r3 = r2 * r;
    float r4 = r2 * r2;
    float poly = 1.0f + r + r2 * 0.5f + r3 * 0.16666667f + r4 * 0.041666667f + (r4 * r) * 0.008333333f;
    return poly * u2f((uint32_t)(k + 127) << 23);
}

// fastExpVec lane (internal/backend/simd/ops_avx2.go:98-128), used by SiLU.
__device__ __forceinline__ float fast_exp_vec(float x) {
    const float ln2 = 0.693147180559945309417f;
    const float ln2inv = 1.44269504088896340736f;
    x = fmaxf(x, -88.0f);
    x = fminf(x, 88.0f);
    int32_t k = (int32_t)__builtin_rintf(x * ln2inv);  // round to nearest even
    float kf = (float)k;
    float r = x - kf * ln2;
    float r2 = r * r;
    float r3 = r2 * r;
    float r4 = r2 * r2;
    float r5 = r4 * r;
    float poly = 1.0f + r;
    poly = poly + r2 * 0.5f;
    poly = poly + r3 * 0.16666667f;
    poly = poly + r4 * 0.041666667f;
    poly = poly + r5 * 0.008333333f;
    return poly * u2f((uint32_t)(k + 127) << 23);
}

// fastSiluVec lane (internal/backend/simd/ops_avx2.go:131-141).
__device__ __forceinline__ float fast_silu_vec(float x) {
    float e = fast_exp_vec(0.0f - x);
    return x * (1.0f / (1.0f + e));
}

// Go-style round half away from zero on an fp32 value (math.Round on float64(v)).
__device__ __forceinline__ int32_t go_round(float v) { return (int32_t)roundf(v); }

// Mantle's RMS scale: 1 / float32(sqrt(float64(mean + eps))), correctly rounded sqrt.
__device__ __forceinline__ float rms_scale(float sum, int n, float eps) {
    float mean = sum / (float)n;
    return 1.0f / (float)__dsqrt_rn((double)(mean + eps));
}

}  // namespace mantle
