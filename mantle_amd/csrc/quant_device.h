// quant_device.h -- device helpers shared by the gfx950 kernels: Mantle's
// lane-ordered reductions (sum of squares, dot, ordered sums) and the int8
// activation quantiser of its W4A8 CPU path.
#pragma once

#include <hip/hip_fp16.h>
#include <stdint.h>

#include "device_common.h"
#include "kernels.h"

namespace mantle {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

static constexpr int kThreads = 256;
static constexpr int kMaxPairs = 8;  // 32-weight blocks per lane per pass

// Byte position of element e (0..31) of a block in the even/odd permuted
// activation layout that k4_block_dot consumes.
__device__ __forceinline__ int qx_perm(int e) { return ((e & 1) << 4) | ((e >> 3) << 2) | ((e >> 1) & 3); }

// ---------------------------------------------------------------------------
// Parity reductions (Mantle's archsimd lane orders)

// Sum of squares exactly as rmsNormAVX512 / rmsNormSIMD / rmsNormScalar do it
// (internal/backend/simd/ops_avx512.go:92-112, ops_avx2.go:54-77, ops.go:70-76):
// lane l accumulates fma(x, x, acc) over i = l, l+L, ... (L = 16 / 8), then the L
// partial sums are added left to right and the scalar tail follows.  Each lane
// loads 8 operands ahead of its dependent FMA chain.  Whole workgroup; red >= 17 floats.
__device__ inline float wg_sumsq_parity(const float* src, int n, int isa, float* red) {
    const int lanes = isa == kIsaAvx512 ? 16 : (isa == kIsaAvx2 ? 8 : 0);
    const int nfull = lanes ? (n / lanes) * lanes : 0;
    const int tid = threadIdx.x;
    if (lanes && tid < lanes) {
        float acc = 0.0f;
        int i = tid;
        for (; i + 7 * lanes < nfull; i += 8 * lanes) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = src[i + k * lanes];
#pragma unroll
            for (int k = 0; k < 8; k++) acc = __builtin_fmaf(v[k], v[k], acc);
        }
        for (; i < nfull; i += lanes) acc = __builtin_fmaf(src[i], src[i], acc);
        red[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        if (lanes) {
            sum = red[0];
            for (int l = 1; l < lanes; l++) sum += red[l];
        }
        int i = nfull;
        for (; i + 8 <= n; i += 8) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = src[i + k];
#pragma unroll
            for (int k = 0; k < 8; k++) sum += v[k] * v[k];
        }
        for (; i < n; i++) sum += src[i] * src[i];
        red[16] = sum;
    }
    __syncthreads();
    float r = red[16];
    __syncthreads();
    return r;
}

// sum = ((t[0] + t[s]) + t[2s]) + ... in order, loads issued 8 ahead of the adds.
__device__ __forceinline__ float ordered_sum(const float* t, int stride, int n) {
    float sum = 0.0f;
    int b = 0;
    for (; b + 16 <= n; b += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = t[(b + k) * stride];
#pragma unroll
        for (int k = 0; k < 16; k++) sum += v[k];
    }
    for (; b < n; b++) sum += t[b * stride];
    return sum;
}

// ordered_sum over contiguous (16-byte aligned) values in batches of 64 (then
// 16), continuing the running sum `sum`: one LDS / memory latency per 64
// dependent adds instead of per 16.
__device__ __forceinline__ float ordered_sum_contig(const float* t, int n, float sum = 0.0f) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    int b = 0;
    for (; b + 64 <= n; b += 64) {
        f4 v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = *reinterpret_cast<const f4*>(t + b + 4 * k);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            sum += v[k].x;
            sum += v[k].y;
            sum += v[k].z;
            sum += v[k].w;
        }
    }
    for (; b + 16 <= n; b += 16) {
        f4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = *reinterpret_cast<const f4*>(t + b + 4 * k);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            sum += v[k].x;
            sum += v[k].y;
            sum += v[k].z;
            sum += v[k].w;
        }
    }
    for (; b < n; b++) sum += t[b];
    return sum;
}

// Dot exactly as dotAVX512 / dotSIMD / dotScalar (internal/backend/simd/ops_avx512.go:27-90,
// ops_avx2.go:25-51, ops.go:49-55).  One thread computes the whole dot.
// Compile-time length: every accumulator stays in a register.
template <int N, int ISA>
__device__ __forceinline__ float dot_parity_t(const float* a, const float* b) {
    if constexpr (ISA == kIsaAvx512) {
        float acc[64];
#pragma unroll
        for (int k = 0; k < 64; k++) acc[k] = 0.0f;
        constexpr int n64 = (N / 64) * 64;
        constexpr int n32 = n64 + ((N - n64) / 32) * 32;
        constexpr int n16 = n32 + ((N - n32) / 16) * 16;
#pragma unroll
        for (int i = 0; i < n64; i += 64)
#pragma unroll
            for (int k = 0; k < 64; k++) acc[k] = __builtin_fmaf(a[i + k], b[i + k], acc[k]);
#pragma unroll
        for (int i = n64; i < n32; i += 32)
#pragma unroll
            for (int k = 0; k < 32; k++) acc[k] = __builtin_fmaf(a[i + k], b[i + k], acc[k]);
#pragma unroll
        for (int i = n32; i < n16; i += 16)
#pragma unroll
            for (int k = 0; k < 16; k++) acc[k] = __builtin_fmaf(a[i + k], b[i + k], acc[k]);
        float sum = acc[0];
#pragma unroll
        for (int k = 1; k < 64; k++) sum += acc[k];
#pragma unroll
        for (int i = n16; i < N; i++) sum += a[i] * b[i];
        return sum;
    } else if constexpr (ISA == kIsaAvx2) {
        float a0[8], a1[8];
#pragma unroll
        for (int l = 0; l < 8; l++) { a0[l] = 0.0f; a1[l] = 0.0f; }
        constexpr int n16 = (N / 16) * 16;
        constexpr int n8 = n16 + ((N - n16) / 8) * 8;
#pragma unroll
        for (int i = 0; i < n16; i += 16) {
#pragma unroll
            for (int l = 0; l < 8; l++) {
                a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
                a1[l] = __builtin_fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
            }
        }
#pragma unroll
        for (int i = n16; i < n8; i += 8)
#pragma unroll
            for (int l = 0; l < 8; l++) a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
#pragma unroll
        for (int l = 0; l < 8; l++) a0[l] = a0[l] + a1[l];
        float sum = a0[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum += a0[l];
#pragma unroll
        for (int i = n8; i < N; i++) sum += a[i] * b[i];
        return sum;
    } else {
        float sum = 0.0f;
#pragma unroll 16
        for (int i = 0; i < N; i++) sum += a[i] * b[i];
        return sum;
    }
}

// Runtime-length version (any n), same orders; used off the common head dims.
__device__ inline float dot_parity_n(const float* a, const float* b, int n, int isa) {
    if (isa == kIsaAvx512) {
        if (n == 0) return 0.0f;
        float acc[4][16];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 16; l++) acc[j][l] = 0.0f;
        int i = 0;
        for (; i + 64 <= n; i += 64) {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 16; l++) acc[j][l] = __builtin_fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        }
        for (; i + 32 <= n; i += 32) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int l = 0; l < 16; l++) acc[j][l] = __builtin_fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        }
        for (; i + 16 <= n; i += 16) {
#pragma unroll
            for (int l = 0; l < 16; l++) acc[0][l] = __builtin_fmaf(a[i + l], b[i + l], acc[0][l]);
        }
        float sum = acc[0][0];
#pragma unroll
        for (int k = 1; k < 64; k++) sum += acc[k / 16][k % 16];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    if (isa == kIsaAvx2) {
        if (n == 0) return 0.0f;
        float a0[8], a1[8];
#pragma unroll
        for (int l = 0; l < 8; l++) { a0[l] = 0.0f; a1[l] = 0.0f; }
        int i = 0;
        for (; i + 16 <= n; i += 16) {
#pragma unroll
            for (int l = 0; l < 8; l++) {
                a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
                a1[l] = __builtin_fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
            }
        }
        if (i + 8 <= n) {
#pragma unroll
            for (int l = 0; l < 8; l++) a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
            i += 8;
        }
#pragma unroll
        for (int l = 0; l < 8; l++) a0[l] = a0[l] + a1[l];
        float sum = a0[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum += a0[l];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

__device__ __forceinline__ float dot_parity(const float* a, const float* b, int n, int isa) {
    if (n == 128) {
        if (isa == kIsaAvx512) return dot_parity_t<128, kIsaAvx512>(a, b);
        if (isa == kIsaAvx2) return dot_parity_t<128, kIsaAvx2>(a, b);
        return dot_parity_t<128, kIsaScalar>(a, b);
    }
    if (n == 64) {
        if (isa == kIsaAvx512) return dot_parity_t<64, kIsaAvx512>(a, b);
        if (isa == kIsaAvx2) return dot_parity_t<64, kIsaAvx2>(a, b);
        return dot_parity_t<64, kIsaScalar>(a, b);
    }
    return dot_parity_n(a, b, n, isa);
}

// ---------------------------------------------------------------------------
// Activation quantiser (+ optional RMSNorm), one workgroup per row.

// Load 16 values (half h of block b) of x, and of the gains when weight != null.
__device__ __forceinline__ void load_half16(const float* __restrict__ x, const float* __restrict__ weight, int n,
                                            int base, bool vec4, float (&v)[16], float (&g)[16]) {
    if (vec4 && base + 16 <= n) {
        const float4* x4 = reinterpret_cast<const float4*>(x + base);
        const float4* w4 = reinterpret_cast<const float4*>(weight + base);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 t = x4[k];
            v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
            if (weight) {
                const float4 u = w4[k];
                g[4 * k] = u.x; g[4 * k + 1] = u.y; g[4 * k + 2] = u.z; g[4 * k + 3] = u.w;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int idx = base + k;
            v[k] = idx < n ? x[idx] : 0.0f;
            if (weight) g[k] = idx < n ? weight[idx] : 0.0f;
        }
    }
}

// Stage one activation vector as Mantle's W4A8 operand: optional RMSNorm
// (weight != null), then per-32-block int8 quantisation (quantizeVecBlocksInto,
// internal/backend/simd/matvec_quant.go:746-797).  Two adjacent lanes own one
// 32-element block (16 values each, loaded once up front); the block max is
// one lane-pair exchange (max is exact in any order).  The RMS sum of squares
// runs on 16 / 8 lanes in Mantle's lane-striped order over an LDS copy (vals,
// ceil32(n) floats, only touched with weight).  Whole workgroup; red >= 17
// floats; q_out / s_out may be LDS or global (q_out in the even/odd permuted
// layout: dword j of the first 16 bytes holds elements 8j+0,2,4,6, of the
// second 16 bytes elements 8j+1,3,5,7).
// First-trip loads of wg_quantize_vec (this lane's 16 values and gains), so a
// caller can put them in flight ahead of its own, larger loads.
__device__ __forceinline__ void wg_quantize_vec_load(const float* __restrict__ x, const float* __restrict__ weight,
                                                     int n, float (&v)[16], float (&g)[16]) {
    const int halves = ((n + 31) >> 5) * 2;
    const bool vec4 = (n & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15) == 0;
    if ((int)threadIdx.x < halves) load_half16(x, weight, n, threadIdx.x * 16, vec4, v, g);
}

// Mantle's per-block int8 quantiser arithmetic (quantizeVecBlocksInto,
// internal/backend/simd/matvec_quant.go:746-797) for a block whose max |v| is
// m: scale = m / 127 (0 for an all-zero block), q = clamp(round(v * (1 /
// scale)), +-127), round half away from zero.
__device__ __forceinline__ float quant_block_inv(float m, float* scale) {
    if (m == 0.0f) {
        *scale = 0.0f;
        return 0.0f;
    }
    const float sc = m / 127.0f;
    *scale = sc;
    return 1.0f / sc;
}
__device__ __forceinline__ int32_t quant_value(float v, float inv) {
    const int32_t q = go_round(v * inv);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// One value per lane, 32 consecutive lanes = one block (lanes 0-31 and 32-63
// of a wave are two blocks): block max through five xor exchanges, then q of
// this lane's value and the block scale.
__device__ __forceinline__ int32_t quant_lane32(float v, float* scale) {
    float m = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 32));
    const float inv = quant_block_inv(m, scale);
    return quant_value(v, inv);
}

// Quantise one 16-value half (half hh & 1 of block hh >> 1) of an activation
// row into Mantle's int8 block layout (quantizeVecBlocksInto,
// internal/backend/simd/matvec_quant.go:746-797): the block max is one
// lane-pair exchange (max is exact in any order), scale = max/127, q =
// clamp(round(v * (1/scale)), +-127).  Both lanes of the pair call it (live
// or not: the exchange needs them).  q_out is the even/odd permuted layout:
// dword j of the first 16 bytes holds elements 8j+0,2,4,6, of the second 16
// bytes elements 8j+1,3,5,7.
__device__ __forceinline__ void quantize_half16(const float (&v)[16], bool live, int hh, int8_t* q_out,
                                                float* s_out) {
    float m = 0.0f;
    if (live) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float a = v[k] < 0 ? -v[k] : v[k];
            m = a > m ? a : m;
        }
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    if (!live) return;
    uint32_t we[2] = {0, 0}, wo[2] = {0, 0};
    float sc;
    const float inv = quant_block_inv(m, &sc);
    if (m != 0.0f) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const uint32_t byte = (uint32_t)(uint8_t)(int8_t)quant_value(v[k], inv);
            // element e = 16*half + k of the block: dword (e>>3) of the even/odd half
            const int dw = (k >> 3), sh = ((k >> 1) & 3) * 8;
            if (k & 1) wo[dw] |= byte << sh; else we[dw] |= byte << sh;
        }
    }
    const int blk = hh >> 1, half = hh & 1;
    uint2* qb = reinterpret_cast<uint2*>(q_out + blk * 32);
    qb[half] = make_uint2(we[0], we[1]);      // even elements: bytes 8*half .. +7
    qb[2 + half] = make_uint2(wo[0], wo[1]);  // odd elements: bytes 16 + 8*half .. +7
    if (half == 0) s_out[blk] = sc;
}

// VPT consecutive floats (16-byte aligned for VPT >= 4, 8-byte for 2).
template <int VPT>
__device__ __forceinline__ void load_piece(const float* __restrict__ src, float (&v)[VPT]) {
    if constexpr (VPT >= 4) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
        for (int k = 0; k < VPT / 4; k++) {
            const float4 u = s4[k];
            v[4 * k] = u.x; v[4 * k + 1] = u.y; v[4 * k + 2] = u.z; v[4 * k + 3] = u.w;
        }
    } else {
        const float2 u = *reinterpret_cast<const float2*>(src);
        v[0] = u.x; v[1] = u.y;
    }
}

// quantize_half16 for a piece of VPT (2..16) consecutive values: piece pc
// holds elements VPT*pc .. VPT*pc+VPT-1 of the row, the 32/VPT pieces of a
// block sit in consecutive lanes of one wave (their max is an xor exchange
// over those lanes; max is exact in any order), and every lane of the wave
// calls it.  Same arithmetic and byte layout as quantize_half16.
template <int VPT>
__device__ __forceinline__ void quantize_piece(const float (&v)[VPT], bool live, int pc, int8_t* q_out,
                                               float* s_out) {
    static_assert(VPT == 2 || VPT == 4 || VPT == 8 || VPT == 16, "a block is 32 / VPT pieces");
    float m = 0.0f;
    if (live) {
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const float a = v[k] < 0 ? -v[k] : v[k];
            m = a > m ? a : m;
        }
    }
#pragma unroll
    for (int off = 1; off < 32 / VPT; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (!live) return;
    float sc;
    const float inv = quant_block_inv(m, &sc);
    const int e0 = (pc * VPT) & 31;  // first element of the piece within its block
    int8_t* qb = q_out + (pc * VPT - e0);
    if constexpr (VPT == 16) {
        uint32_t we[2] = {0, 0}, wo[2] = {0, 0};
        if (m != 0.0f) {
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const uint32_t byte = (uint32_t)(uint8_t)(int8_t)quant_value(v[k], inv);
                const int dw = (k >> 3), sh = ((k >> 1) & 3) * 8;
                if (k & 1) wo[dw] |= byte << sh; else we[dw] |= byte << sh;
            }
        }
        uint2* q2 = reinterpret_cast<uint2*>(qb);
        const int half = e0 >> 4;
        q2[half] = make_uint2(we[0], we[1]);
        q2[2 + half] = make_uint2(wo[0], wo[1]);
    } else {
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const int8_t q = m != 0.0f ? (int8_t)quant_value(v[k], inv) : (int8_t)0;
            qb[qx_perm(e0 + k)] = q;
        }
    }
    if (e0 == 0) s_out[(pc * VPT) >> 5] = sc;
}

// rms_stage_half for a piece of VPT consecutive values: x[VPT*pc + k] goes to
// tv[((VPT*pc + k) & 15) * pitch + ((VPT*pc + k) >> 4)].
template <int VPT>
__device__ __forceinline__ void rms_stage_piece(float* tv, int pitch, int pc, const float (&v)[VPT]) {
#pragma unroll
    for (int k = 0; k < VPT; k++) {
        const int i = VPT * pc + k;
        tv[(i & 15) * pitch + (i >> 4)] = v[k];
    }
}

// Row pitch (floats) of the transposed staging of an N-value row: value
// x[16m + l] sits at tv[l * pitch + m], so parity lane l's operands are one
// contiguous run (read as float4); the +4 spreads the 16 runs over the banks.
__host__ __device__ constexpr int rms_stage_pitch(int n) { return n / 16 + 4; }

// Store this lane's 16 consecutive values x[16h .. 16h+15] (half h) into the
// transposed staging (for a fixed k the lanes write consecutive words).
__device__ __forceinline__ void rms_stage_half(float* tv, int pitch, int h, const float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 16; k++) tv[k * pitch + h] = v[k];
}

// RMSNorm scale 1/sqrt(mean(x^2) + eps) of an N-value row in the transposed
// staging, with the sum of squares in Mantle's order (rmsNormAVX512 /
// rmsNormSIMD / rmsNormScalar, internal/backend/simd/ops_avx512.go:92-112,
// ops_avx2.go:54-77, ops.go:70-76): lane l of 16 / 8 accumulates fma(x, x, acc)
// over i = l, l+L, l+2L, ...; the L partials are then added left to right (N
// is a multiple of 16: no tail).  Wave 0 does the work; with more waves the
// scale passes through red[0].
template <int N, int NW>
__device__ __forceinline__ float wg_rms_scale_t(const float* tv, float eps, int isa, float* red) {
    static_assert(N % 64 == 0, "row length must be a multiple of 64");
    constexpr int P = rms_stage_pitch(N);
    constexpr int M4 = N / 64;  // float4 per staged row
    const int tid = threadIdx.x;
    float scale = 0.0f;
    if (tid < 64) {
        float sum = 0.0f;
        if (isa == kIsaAvx512) {
            float acc = 0.0f;
            if (tid < 16) {
                const float4* r = reinterpret_cast<const float4*>(tv + tid * P);
#pragma unroll
                for (int c = 0; c < M4; c++) {
                    const float4 a = r[c];
                    acc = __builtin_fmaf(a.x, a.x, acc);
                    acc = __builtin_fmaf(a.y, a.y, acc);
                    acc = __builtin_fmaf(a.z, a.z, acc);
                    acc = __builtin_fmaf(a.w, a.w, acc);
                }
            }
            float part[16];
#pragma unroll
            for (int l = 0; l < 16; l++) part[l] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
            sum = part[0];
#pragma unroll
            for (int l = 1; l < 16; l++) sum += part[l];
        } else if (isa == kIsaAvx2) {
            // lane l: i = l + 8m' -> staged row l (m' even) and row l + 8 (m' odd)
            float acc = 0.0f;
            if (tid < 8) {
                const float4* ra = reinterpret_cast<const float4*>(tv + tid * P);
                const float4* rb = reinterpret_cast<const float4*>(tv + (tid + 8) * P);
#pragma unroll
                for (int c = 0; c < M4; c++) {
                    const float4 a = ra[c], b = rb[c];
                    acc = __builtin_fmaf(a.x, a.x, acc);
                    acc = __builtin_fmaf(b.x, b.x, acc);
                    acc = __builtin_fmaf(a.y, a.y, acc);
                    acc = __builtin_fmaf(b.y, b.y, acc);
                    acc = __builtin_fmaf(a.z, a.z, acc);
                    acc = __builtin_fmaf(b.z, b.z, acc);
                    acc = __builtin_fmaf(a.w, a.w, acc);
                    acc = __builtin_fmaf(b.w, b.w, acc);
                }
            }
            float part[8];
#pragma unroll
            for (int l = 0; l < 8; l++) part[l] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
            sum = part[0];
#pragma unroll
            for (int l = 1; l < 8; l++) sum += part[l];
        } else {
            for (int i = 0; i < N; i++) {
                const float v = tv[(i & 15) * P + (i >> 4)];
                sum += v * v;
            }
        }
        scale = rms_scale(sum, N, eps);
    }
    if constexpr (NW > 1) {
        if (tid == 0) red[0] = scale;
        __syncthreads();
        scale = red[0];
    }
    return scale;
}

// wg_rms_scale_t for a run-time row length n (a multiple of 64, staged with
// rms_stage_pitch(n)); the same orders, the wave-0 result returned to every
// thread through red[0].
__device__ __forceinline__ float wg_rms_scale_rt(const float* tv, int n, float eps, int isa, float* red) {
    const int P = rms_stage_pitch(n);
    const int m4 = n / 64;
    const int tid = threadIdx.x;
    if (tid < 64) {
        float sum = 0.0f;
        if (isa == kIsaAvx512) {
            float acc = 0.0f;
            if (tid < 16) {
                const float4* r = reinterpret_cast<const float4*>(tv + tid * P);
                for (int c = 0; c < m4; c++) {
                    const float4 a = r[c];
                    acc = __builtin_fmaf(a.x, a.x, acc);
                    acc = __builtin_fmaf(a.y, a.y, acc);
                    acc = __builtin_fmaf(a.z, a.z, acc);
                    acc = __builtin_fmaf(a.w, a.w, acc);
                }
            }
            float part[16];
#pragma unroll
            for (int l = 0; l < 16; l++) part[l] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
            sum = part[0];
#pragma unroll
            for (int l = 1; l < 16; l++) sum += part[l];
        } else if (isa == kIsaAvx2) {
            float acc = 0.0f;
            if (tid < 8) {
                const float4* ra = reinterpret_cast<const float4*>(tv + tid * P);
                const float4* rb = reinterpret_cast<const float4*>(tv + (tid + 8) * P);
                for (int c = 0; c < m4; c++) {
                    const float4 a = ra[c], b = rb[c];
                    acc = __builtin_fmaf(a.x, a.x, acc);
                    acc = __builtin_fmaf(b.x, b.x, acc);
                    acc = __builtin_fmaf(a.y, a.y, acc);
                    acc = __builtin_fmaf(b.y, b.y, acc);
                    acc = __builtin_fmaf(a.z, a.z, acc);
                    acc = __builtin_fmaf(b.z, b.z, acc);
                    acc = __builtin_fmaf(a.w, a.w, acc);
                    acc = __builtin_fmaf(b.w, b.w, acc);
                }
            }
            float part[8];
#pragma unroll
            for (int l = 0; l < 8; l++) part[l] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
            sum = part[0];
#pragma unroll
            for (int l = 1; l < 8; l++) sum += part[l];
        } else {
            for (int i = 0; i < n; i++) {
                const float v = tv[(i & 15) * P + (i >> 4)];
                sum += v * v;
            }
        }
        if (tid == 0) red[0] = rms_scale(sum, n, eps);
    }
    __syncthreads();
    return red[0];
}

template <int NT = kThreads>
__device__ void wg_quantize_vec_pre(const float* __restrict__ x, const float* __restrict__ weight, float eps, int n,
                                    int isa, float* vals, float* red, int8_t* q_out, float* s_out, float* norm_out,
                                    float (&v)[16], float (&g)[16]) {
    const int tid = threadIdx.x;
    const int halves = ((n + 31) >> 5) * 2;
    const bool vec4 = (n & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15) == 0;
    float scale = 1.0f;
    if (weight) {
        if (halves <= NT) {
            if (tid < halves) {
                float4* d4 = reinterpret_cast<float4*>(vals + tid * 16);
#pragma unroll
                for (int k = 0; k < 4; k++) d4[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
            }
        } else {
            for (int i = tid; i < halves * 16; i += NT) vals[i] = i < n ? x[i] : 0.0f;
        }
        __syncthreads();
        const int lanes = isa == kIsaAvx512 ? 16 : (isa == kIsaAvx2 ? 8 : 0);
        const int nfull = lanes ? (n / lanes) * lanes : 0;
        if (lanes && tid < lanes) {
            float acc = 0.0f;
            int i = tid;
            for (; i + 15 * lanes < nfull; i += 16 * lanes) {
                float t[16];
#pragma unroll
                for (int k = 0; k < 16; k++) t[k] = vals[i + k * lanes];
#pragma unroll
                for (int k = 0; k < 16; k++) acc = __builtin_fmaf(t[k], t[k], acc);
            }
            for (; i < nfull; i += lanes) acc = __builtin_fmaf(vals[i], vals[i], acc);
            red[tid] = acc;
        }
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            if (lanes) {
                sum = red[0];
                for (int l = 1; l < lanes; l++) sum += red[l];
            }
            for (int i = nfull; i < n; i++) sum += vals[i] * vals[i];
            red[16] = rms_scale(sum, n, eps);
        }
        __syncthreads();
        scale = red[16];
    }
    // halves is even and NT a multiple of 2: both lanes of a pair take the same trips.
    for (int hh = tid; hh < ((halves + NT - 1) / NT) * NT; hh += NT) {
        const bool live = hh < halves;
        const int base = hh * 16;
        if (hh != tid && live) load_half16(x, weight, n, base, vec4, v, g);
        if (live && weight) {
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = (v[k] * scale) * g[k];
        }
        if (live && norm_out)
            for (int k = 0; k < 16 && base + k < n; k++) norm_out[base + k] = v[k];
        quantize_half16(v, live, hh, q_out, s_out);
    }
    __syncthreads();
}

template <int NT = kThreads>
__device__ void wg_quantize_vec(const float* __restrict__ x, const float* __restrict__ weight, float eps, int n,
                                int isa, float* vals, float* red, int8_t* q_out, float* s_out, float* norm_out) {
    float v[16], g[16];
    wg_quantize_vec_load(x, weight, n, v, g);
    wg_quantize_vec_pre<NT>(x, weight, eps, n, isa, vals, red, q_out, s_out, norm_out, v, g);
}

}  // namespace mantle
