// attention.hip -- batch-1 decode attention for Mantle's k4 decode path
// (internal/backend/simd/attn.go:255-419, attnpool.go:77-153), bit-exact to
// the CPU order: per-head q/k RMSNorm, RoPE, KV append, scores in Mantle's
// dot order, softmax with its ordered sum, and the V sum in key order.
//
// Two kernels, one workgroup per query head:
//  * attention_decode_v4 (head_dim 64 or 128): the q, k and v
//    vectors are prepared by one wave each with no block barrier; K is staged
//    in LDS chunk by chunk (pitch head_dim + 4: float4 traffic, no bank
//    conflicts) and the scores are one key per lane of wave 0; waves 2-3
//    stream V from HBM into a register ring from the start and do the V sum.
//  * attention_decode_kernel: any head_dim <= 256 (the general fallback).
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <atomic>
#include <type_traits>
#include <mutex>

#include "device_common.h"
#include "kernels.h"
#include "phase_trace.h"
#include "quant_device.h"

#if !MANTLE_F16_INPUT_FTZ
#error "attention.hip needs f16 denormal flushing: -fdenormal-fp-math=preserve-sign -Xclang -fdenormal-fp-math-f32=ieee"
#endif

namespace mantle {

// An f16 KV cache element as Mantle reads it (Float16ToFloat32,
// internal/backend/core/float16.go:42-64: subnormals flush to signed zero).
// This file is compiled with f16 denormals flushed, so the hardware
// conversion alone does it (one instruction per element on the V-sum chain
// wave, against three for an explicit compare and select).
__device__ __forceinline__ float f16_cache_load(uint16_t h) { return __half2float(__ushort_as_half(h)); }

static constexpr int kAttnKeys = 64;          // keys staged in LDS per chunk (head_dim <= 128)
static constexpr int kAttnLdsScores = 4096;    // contexts up to this keep scores in LDS
static constexpr int kAttnHdr = 832;           // q, k, v (256 each) + 64 reduction floats

// Up to 8 float4 of one chunk of cache rows (keys t0 .. t0+nk-1 of one kv head)
// per lane, held in registers so the loads of the next chunk are in flight
// while this one is used.  Row `skip` (the fused step's own row) is not loaded.
typedef float f32x4 __attribute__((ext_vector_type(4)));  // a native vector: no struct copies through scratch

struct ChunkRegs {
    f32x4 r[8];
    int off[8];  // LDS offset (row * pitch + col), -1: nothing to store
};

// Cache row of window key t (RunAttnHeads, attnpool.go:88-99): keys are
// numbered from the window start `base`; a ring of `ring` rows (0: none) puts
// key position p at row p % ring.
struct KeyMap {
    int base = 0, ring = 0;
};
__device__ __forceinline__ int krow(const KeyMap& km, int t) {
    const int p = km.base + t;
    return km.ring ? p % km.ring : p;
}

__device__ __forceinline__ void chunk_issue(ChunkRegs& c, const float* __restrict__ base, int stride, int t0, int nk,
                                            int hd, int kp, int skip) {
    // Loads are unconditional (lanes past the chunk re-read row t0, column 0) so
    // that no branch sits between them and their first use: the wait counts
    // then only wait for the data actually needed.
    const int hd4 = hd >> 2;
    const int total4 = nk * hd4;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = j * kThreads + threadIdx.x;
        const bool live = e < total4;
        const int ee = live ? e : 0;
        const int tl = ee / hd4;
        const int i4 = ee - tl * hd4;
        const int t = t0 + tl;
        const int o = tl * kp + 4 * i4;
        c.r[j] = *reinterpret_cast<const f32x4*>(base + (size_t)t * stride + 4 * i4);
        c.off[j] = (!live || t == skip) ? -1 : o;
    }
}

// chunk_issue with the head size known at compile time (no integer division).
template <int HD>
__device__ __forceinline__ void chunk_issue_t(ChunkRegs& c, const float* __restrict__ base, int stride, int t0, int nk,
                                              int hd, int kp, int skip, KeyMap km = KeyMap()) {
    constexpr int hd4 = HD / 4;
    const int total4 = nk * hd4;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = j * kThreads + threadIdx.x;
        const bool live = e < total4;
        const int ee = live ? e : 0;
        const int tl = ee / hd4;
        const int i4 = ee - tl * hd4;
        const int t = t0 + tl;
        const int o = tl * kp + 4 * i4;
        c.r[j] = *reinterpret_cast<const f32x4*>(base + (size_t)krow(km, t) * stride + 4 * i4);
        c.off[j] = (!live || t == skip) ? -1 : o;
    }
}

__device__ __forceinline__ void chunk_store(const ChunkRegs& c, float* dst, int kp, const float* cur, int t0, int nk,
                                            int skip, int hd) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int o = c.off[j];
        if (o < 0) continue;
        dst[o] = c.r[j].x;
        dst[o + 1] = c.r[j].y;
        dst[o + 2] = c.r[j].z;
        dst[o + 3] = c.r[j].w;
    }
    // the fused step's own row comes from `cur` (written by another workgroup
    // this same launch, so not read back from the cache)
    if (skip >= t0 && skip < t0 + nk && (int)threadIdx.x < hd) dst[(skip - t0) * kp + threadIdx.x] = cur[threadIdx.x];
}

// Decode attention for one query head, any head_dim <= 256 (internal/backend/simd/attn.go:255-419,
// attnpool.go:77-153), bit-exact to the CPU order.  Every global load the head
// needs first -- q, k, v, the RoPE row, the first K and V chunks -- is issued
// at the start; later chunks are loaded one chunk ahead of their use.
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    float* sq = lds;
    float* sk = lds + 256;
    float* sv = lds + 512;
    float* red = lds + 768;
    const int hd = a.head_dim;
    const int kp = hd + 1;  // odd pitch: lane t reads key row t without bank conflicts
    const int kc = hd <= 128 ? kAttnKeys : (kThreads * 32) / hd;  // keys per chunk: <= 8 float4 per lane
    float* kt = lds + kAttnHdr;
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int kvh = h * a.kv_heads / a.n_head;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    float* scores = a.max_ctx <= kAttnLdsScores ? kt + kc * kp : a.scores + (size_t)h * a.max_ctx;
    const float* kbase = a.cache_k + (size_t)kvh * a.head_stride;
    const float* vbase = a.cache_v + (size_t)kvh * a.head_stride;
    const int skip = a.fused ? pos : -1;
    PHASE_SLOT();
    PHASE(0);

    // ---- all first-needed loads in flight together
    // (indices clamped instead of branched around, see chunk_issue)
    const int half = hd / 2;
    const int ti = tid < hd ? tid : 0;
    const int th = tid < half ? tid : 0;
    const float qv = a.q[h * hd + ti];
    const float* kin = a.fused ? a.k : a.q;
    const float* vin = a.fused ? a.v : a.q;
    const float kv = kin[(a.fused ? kvh * hd : 0) + ti];
    const float vv = vin[(a.fused ? kvh * hd : 0) + ti];
    const float* cbase = a.rope_cos ? a.rope_cos + (size_t)pos * half : a.q;
    const float* sbase = a.rope_sin ? a.rope_sin + (size_t)pos * half : a.q;
    const float cs = cbase[th];
    const float sn = sbase[th];
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the chunk loads
    ChunkRegs ck, cv;
    const int nk0 = min(kc, pos + 1);
    chunk_issue(ck, kbase, a.kv_stride, 0, nk0, hd, kp, skip);
    chunk_issue(cv, vbase, a.kv_stride, 0, nk0, hd, kp, skip);
    if (tid < hd) {
        sq[tid] = qv;
        sk[tid] = kv;
        sv[tid] = vv;
    }
    __syncthreads();
    PHASE(1);
    if (a.fused) {
        // attn.go:265-286 per-head RMSNorm: q's lane-striped sum on lanes 0..L-1,
        // k's on lanes 64..64+L-1 (another wave), both at once.
        const int lanes = a.isa == kIsaAvx512 ? 16 : (a.isa == kIsaAvx2 ? 8 : 0);
        const int nfull = lanes ? (hd / lanes) * lanes : 0;
        const bool qlane = lanes && tid < lanes;
        const bool klane = lanes && tid >= 64 && tid < 64 + lanes;
        if (qlane || klane) {
            const float* src = qlane ? sq : sk;
            const int l = qlane ? tid : tid - 64;
            float acc = 0.0f;
            for (int i = l; i < nfull; i += lanes) acc = __builtin_fmaf(src[i], src[i], acc);
            red[(qlane ? 0 : 32) + l] = acc;
        }
        __syncthreads();
        if (tid == 0 || tid == 64) {
            const float* src = tid == 0 ? sq : sk;
            const float* pr = red + (tid == 0 ? 0 : 32);
            float sum = 0.0f;
            if (lanes) {
                sum = pr[0];
                for (int l = 1; l < lanes; l++) sum += pr[l];
            }
            for (int i = nfull; i < hd; i++) sum += src[i] * src[i];
            red[tid == 0 ? 16 : 48] = rms_scale(sum, hd, a.eps);
        }
        __syncthreads();
        if (tid < hd) {
            float q1 = sq[tid], k1 = sk[tid];
            if (a.q_norm) q1 = (q1 * red[16]) * a.q_norm[tid];
            if (a.k_norm) k1 = (k1 * red[48]) * a.k_norm[tid];
            sq[tid] = q1;
            sk[tid] = k1;
        }
        __syncthreads();
        if (a.rope_cos && tid < half) {  // ops_avx512.go:162-190: y0 = x0*c - x1*s, y1 = fma(x0, s, x1*c)
            float x0 = sq[tid], x1 = sq[tid + half];
            sq[tid] = x0 * cs - x1 * sn;
            sq[tid + half] = __builtin_fmaf(x0, sn, x1 * cs);
            x0 = sk[tid];
            x1 = sk[tid + half];
            sk[tid] = x0 * cs - x1 * sn;
            sk[tid + half] = __builtin_fmaf(x0, sn, x1 * cs);
        }
        __syncthreads();
        // ops_runtime.go:112-131 StoreKV: the first q-head of each kv group writes.
        const int first = (kvh * a.n_head + a.kv_heads - 1) / a.kv_heads;
        if (h == first && tid < hd) {
            a.cache_k[(size_t)kvh * a.head_stride + (size_t)pos * a.kv_stride + tid] = sk[tid];
            a.cache_v[(size_t)kvh * a.head_stride + (size_t)pos * a.kv_stride + tid] = sv[tid];
        }
    }
    PHASE(2);

    // ---- scores_t = Dot(q, k_t) * scale, one lane per key of the staged chunk
    float lmax = -INFINITY;
    for (int t0 = 0; t0 <= pos; t0 += kc) {
        const int nk = min(kc, pos + 1 - t0);
        chunk_store(ck, kt, kp, sk, t0, nk, skip, hd);
        __syncthreads();
        if (t0 + kc <= pos) chunk_issue(ck, kbase, a.kv_stride, t0 + kc, min(kc, pos + 1 - t0 - kc), hd, kp, skip);
        if (tid < nk) {
            const float sc = dot_parity(sq, kt + tid * kp, hd, a.isa) * a.scale;
            scores[t0 + tid] = sc;
            lmax = fmaxf(lmax, sc);
        }
        __syncthreads();
    }
    PHASE(3);
    for (int off = 32; off > 0; off >>= 1) lmax = fmaxf(lmax, __shfl_down(lmax, off, 64));
    if ((tid & 63) == 0) red[20 + (tid >> 6)] = lmax;
    __syncthreads();
    float maxv = red[20];
    for (int i = 1; i < kThreads / 64; i++) maxv = fmaxf(maxv, red[20 + i]);
    // Softmax (ops.go:83-106): exponentials, ordered sum, x *= 1/sum
    for (int t = tid; t <= pos; t += kThreads) scores[t] = fast_exp_scalar(scores[t] - maxv);
    __syncthreads();
    if (tid == 0) red[24] = ordered_sum(scores, 1, pos + 1);
    __syncthreads();
    const float sum = red[24];
    if (sum != 0.0f) {
        const float inv = 1.0f / sum;
        for (int t = tid; t <= pos; t += kThreads) scores[t] = scores[t] * inv;
    }
    __syncthreads();
    PHASE(4);
    // ---- out_d = sum_t p_t * v_t,d in t order (no FMA)
    float acc = 0.0f;
    for (int t0 = 0; t0 <= pos; t0 += kc) {
        const int nk = min(kc, pos + 1 - t0);
        chunk_store(cv, kt, kp, sv, t0, nk, skip, hd);
        __syncthreads();
        if (t0 + kc <= pos) chunk_issue(cv, vbase, a.kv_stride, t0 + kc, min(kc, pos + 1 - t0 - kc), hd, kp, skip);
        if (tid < hd) {
            const float* ps = scores + t0;
            int tl = 0;
            for (; tl + 8 <= nk; tl += 8) {
                float pv[8], vx[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    pv[k] = ps[tl + k];
                    vx[k] = kt[(tl + k) * kp + tid];
                }
#pragma unroll
                for (int k = 0; k < 8; k++) acc += pv[k] * vx[k];
            }
            for (; tl < nk; tl++) acc += ps[tl] * kt[tl * kp + tid];
        }
        __syncthreads();
    }
    if (tid < hd) a.out[h * hd + tid] = acc;
    if (a.q_out) {
        // The head's output is hd/32 whole int8 blocks of the Wo activation:
        // quantise them here rather than in every workgroup of the Wo GEMV.
        float sc;
        const int32_t qv = quant_lane32(tid < hd ? acc : 0.0f, &sc);
        if (tid < hd) {
            const int gi = h * hd + tid;
            a.q_out[(gi >> 5) * 32 + qx_perm(gi & 31)] = (int8_t)qv;
            if ((gi & 31) == 0) a.q_scale[gi >> 5] = sc;
        }
    }
    PHASE(5);
}


// ---------------------------------------------------------------------------
// Attention v4

// Dot of two LDS vectors read as float4, exactly as dotAVX512 / dotSIMD /
// dotScalar (internal/backend/simd/ops_avx512.go:27-90, ops_avx2.go:25-51,
// ops.go:49-55); N a multiple of 16, so no scalar tail.
template <int N, int ISA>
__device__ __forceinline__ float dot_parity_v4(const float4* a, const float4* b) {
    static_assert(N % 16 == 0, "length must be a multiple of 16");
    auto el = [](const float4& v, int c) { return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w)); };
    if constexpr (ISA == kIsaAvx512) {
        constexpr int n64 = (N / 64) * 64;
        constexpr int n32 = n64 + ((N - n64) / 32) * 32;
        float acc[64];
#pragma unroll
        for (int k = 0; k < 64; k++) acc[k] = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < N / 4; i4++) {
            const float4 x = a[i4], y = b[i4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int i = 4 * i4 + c;
                const int k = i < n64 ? (i & 63) : (i < n32 ? i - n64 : i - n32);
                acc[k] = __builtin_fmaf(el(x, c), el(y, c), acc[k]);
            }
        }
        float sum = acc[0];
#pragma unroll
        for (int k = 1; k < 64; k++) sum += acc[k];
        return sum;
    } else if constexpr (ISA == kIsaAvx2) {
        constexpr int n16 = (N / 16) * 16;
        float a0[8], a1[8];
#pragma unroll
        for (int l = 0; l < 8; l++) { a0[l] = 0.0f; a1[l] = 0.0f; }
#pragma unroll
        for (int i4 = 0; i4 < N / 4; i4++) {
            const float4 x = a[i4], y = b[i4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int i = 4 * i4 + c;
                const int l = i & 7;
                if (i < n16 && (i & 8)) a1[l] = __builtin_fmaf(el(x, c), el(y, c), a1[l]);
                else a0[l] = __builtin_fmaf(el(x, c), el(y, c), a0[l]);
            }
        }
#pragma unroll
        for (int l = 0; l < 8; l++) a0[l] = a0[l] + a1[l];
        float sum = a0[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum += a0[l];
        return sum;
    } else {
        float sum = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < N / 4; i4++) {
            const float4 x = a[i4], y = b[i4];
            sum += x.x * y.x;
            sum += x.y * y.y;
            sum += x.z * y.z;
            sum += x.w * y.w;
        }
        return sum;
    }
}

template <int N>
__device__ __forceinline__ float dot_v4_isa(const float4* a, const float4* b, int isa) {
    if (isa == kIsaAvx512) return dot_parity_v4<N, kIsaAvx512>(a, b);
    if (isa == kIsaAvx2) return dot_parity_v4<N, kIsaAvx2>(a, b);
    return dot_parity_v4<N, kIsaScalar>(a, b);
}

// chunk_store for a pitch that is a multiple of 4: one float4 store per value.
__device__ __forceinline__ void chunk_store_v4(const ChunkRegs& c, float* dst, int kp, const float* cur, int t0,
                                               int nk, int skip, int hd) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int o = c.off[j];
        if (o < 0) continue;
        *reinterpret_cast<f32x4*>(dst + o) = c.r[j];
    }
    if (skip >= t0 && skip < t0 + nk && (int)threadIdx.x < hd) dst[(skip - t0) * kp + threadIdx.x] = cur[threadIdx.x];
}

// The f16-cache form of ChunkRegs / chunk_issue_t / chunk_store_v4: four
// f16 keys-elements (8 bytes) per load, widened to fp32 when staged.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
struct ChunkRegs16 {
    u32x2 r[8];
    int off[8];
};

template <int HD>
__device__ __forceinline__ void chunk_issue16_t(ChunkRegs16& c, const uint16_t* __restrict__ base, int stride, int t0,
                                                int nk, int kp, int skip, KeyMap km = KeyMap()) {
    constexpr int hd4 = HD / 4;
    const int total4 = nk * hd4;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int e = j * kThreads + threadIdx.x;
        const bool live = e < total4;
        const int ee = live ? e : 0;
        const int tl = ee / hd4;
        const int i4 = ee - tl * hd4;
        const int t = t0 + tl;
        c.r[j] = *reinterpret_cast<const u32x2*>(base + (size_t)krow(km, t) * stride + 4 * i4);
        c.off[j] = (!live || t == skip) ? -1 : tl * kp + 4 * i4;
    }
}

__device__ __forceinline__ void chunk_store16(const ChunkRegs16& c, float* dst, int kp, const float* cur, int t0,
                                              int nk, int skip, int hd) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int o = c.off[j];
        if (o < 0) continue;
        f32x4 v;
        v.x = f16_cache_load((uint16_t)(c.r[j].x & 0xFFFFu));
        v.y = f16_cache_load((uint16_t)(c.r[j].x >> 16));
        v.z = f16_cache_load((uint16_t)(c.r[j].y & 0xFFFFu));
        v.w = f16_cache_load((uint16_t)(c.r[j].y >> 16));
        *reinterpret_cast<f32x4*>(dst + o) = v;
    }
    // the step's own row: `cur` already holds its f16-rounded values
    if (skip >= t0 && skip < t0 + nk && (int)threadIdx.x < hd) dst[(skip - t0) * kp + threadIdx.x] = cur[threadIdx.x];
}

// The q8_0-cache form: sixteen int8 key elements (16 bytes) per load, up to
// two loads per lane for a 64-key chunk of head_dim <= 128, widened to fp32
// (exactly) when staged.  The step's own row is already in the cache.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
struct ChunkRegs8 {
    u32x4 r[2];
    int off[2];
};

// Byte C of w, sign-extended, as fp32 in one instruction (SDWA byte select).
// Spelled out so that the compiler keeps the raw words and converts at the
// use, instead of splitting them into one register per byte ahead of it.
template <int C>
__device__ __forceinline__ float q8_byte_sdwa(uint32_t w) {
    float r;
    if constexpr (C == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (C == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (C == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

template <int HD>
__device__ __forceinline__ void chunk_issue8_t(ChunkRegs8& c, const int8_t* __restrict__ base, int stride, int t0,
                                               int nk, int kp, KeyMap km = KeyMap()) {
    constexpr int hd16 = HD / 16;
    const int total = nk * hd16;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int e = j * kThreads + threadIdx.x;
        const bool live = e < total;
        const int ee = live ? e : 0;
        const int tl = ee / hd16;
        const int i16 = ee - tl * hd16;
        c.r[j] = *reinterpret_cast<const u32x4*>(base + (size_t)krow(km, t0 + tl) * stride + 16 * i16);
        c.off[j] = live ? tl * kp + 16 * i16 : -1;
    }
}

__device__ __forceinline__ void chunk_store8(const ChunkRegs8& c, float* dst) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int o = c.off[j];
        if (o < 0) continue;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t x = c.r[j][w];
            f32x4 v;
            v.x = q8_byte_sdwa<0>(x);
            v.y = q8_byte_sdwa<1>(x);
            v.z = q8_byte_sdwa<2>(x);
            v.w = q8_byte_sdwa<3>(x);
            *reinterpret_cast<f32x4*>(dst + o + 4 * w) = v;
        }
    }
}

static constexpr int kAttnV4Hdr = 704;  // sq, sk, sv (128 each), two 128-float wave stagings, 64 reduction

// RMS scale of one head vector held two values per lane (x0 = element i,
// x1 = element i + hd/2, lanes i < hd/2), in Mantle's lane order (see
// wg_rms_scale_t).  One wave, wave-private staging `buf` (hd floats).
__device__ __forceinline__ float wave_rms_scale(float x0, float x1, int hd, float eps, int isa, float* buf) {
    const int lane = threadIdx.x & 63, half = hd >> 1;
    if (lane < half) {
        buf[lane] = x0;
        buf[lane + half] = x1;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float sum = 0.0f;
    if (isa == kIsaAvx512 || isa == kIsaAvx2) {
        const int L = isa == kIsaAvx512 ? 16 : 8;
        float acc = 0.0f;
        if (lane < L)
            for (int i = lane; i < hd; i += L) acc = __builtin_fmaf(buf[i], buf[i], acc);
        sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
        for (int l = 1; l < L; l++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
    } else {
        for (int i = 0; i < hd; i++) sum += buf[i] * buf[i];
    }
    return rms_scale(sum, hd, eps);
}

// The per-head vector prologue, one wave per vector: wave 0 q, wave 1 k,
// wave 2 v (fused steps), lane i < hd/2 holding elements i and i + hd/2 (the
// RoPE pair).  prep_load issues the loads (unconditional: wave-uniform
// sources, lanes clamped); prep_finish applies the per-head RMSNorm and RoPE,
// writes q / k / v to LDS and, when `append`, the step's K and V rows to the
// cache (ops_runtime.go:112-131 StoreKV).
struct PrepRegs {
    float x0, x1, g0, g1, cs, sn;
    bool has_norm, rope;
};

// Per-head RMSNorm (attn.go:265-286, gains g0 / g1) and RoPE
// (ops_avx512.go:162-190: y0 = x0*c - x1*s, y1 = fma(x0, s, x1*c)) of one
// vector held as RoPE pairs (x0 = element i, x1 = element i + HD/2, lanes
// i < HD/2).  `norm` must be wave-uniform; buf: HD floats of wave-private LDS.
template <int HD>
__device__ __forceinline__ void prep_pair(float& x0, float& x1, float g0, float g1, float cs, float sn, bool norm,
                                          bool rope, float eps, int isa, float* buf) {
    if (norm) {
        const float s = wave_rms_scale(x0, x1, HD, eps, isa, buf);
        x0 = (x0 * s) * g0;
        x1 = (x1 * s) * g1;
    }
    if (rope) {
        const float y0 = x0 * cs - x1 * sn;
        const float y1 = __builtin_fmaf(x0, sn, x1 * cs);
        x0 = y0;
        x1 = y1;
    }
}

template <int HD>
__device__ __forceinline__ PrepRegs prep_load(const AttnArgs& a, int h, int kvh, int pos) {
    constexpr int half = HD / 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane < half ? lane : 0;
    const float* src = a.q + h * HD;
    const float* nw = a.q_norm;
    if (a.fused && wave == 1) { src = a.k + kvh * HD; nw = a.k_norm; }
    if (a.fused && wave == 2) { src = a.v + kvh * HD; nw = nullptr; }
    PrepRegs r;
    r.has_norm = a.fused && wave < 2 && nw != nullptr;
    r.rope = a.fused && a.rope_cos != nullptr;
    const float* gsrc = r.has_norm ? nw : src;
    const float* cbase = r.rope ? a.rope_cos + (size_t)pos * half : src;
    const float* sbase = r.rope ? a.rope_sin + (size_t)pos * half : src;
    r.x0 = src[li];
    r.x1 = src[li + half];
    r.g0 = gsrc[li];
    r.g1 = gsrc[li + half];
    r.cs = cbase[li];
    r.sn = sbase[li];
    return r;
}

template <int HD>
__device__ __forceinline__ void prep_finish(const AttnArgs& a, PrepRegs r, int kvh, int pos, bool append, float* sq,
                                            float* sk, float* sv, float* wbuf) {
    constexpr int half = HD / 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave >= 3) return;
    float x0 = r.x0, x1 = r.x1;
    prep_pair<HD>(x0, x1, r.g0, r.g1, r.cs, r.sn, r.has_norm, r.rope && wave < 2, a.eps, a.isa, wbuf + wave * 128);
    const int ctype = wave == 1 ? a.k_type : a.v_type;  // this wave's cache (waves 1 and 2)
    if (wave > 0 && ctype == kKvF16) {  // the f16 cache holds (and the step reads back) the rounded row
        x0 = f16_cache_round(x0);
        x1 = f16_cache_round(x1);
    }
    if (lane < half && (wave == 0 || a.fused)) {
        float* dst = wave == 0 ? sq : (wave == 1 ? sk : sv);
        dst[lane] = x0;
        dst[lane + half] = x1;
        if (a.fused && wave > 0 && append && ctype != kKvQ8) {  // (q8_0 rows: launch_kv_append_q8)
            if (ctype == kKvF16) {
                uint16_t* c16 = reinterpret_cast<uint16_t*>(wave == 1 ? a.cache_k : a.cache_v);
                const uint16_t h0 = mantle_f32_to_f16_trunc(x0), h1 = mantle_f32_to_f16_trunc(x1);
                if (wave == 2 && a.vt_stride > 0) {
                    uint16_t* col = c16 + (size_t)(kvh * HD + lane) * a.vt_stride + pos;
                    col[0] = h0;
                    col[(size_t)half * a.vt_stride] = h1;
                } else {
                    uint16_t* row = c16 + (size_t)kvh * a.head_stride + (size_t)pos * a.kv_stride;
                    row[lane] = h0;
                    row[lane + half] = h1;
                }
            } else if (wave == 2 && a.vt_stride > 0) {  // transposed V: one column per row of the cache
                float* col = a.cache_v + (size_t)(kvh * HD + lane) * a.vt_stride + pos;
                col[0] = x0;
                col[(size_t)half * a.vt_stride] = x1;
            } else {
                float* cache = (wave == 1 ? a.cache_k : a.cache_v) + (size_t)kvh * a.head_stride + (size_t)pos * a.kv_stride;
                cache[lane] = x0;
                cache[lane + half] = x1;
            }
        }
    }
}

// The first query head of each KV group appends the step's K / V row.
__device__ __forceinline__ bool first_of_group(const AttnArgs& a, int h, int kvh) {
    return h == (kvh * a.n_head + a.kv_heads - 1) / a.kv_heads;
}

template <int HD>
__global__ __launch_bounds__(kThreads) void attention_decode_v4(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    float* sq = lds;
    float* sk = lds + 128;
    float* sv = lds + 256;
    float* wbuf = lds + 384;
    float* red = lds + 640;
    constexpr int hd = HD;
    constexpr int kp = hd + 4;  // staged key pitch (floats)
    constexpr int kc = kAttnKeys;
    float* kt = lds + kAttnV4Hdr;
    // Workgroup w runs on XCD w % 8.  Query heads that share a KV head are
    // given workgroups on the same XCD, so the second reads K and V from that
    // XCD's L2: head = group * (w % G) + w / G, G = n_head / group heads.
    const int w = blockIdx.x;
    const int grp = a.n_head / a.kv_heads;  // query heads per KV head
    const int G = a.n_head / grp;
    const int h = a.n_head % a.kv_heads == 0 ? grp * (w % G) + w / G : w;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = h * a.kv_heads / a.n_head;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    const bool lds_scores = a.max_ctx <= kAttnLdsScores;
    float* scores = lds_scores ? kt + kc * kp : a.scores + (size_t)h * a.max_ctx;
    const float* kbase = a.cache_k + (size_t)kvh * a.head_stride;
    const float* vbase = a.cache_v + (size_t)kvh * a.head_stride;
    const int skip = a.fused ? pos : -1;
    PHASE_SLOT();
    PHASE(0);

    // ---- every first-needed load in flight: this wave's vector pair (wave 0
    // q, 1 k, 2 v), its norm gains and RoPE row, then the first K chunk.
    // Loads are unconditional (wave-uniform sources, lanes clamped).
    const PrepRegs pr = prep_load<HD>(a, h, kvh, pos);
    __builtin_amdgcn_sched_barrier(0);
    // K chunks are loaded two ahead of their use (ck0: even chunks, ck1: odd)
    ChunkRegs ck0, ck1;
    chunk_issue_t<HD>(ck0, kbase, a.kv_stride, 0, min(kc, pos + 1), hd, kp, skip);
    if (kc <= pos) chunk_issue_t<HD>(ck1, kbase, a.kv_stride, kc, min(kc, pos + 1 - kc), hd, kp, skip);
    // Waves 2-3 own the V sum (lane d = tid - 128): they have nothing to do
    // until the softmax is done, so they hold a ring of NG groups of VG keys'
    // V values in registers, loaded from HBM from the start.
    constexpr int VG = 32, NG = 5;
    const bool pv_wave = wave >= 2;
    const int d = pv_wave && tid - 128 < hd ? tid - 128 : 0;
    const float* vcol = vbase + d;
    const size_t vs = (size_t)a.kv_stride;
    float vr[NG][VG];
    auto vissue = [&](float (&r)[VG], int t0) {
#pragma unroll
        for (int k = 0; k < VG; k++) {
            const int t = t0 + k <= pos ? t0 + k : pos;
            r[k] = vcol[(size_t)t * vs];
        }
    };
    if (pv_wave) {
#pragma unroll
        for (int g = 0; g < NG; g++)
            if (g * VG <= pos) vissue(vr[g], g * VG);
    }
    PHASE(1);

    prep_finish<HD>(a, pr, kvh, pos, a.fused && first_of_group(a, h, kvh), sq, sk, sv, wbuf);
    __syncthreads();
    PHASE(2);

    // ---- scores_t = Dot(q, k_t) * scale, one lane of wave 0 per key
    float lmax = -INFINITY;
    auto score_chunk = [&](ChunkRegs& ck, int t0) {
        const int nk = min(kc, pos + 1 - t0);
        chunk_store_v4(ck, kt, kp, sk, t0, nk, skip, hd);
        __syncthreads();
        if (t0 == 2 * kc) PHASE(6);  // third chunk staged
        const int tn = t0 + 2 * kc;  // the chunk two ahead reuses these registers
        if (tn <= pos) chunk_issue_t<HD>(ck, kbase, a.kv_stride, tn, min(kc, pos + 1 - tn), hd, kp, skip);
        if (tid < nk) {
            const float sc = dot_v4_isa<HD>(reinterpret_cast<const float4*>(sq),
                                            reinterpret_cast<const float4*>(kt + tid * kp), a.isa) * a.scale;
            scores[t0 + tid] = sc;
            lmax = fmaxf(lmax, sc);
        }
        if (t0 == 2 * kc) PHASE_AFTER(7, lmax);  // third chunk's dots done
        __syncthreads();
    };
    for (int t0 = 0; t0 <= pos; t0 += 2 * kc) {
        score_chunk(ck0, t0);
        if (t0 + kc <= pos) score_chunk(ck1, t0 + kc);
    }
    PHASE(3);
    // ---- softmax (ops.go:83-106): max, exponentials, ordered sum, x *= 1/sum
    if (wave == 0) {
        for (int off = 32; off > 0; off >>= 1) lmax = fmaxf(lmax, __shfl_down(lmax, off, 64));
    }
    const float maxv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(lmax)));
    if (wave == 0 && lane == 0) red[0] = maxv;
    __syncthreads();
    const float mx = red[0];
    for (int t = tid; t <= pos; t += kThreads) scores[t] = fast_exp_scalar(scores[t] - mx);
    __syncthreads();
    if (tid == 0) red[1] = ordered_sum(scores, 1, pos + 1);
    __syncthreads();
    const float sum = red[1];
    if (sum != 0.0f) {
        const float inv = 1.0f / sum;
        for (int t = tid; t <= pos; t += kThreads) scores[t] = scores[t] * inv;
    }
    __syncthreads();
    PHASE(4);

    // ---- out_d = sum_t p_t * v_t,d in t order (no FMA), on waves 2-3; the
    // ring refills group g with keys g + NG groups ahead as it is consumed.
    // The step's own V row comes from LDS (another workgroup appends it).
    float acc = 0.0f;
    if (pv_wave) {
        const float own = sv[d];
        for (int g0 = 0; g0 * VG <= pos; g0 += NG) {
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                const int t0 = (g0 + gi) * VG;
                if (t0 <= pos) {
                    // the group's probabilities first (float4 reads; LDS scores are
                    // padded to a multiple of VG), then the adds, branch-free
                    // (keys past pos leave acc unchanged) so the ring stays in registers
                    float pg[VG];
                    if (lds_scores) {
#pragma unroll
                        for (int i4 = 0; i4 < VG / 4; i4++) {
                            const f32x4 p4 = *reinterpret_cast<const f32x4*>(scores + t0 + 4 * i4);
                            pg[4 * i4] = p4.x; pg[4 * i4 + 1] = p4.y; pg[4 * i4 + 2] = p4.z; pg[4 * i4 + 3] = p4.w;
                        }
                    } else {
#pragma unroll
                        for (int k = 0; k < VG; k++) pg[k] = scores[t0 + k <= pos ? t0 + k : pos];
                    }
                    if (t0 + VG <= pos) {
                        // a whole group below pos (the step's own row is pos): plain adds
#pragma unroll
                        for (int k = 0; k < VG; k++) acc = acc + pg[k] * vr[gi][k];
                    } else {
                        // the last group: keys up to pos, the own row from LDS
#pragma unroll
                        for (int k = 0; k < VG; k++) {
                            const int t = t0 + k;
                            const float v = t == skip ? own : vr[gi][k];
                            const float nacc = acc + pg[k] * v;
                            acc = t <= pos ? nacc : acc;
                        }
                    }
                    if (t0 + NG * VG <= pos) vissue(vr[gi], t0 + NG * VG);
                }
            }
        }
        if (tid - 128 < hd) a.out[h * hd + d] = acc;
    }
    if (a.q_out && pv_wave) {
        // The head's output is hd/32 whole int8 blocks of the Wo activation:
        // quantise them here rather than in every workgroup of the Wo GEMV.
        float sc;
        const bool live = tid - 128 < hd;
        const int32_t qv = quant_lane32(live ? acc : 0.0f, &sc);
        if (live) {
            const int gi = h * hd + d;
            a.q_out[(gi >> 5) * 32 + qx_perm(gi & 31)] = (int8_t)qv;
            if ((gi & 31) == 0) a.q_scale[gi >> 5] = sc;
        }
    }
#ifdef MANTLE_PHASE_TRACE
    __syncthreads();  // the stamp below then marks the whole workgroup's end
#endif
    PHASE(5);
}


// ---------------------------------------------------------------------------
// Split-key attention: two launches that spread one head over many CUs.
//
// attention_scores_split: workgroup (h, s) of kSplitWgs per head scores the
// 64-key chunks s, s + kSplitWgs, ... of head h into the scores buffer; the
// q / k prologue is recomputed by each (it is a few hundred cycles), and the
// (first head, s = 0) workgroup appends the step's K and V rows.
// attention_pv_split: workgroup (h, column block) runs the softmax over the
// head's scores (max, exponentials, the ordered sum, x *= 1/sum) and the V sum
// of its 32 output columns in key order, and quantises them for Wo.  Both
// keep the single-kernel arithmetic and order exactly.
static constexpr int kSplitWgs = 16;

// Kernel variant: kAttnPathSplit (two launches up to kSplitMaxCtx keys, the
// one-launch attention_split_fused beyond), kAttnPathFused (always one
// launch), kAttnPathSingle (attention_decode_v4) or kAttnPathGeneral; the
// first read takes MANTLE_HIP_ATTN ("fused", "single", "general"; anything
// else: split) when set_attention_path has not been called.
//
// Measured on MI355X, the one-launch form is the slower one where both apply
// (Qwen3-0.6B decode 1135 -> 986 tok/s; Qwen3-8B after 16k tokens, 29 tok/s
// against 44 for the split form, both before the transposed V): its V sum runs in one workgroup per
// head, whose CU's memory pipeline then bounds the head's V stream, while the
// second launch of the split form spreads it over head_dim / 32 workgroups.
static std::atomic<int> g_attn_path{-1};

int attention_path() {
    int v = g_attn_path.load();
    if (v >= 0) return v;
    const char* e = getenv("MANTLE_HIP_ATTN");
    v = kAttnPathSplit;
    if (e && !strcmp(e, "fused")) v = kAttnPathFused;
    if (e && !strcmp(e, "single")) v = kAttnPathSingle;
    if (e && !strcmp(e, "general")) v = kAttnPathGeneral;
    int expect = -1;
    g_attn_path.compare_exchange_strong(expect, v);
    return g_attn_path.load();
}

// MANTLE_HIP_PV_LDS=0 keeps the register-ring V sum for the f32 cache.
static bool pv_lds_enabled() {
    const char* e = getenv("MANTLE_HIP_PV_LDS");
    return !(e && !strcmp(e, "0"));
}

static std::atomic<int> g_kv_type{0};
int kv_cache_type() { return g_kv_type.load(); }
bool set_kv_cache_type(int t) {
    if (t != kKvF32 && t != kKvF16 && t != kKvQ8) return false;
    g_kv_type.store(t);
    return true;
}

bool set_attention_path(int path) {
    if (path != kAttnPathSplit && path != kAttnPathSingle && path != kAttnPathGeneral && path != kAttnPathFused)
        return false;
    g_attn_path.store(path);
    return true;
}
// The V-sum launch keeps the probabilities in LDS: up to 128 KiB of the 160
// KiB a gfx950 workgroup may hold.
static constexpr int kSplitMaxCtx = 32768;
static constexpr size_t kMaxLds = 160 * 1024;  // dynamic LDS one gfx950 workgroup may hold

// Dynamic LDS above 64 KiB is allowed per kernel before its launch.
static hipError_t allow_lds(void (*kern)(AttnArgs), size_t bytes) {
    if (bytes <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)bytes);
}

// Query row blockIdx.y of a launch_attention_rows launch: moves a's per-row
// pointers to that row and returns its offset from the first row's position
// (0 and nothing moved for the single-row launches, whose grid has one row).
__device__ __forceinline__ int token_row(AttnArgs& a) {
    const int r = (int)blockIdx.y;
    if (r == 0) return 0;
    a.q += (size_t)r * a.q_row;
    a.out += (size_t)r * a.out_row;
    a.scores += (size_t)r * a.scores_row;
    if (a.q_out) {
        a.q_out += (size_t)r * a.out_row;
        a.q_scale += (size_t)r * (a.out_row / 32);
    }
    return r;
}

// Scores of head h, chunks sidx, sidx + S, ... into the scores buffer (the
// body of attention_scores_split; attention_split_fused runs it first).  KV:
// the cache element type.  kKvF16: DotF16, the scalar order in every ISA
// (internal/backend/simd/ops.go:35-46).  kKvQ8: DotQ8 (ops.go:240-246, the
// scalar order, then times the position's scale) as attnpool.go:100-102 calls
// it; the step's row is already in the cache, so nothing is appended here.
template <int HD, int KV>
__device__ __forceinline__ void scores_split_chunks(const AttnArgs& a, float* lds, int h, int sidx, int S, int pos) {
    constexpr bool F16 = KV == kKvF16, Q8 = KV == kKvQ8;
    float* sq = lds;
    float* sk = lds + 128;
    float* sv = lds + 256;
    float* wbuf = lds + 384;
    constexpr int kp = HD + 4;
    constexpr int kc = kAttnKeys;
    float* kt = lds + kAttnV4Hdr;
    const int tid = threadIdx.x;
    const int kvh = h * a.kv_heads / a.n_head;
    const int nchunks = pos / kc + 1;
    const float* kbase = a.cache_k + (size_t)kvh * a.head_stride;
    const uint16_t* kbase16 = reinterpret_cast<const uint16_t*>(a.cache_k) + (size_t)kvh * a.head_stride;
    const int8_t* kbase8 = reinterpret_cast<const int8_t*>(a.cache_k) + (size_t)kvh * a.head_stride;
    const int skip = a.fused && !Q8 ? pos : -1;
    float* sg = a.scores + (size_t)h * a.max_ctx;
    KeyMap km;
    km.base = a.key_base;
    km.ring = a.key_ring;
    const PrepRegs pr = prep_load<HD>(a, h, kvh, pos);
    __builtin_amdgcn_sched_barrier(0);
    ChunkRegs ck;
    ChunkRegs16 ck16;
    ChunkRegs8 ck8;
    auto issue = [&](int c) {
        const int nk = min(kc, pos + 1 - c * kc);
        if constexpr (Q8) chunk_issue8_t<HD>(ck8, kbase8, a.kv_stride, c * kc, nk, kp, km);
        else if constexpr (F16) chunk_issue16_t<HD>(ck16, kbase16, a.kv_stride, c * kc, nk, kp, skip, km);
        else chunk_issue_t<HD>(ck, kbase, a.kv_stride, c * kc, nk, HD, kp, skip, km);
    };
    issue(sidx);
    prep_finish<HD>(a, pr, kvh, pos, a.fused && sidx == 0 && first_of_group(a, h, kvh), sq, sk, sv, wbuf);
    __syncthreads();
    for (int c = sidx; c < nchunks; c += S) {
        const int t0 = c * kc;
        const int nk = min(kc, pos + 1 - t0);
        if constexpr (Q8) chunk_store8(ck8, kt);
        else if constexpr (F16) chunk_store16(ck16, kt, kp, sk, t0, nk, skip, HD);
        else chunk_store_v4(ck, kt, kp, sk, t0, nk, skip, HD);
        __syncthreads();
        const int cn = c + S;
        if (cn < nchunks) issue(cn);
        if (tid < nk) {
            const float4* qv = reinterpret_cast<const float4*>(sq);
            const float4* kv = reinterpret_cast<const float4*>(kt + tid * kp);
            if constexpr (Q8) sg[t0 + tid] = (dot_parity_v4<HD, kIsaScalar>(qv, kv) * a.k_scale[krow(km, t0 + tid)]) * a.scale;
            else sg[t0 + tid] = (F16 ? dot_parity_v4<HD, kIsaScalar>(qv, kv) : dot_v4_isa<HD>(qv, kv, a.isa)) * a.scale;
        }
        __syncthreads();
    }
}

template <int HD, int KV>
__global__ __launch_bounds__(kThreads) void attention_scores_split(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x % a.n_head, sidx = blockIdx.x / a.n_head;
    const int S = gridDim.x / a.n_head;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos_host) + token_row(a);
    if (sidx >= pos / kAttnKeys + 1) return;  // whole workgroup: no chunk of this context for it
    PHASE_SLOT();
    PHASE(0);
    scores_split_chunks<HD, KV>(a, lds, h, sidx, S, pos);
}

// V column d of one head for the V sum out_d = sum_t p_t * v_t,d (key order,
// no FMA), streamed into a register ring of NG groups of VG keys that is
// filled ahead of its use.  VT (transposed cache): the column's keys are
// contiguous and one load brings several of them (16 bytes of fp32, 8 of f16
// or 16 of int8, widened when used); otherwise one load per key (rows
// kv_stride apart).  `own` (the fused step's V row, a workgroup of this
// launch may still be appending it) replaces key `skip`.  KV = kKvQ8: the sum
// is sum_t (p_t * q_t,d) * s_t (attnpool.go:122-130).  The scales are the same
// for every column: SL, they are staged in LDS beside the probabilities and
// read the same way; otherwise lane k of the wave holds the scale of key
// t0 + k of each group in flight, read back per key with readlane.
template <bool VT, int KV = kKvF32, bool SL = false>
struct VColumn {
    static constexpr bool F16 = KV == kKvF16, Q8 = KV == kKvQ8;
    // a narrow transposed ring costs fewer registers per key: twice the groups
    static constexpr int VG = 32, NG = (F16 || Q8) && VT ? 10 : 5;
    // PF: a group's probabilities are read while the group before it is
    // summed, alternating between two register buffers (NG even).  It pays
    // for the q8_0 sum (4B after 2k tokens 237 -> 269 tok/s); the f32 / f16
    // sums keep their deeper V rings instead (the extra buffer cost them a
    // ring group: 310 -> 299 tok/s).
    static constexpr bool PF = Q8 && VT;
    static_assert(!PF || NG % 2 == 0, "groups alternate between two probability buffers");
    static constexpr bool RAW = (F16 || Q8) && VT;
    f32x4 r[RAW ? 1 : NG][VG / 4];  // fp32 keys (for RAW: the group being summed, slot 0)
    u32x2 h[F16 && VT ? NG : 1][VG / 4];  // raw f16 keys (VT) until used
    u32x4 b[Q8 && VT ? NG : 1][VG / 16];  // raw int8 keys (VT) until used
    float sr[Q8 && !SL ? NG : 1];         // Q8 without SL: per-key scales, key t0 + k in lane k
    const float* col;
    const uint16_t* col16;
    const int8_t* col8;
    const float* vscale;
    size_t step;
    float own;
    int skip, pos;
    KeyMap km;  // window / ring rows (row-major caches only)

    __device__ __forceinline__ void init(const AttnArgs& a, int kvh, int hd, int d, int pos_) {
        pos = pos_;
        skip = a.fused && !Q8 ? pos : -1;
        km.base = a.key_base;
        km.ring = a.key_ring;
        const uint16_t* c16 = reinterpret_cast<const uint16_t*>(a.cache_v);
        const int8_t* c8 = reinterpret_cast<const int8_t*>(a.cache_v);
        vscale = a.v_scale;
        if (VT) {
            col = a.cache_v + (size_t)(kvh * hd + d) * a.vt_stride;
            col16 = c16 + (size_t)(kvh * hd + d) * a.vt_stride;
            col8 = c8 + (size_t)(kvh * hd + d) * a.vt_stride;
            step = 1;
        } else {
            col = a.cache_v + (size_t)kvh * a.head_stride + d;
            col16 = c16 + (size_t)kvh * a.head_stride + d;
            col8 = c8 + (size_t)kvh * a.head_stride + d;
            step = (size_t)a.kv_stride;
        }
        own = skip >= 0 ? (F16 ? f16_cache_round(a.v[kvh * hd + d]) : a.v[kvh * hd + d]) : 0.0f;
    }
    __device__ __forceinline__ f32x4 patch(f32x4 v, int t) const {
        if (skip >= 0) {
            v.x = t == skip ? own : v.x;
            v.y = t + 1 == skip ? own : v.y;
            v.z = t + 2 == skip ? own : v.z;
            v.w = t + 3 == skip ? own : v.w;
        }
        return v;
    }
    __device__ __forceinline__ int vt_key(int t0, int k4) const { return t0 + 4 * k4 <= pos ? t0 + 4 * k4 : (pos & ~3); }
    __device__ __forceinline__ void issue(int g, int t0) {
        if constexpr (Q8 && !SL) {
            const int tk = t0 + (int)(threadIdx.x & 31);
            sr[g] = vscale[krow(km, tk <= pos ? tk : pos)];
        }
        if (VT && t0 + VG <= pos) {
            // the whole group lies below pos: no clamp and no own row, so the
            // loads are one base address plus immediate offsets
            if constexpr (Q8) {
#pragma unroll
                for (int j = 0; j < VG / 16; j++) b[g][j] = reinterpret_cast<const u32x4*>(col8 + t0)[j];
            } else {
#pragma unroll
                for (int k4 = 0; k4 < VG / 4; k4++) {
                    if constexpr (F16) h[g][k4] = reinterpret_cast<const u32x2*>(col16 + t0)[k4];
                    else r[g][k4] = reinterpret_cast<const f32x4*>(col + t0)[k4];
                }
            }
        } else if (VT) {
            if constexpr (Q8) {
#pragma unroll
                for (int j = 0; j < VG / 16; j++) {
                    const int t = t0 + 16 * j <= pos ? t0 + 16 * j : (pos & ~15);  // read, never added
                    b[g][j] = *reinterpret_cast<const u32x4*>(col8 + t);
                }
            } else {
#pragma unroll
                for (int k4 = 0; k4 < VG / 4; k4++) {
                    const int t = vt_key(t0, k4);  // keys past pos are read, never added
                    if constexpr (F16) h[g][k4] = *reinterpret_cast<const u32x2*>(col16 + t);
                    else r[g][k4] = patch(*reinterpret_cast<const f32x4*>(col + t), t);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < VG; k++) {
                const int t = t0 + k <= pos ? t0 + k : pos;
                const size_t row = (size_t)krow(km, t);
                const float v = Q8 ? (float)col8[row * step]
                                   : (F16 ? f16_cache_load(col16[row * step]) : col[row * step]);
                r[g][k >> 2][k & 3] = t == skip ? own : v;
            }
        }
    }
    // Group g as fp32 (a narrow transposed ring is widened here, when its loads are needed).
    __device__ __forceinline__ void widen(int g, int t0) {
        if constexpr (Q8 && VT) {
#pragma unroll
            for (int j = 0; j < VG / 16; j++)
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t x = b[g][j][w];
                    f32x4 v;
                    v.x = q8_byte_sdwa<0>(x);
                    v.y = q8_byte_sdwa<1>(x);
                    v.z = q8_byte_sdwa<2>(x);
                    v.w = q8_byte_sdwa<3>(x);
                    r[0][4 * j + w] = v;
                }
        } else if constexpr (F16 && VT) {
            const bool whole = t0 + VG <= pos;  // as in issue(): no own row to patch
#pragma unroll
            for (int k4 = 0; k4 < VG / 4; k4++) {
                f32x4 v;
                v.x = f16_cache_load((uint16_t)(h[g][k4].x & 0xFFFFu));
                v.y = f16_cache_load((uint16_t)(h[g][k4].x >> 16));
                v.z = f16_cache_load((uint16_t)(h[g][k4].y & 0xFFFFu));
                v.w = f16_cache_load((uint16_t)(h[g][k4].y >> 16));
                r[0][k4] = whole ? v : patch(v, vt_key(t0, k4));
            }
        }
    }
    // Term k of group g: p * v, or for Q8 (p * q) * s (s: sl, the key's scale read from LDS, for SL).
    __device__ __forceinline__ float term(float p, float v, int g, int k, float sl) const {
        if constexpr (Q8 && SL) {
            return (p * v) * sl;
        } else if constexpr (Q8) {
            const float sk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sr[g]), k));
            return (p * v) * sk;
        } else {
            return p * v;
        }
    }
    // Fill the ring (before the probabilities are ready).
    __device__ __forceinline__ void prime() {
#pragma unroll
        for (int g = 0; g < NG; g++)
            if (g * VG <= pos) issue(g, g * VG);
    }
    // The ordered sum over keys 0 .. pos with probabilities p[0 .. pos] (and,
    // SL, the keys' scales ls[0 .. pos]; both readable up to a multiple of VG).
    __device__ __forceinline__ float sum(const float* p, const float* ls = nullptr) {
        float acc = 0.0f;
        float pb[PF ? 2 : 1][VG];
        auto load_p = [&](float* dst, int t0) {
#pragma unroll
            for (int i4 = 0; i4 < VG / 4; i4++) {
                const f32x4 p4 = *reinterpret_cast<const f32x4*>(p + t0 + 4 * i4);
                dst[4 * i4] = p4.x; dst[4 * i4 + 1] = p4.y; dst[4 * i4 + 2] = p4.z; dst[4 * i4 + 3] = p4.w;
            }
        };
        if constexpr (PF) load_p(pb[0], 0);
        for (int g0 = 0; g0 * VG <= pos; g0 += NG) {
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                const int t0 = (g0 + gi) * VG;
                if (t0 <= pos) {
                    if constexpr (PF) {
                        if (t0 + VG <= pos) load_p(pb[(gi + 1) & 1], t0 + VG);
                    }
                    widen(gi, t0);
                    const int ri = RAW ? 0 : gi;
                    if constexpr (!PF) load_p(pb[0], t0);
                    const float* pg = pb[PF ? (gi & 1) : 0];
                    float sg[SL ? VG : 1];
                    if constexpr (SL) {
#pragma unroll
                        for (int i4 = 0; i4 < VG / 4; i4++) {
                            const f32x4 s4 = *reinterpret_cast<const f32x4*>(ls + t0 + 4 * i4);
                            sg[4 * i4] = s4.x; sg[4 * i4 + 1] = s4.y; sg[4 * i4 + 2] = s4.z; sg[4 * i4 + 3] = s4.w;
                        }
                    }
                    if (t0 + VG <= pos + 1) {
#pragma unroll
                        for (int k = 0; k < VG; k++) acc = acc + term(pg[k], r[ri][k >> 2][k & 3], gi, k, sg[SL ? k : 0]);
                    } else {
#pragma unroll
                        for (int k = 0; k < VG; k++) {
                            const float nacc = acc + term(pg[k], r[ri][k >> 2][k & 3], gi, k, sg[SL ? k : 0]);
                            acc = t0 + k <= pos ? nacc : acc;
                        }
                    }
                    if (t0 + NG * VG <= pos) issue(gi, t0 + NG * VG);
                }
            }
        }
        return acc;
    }
};

// Softmax of head h's scores (ops.go:83-106: max, exponentials, the ordered
// sum, x *= 1/sum) into p (LDS or, PG, in place in the scores buffer); red:
// 5 floats of LDS.  Whole workgroup.
template <bool PG>
__device__ __forceinline__ void head_softmax(const float* sg, float* p, float* red, int pos) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float m = -INFINITY;
    for (int t = tid; t <= pos; t += kThreads) {
        const float v = sg[t];
        if (!PG) p[t] = v;
        m = fmaxf(m, v);
    }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_down(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int t = tid; t <= pos; t += kThreads) p[t] = fast_exp_scalar(p[t] - mx);
    if (PG) __threadfence_block();
    __syncthreads();
    if (tid == 0) red[4] = ((uintptr_t)p & 15) ? ordered_sum(p, 1, pos + 1) : ordered_sum_contig(p, pos + 1);
    __syncthreads();
    const float sum = red[4];
    if (sum != 0.0f) {
        const float inv = 1.0f / sum;
        for (int t = tid; t <= pos; t += kThreads) p[t] = p[t] * inv;
    }
    if (PG) __threadfence_block();
    __syncthreads();
}

// The output value of column gi (= h*HD + d) and, with q_out, its int8 block
// of the Wo activation (32 consecutive lanes hold one whole block).
__device__ __forceinline__ void store_attn_out(const AttnArgs& a, int gi, float acc, bool live) {
    if (live) a.out[gi] = acc;
    if (a.q_out) {
        float sc;
        const int32_t qv = quant_lane32(acc, &sc);
        if (live) {
            a.q_out[(gi >> 5) * 32 + qx_perm(gi & 31)] = (int8_t)qv;
            if ((gi & 31) == 0) a.q_scale[gi >> 5] = sc;
        }
    }
}

// Softmax and the V sum of all of head h's columns, by the last of the head's
// S score workgroups to finish (attention_split_fused), one column per lane of
// waves 0 .. HD/64-1.
template <int HD, bool PG, bool VT, int KV>
__device__ __forceinline__ void softmax_pv_head(const AttnArgs& a, float* lds, int h, int pos) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = h * a.kv_heads / a.n_head;
    float* sg = a.scores + (size_t)h * a.max_ctx;
    float* p = PG ? sg : lds;
    float* red = PG ? lds : lds + (a.max_ctx + 31) / 32 * 32;
    const bool pv_wave = wave < HD / 64;
    const int d = wave * 64 + lane;
    VColumn<VT, KV> vc;
    vc.init(a, kvh, HD, pv_wave ? d : 0, pos);
    if (pv_wave) vc.prime();  // the ring fills while the softmax runs
    head_softmax<PG>(sg, p, red, pos);
    if (!pv_wave) return;
    store_attn_out(a, h * HD + d, vc.sum(p), true);
}

// One launch for the split-key attention: workgroup (h, s) scores its chunks
// like attention_scores_split, then counts itself done on the head's counter;
// the last of the head's S workgroups (the others have published their scores
// with a device-scope fence before counting) resets the counter and runs
// softmax_pv_head.  Every workgroup counts, with or without a chunk, so the
// last one always arrives and every wave exits.
template <int HD, bool PG, bool VT, int KV>
__global__ __launch_bounds__(kThreads) void attention_split_fused(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x % a.n_head, sidx = blockIdx.x / a.n_head;
    const int S = gridDim.x / a.n_head;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    PHASE_SLOT();
    PHASE(0);
    if (sidx < pos / kAttnKeys + 1) scores_split_chunks<HD, KV>(a, lds, h, sidx, S, pos);
    __threadfence();  // this workgroup's scores (and cache rows) before its arrival
    __syncthreads();
    __shared__ int is_last;  // outside the dynamic LDS that the softmax overwrites
    if (threadIdx.x == 0) {
        const unsigned old = atomicAdd(a.counters + h, 1u);
        const int last = old == (unsigned)(S - 1);
        if (last) atomicExch(a.counters + h, 0u);  // ready for the next launch
        is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();  // the other workgroups' scores, seen after their arrivals
    PHASE(4);
    softmax_pv_head<HD, PG, VT, KV>(a, lds, h, pos);
}

// SL (q8_0 cache): the keys' scales are staged in LDS after the probabilities
// (pcap + 32 floats in), by all four waves before the softmax's barriers.
template <int HD, bool VT, int KV, bool SL = false>
__global__ __launch_bounds__(kThreads) void attention_pv_split(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    constexpr int DB = 32;  // output columns per workgroup: one int8 block of the Wo activation
    const int nd = HD / DB;
    const int h = blockIdx.x / nd, db = blockIdx.x % nd;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = h * a.kv_heads / a.n_head;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos_host) + token_row(a);
    const int pcap = (a.max_ctx + 31) / 32 * 32;
    const float* sg = a.scores + (size_t)h * a.max_ctx;
    PHASE_SLOT();
    PHASE(0);
    // wave 0 (lanes 0-31 the columns; 32-63 shadow them) streams its V
    // columns into a register ring from the start
    const int d = db * DB + (lane & 31);
    VColumn<VT, KV, SL> vc;
    vc.init(a, kvh, HD, d, pos);
    vc.skip = -1;  // the previous launch appended the step's row
    if (wave == 0) vc.prime();
    float* ls = lds + pcap + 32;
    if constexpr (SL)
        for (int t = tid; t <= pos; t += kThreads) ls[t] = a.v_scale[krow(KeyMap{a.key_base, a.key_ring}, t)];
    head_softmax<false>(sg, lds, lds + pcap, pos);
    PHASE(1);
    if (wave != 0) return;
    store_attn_out(a, h * HD + d, vc.sum(lds, ls), lane < 32);
    PHASE(2);
}

// The V-sum launch with V staged in LDS (transposed cache): waves 1-3 load
// the head's 32 columns in chunks of kPvChunk keys (two chunks of loads in
// flight in registers, widened to fp32 -- f16 through the flushing hardware
// conversion, int8 exactly -- and written to a double-buffered LDS slot),
// while wave 0 runs the ordered V sum of each chunk from LDS, one chunk
// behind: the chain wave's operands come from LDS instead of a register ring
// that only reaches 160-320 keys ahead, and it spends no instruction on
// widening.  kKvQ8: the loaders stage each chunk's key scales beside its
// columns and the terms are (p * q) * s.  One barrier per chunk keeps
// the waves in step; every wave runs the same number of them.
static constexpr int kPvChunk = 256;
static constexpr int kPvLdsMinCtx = 512;  // caches of more positions stage V in LDS
static constexpr int kPvPitch = kPvChunk + 4;  // floats per staged column (16-byte rows, banks skewed)
static constexpr int kPvItems = (32 * kPvChunk / 4 + 191) / 192;  // float4 per loader lane per chunk

template <int HD, int KV>
__global__ __launch_bounds__(kThreads) void attention_pv_lds(AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    constexpr bool F16 = KV == kKvF16, Q8 = KV == kKvQ8;
    // raw loader registers: 4 keys of one column per item
    typedef typename std::conditional<F16, u32x2, typename std::conditional<Q8, uint32_t, f32x4>::type>::type Raw;
    constexpr int DB = 32;
    const int nd = HD / DB;
    const int h = blockIdx.x / nd, db = blockIdx.x % nd;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = h * a.kv_heads / a.n_head;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos_host) + token_row(a);
    const int pcap = (a.max_ctx + 31) / 32 * 32;
    const float* sg = a.scores + (size_t)h * a.max_ctx;
    float* p = lds;
    float* red = lds + pcap;
    float* vr = red + 32;                  // [2][32 columns][kPvPitch]
    float* vsc = vr + 2 * 32 * kPvPitch;  // Q8: [2][kPvChunk] key scales
    const int nch = pos / kPvChunk + 1;
    // loader lane lt of waves 1-3: item e = lt + 192 i is keys 4 (e % 64) .. +3 of column e / 64
    const int lt = tid - 64;
    const size_t colofs = (size_t)(kvh * HD + db * DB) * a.vt_stride;
    const char* colbase = reinterpret_cast<const char*>(a.cache_v) + colofs * (F16 ? 2 : (Q8 ? 1 : 4));
    constexpr int esz = F16 ? 2 : (Q8 ? 1 : 4);
    Raw la[kPvItems], lb[kPvItems];
    constexpr int NS = Q8 ? (kPvChunk + 191) / 192 : 1;  // scales per loader lane per chunk
    float sa[NS], sb[NS];
    auto issue_scales = [&](float (&dst)[NS], int c) {
        if constexpr (Q8) {
#pragma unroll
            for (int i = 0; i < NS; i++) {
                const int t = c * kPvChunk + lt + 192 * i;
                dst[i] = a.v_scale[t <= pos ? t : pos];
            }
        }
    };
    auto store_scales = [&](const float (&src)[NS], int slot) {
        if constexpr (Q8) {
#pragma unroll
            for (int i = 0; i < NS; i++)
                if (lt + 192 * i < kPvChunk) vsc[slot * kPvChunk + lt + 192 * i] = src[i];
        }
    };
    auto issue = [&](Raw (&dst)[kPvItems], int c) {
#pragma unroll
        for (int i = 0; i < kPvItems; i++) {
            const int e = lt + 192 * i;
            const int ee = e < 32 * kPvChunk / 4 ? e : 0;
            int t = c * kPvChunk + 4 * (ee & 63);
            t = t <= pos ? t : (pos & ~3);  // keys past pos are staged, never added
            dst[i] = *reinterpret_cast<const Raw*>(colbase + ((size_t)(ee >> 6) * a.vt_stride + t) * esz);
        }
    };
    // the loaders store p_t * v_t (f32 / f16: the whole term; q8_0: p_t * q_t,
    // which the chain wave multiplies by the key's scale) -- the chain wave's
    // own first multiply, done here off its critical path
    auto store = [&](const Raw (&src)[kPvItems], int slot, int c) {
#pragma unroll
        for (int i = 0; i < kPvItems; i++) {
            const int e = lt + 192 * i;
            f32x4 v;
            if constexpr (F16) {
                v.x = f16_cache_load((uint16_t)(src[i].x & 0xFFFFu));
                v.y = f16_cache_load((uint16_t)(src[i].x >> 16));
                v.z = f16_cache_load((uint16_t)(src[i].y & 0xFFFFu));
                v.w = f16_cache_load((uint16_t)(src[i].y >> 16));
            } else if constexpr (Q8) {
                v.x = q8_byte_sdwa<0>(src[i]);
                v.y = q8_byte_sdwa<1>(src[i]);
                v.z = q8_byte_sdwa<2>(src[i]);
                v.w = q8_byte_sdwa<3>(src[i]);
            } else {
                v = src[i];
            }
            {
                const f32x4 p4 = *reinterpret_cast<const f32x4*>(p + c * kPvChunk + 4 * (e & 63));
                v.x = p4.x * v.x; v.y = p4.y * v.y; v.z = p4.z * v.z; v.w = p4.w * v.w;
            }
            if (e < 32 * kPvChunk / 4)
                *reinterpret_cast<f32x4*>(vr + (slot * 32 + (e >> 6)) * kPvPitch + 4 * (e & 63)) = v;
        }
    };
    if (wave != 0) {  // the first chunks' loads overlap the softmax
        issue(la, 0);
        issue_scales(sa, 0);
        if (nch > 1) {
            issue(lb, 1);
            issue_scales(sb, 1);
        }
    }
    head_softmax<false>(sg, p, red, pos);
    if (wave != 0) {
        store(la, 0, 0);
        store_scales(sa, 0);
        if (nch > 2) {
            issue(la, 2);
            issue_scales(sa, 2);
        }
    }
    __syncthreads();
    const int d = lane & 31;
    float acc = 0.0f;
    // wave 0: the ordered sum of chunk c from LDS slot `slot`
    auto sum_chunk = [&](int slot, int c) {
        const float* col = vr + (slot * 32 + d) * kPvPitch;
        const float* cs = vsc + slot * kPvChunk;
        const int t0 = c * kPvChunk;
        const int n = min(kPvChunk, pos + 1 - t0);
        // batches of KB keys: their reads issued together, one LDS latency per batch
        constexpr int KB = 64;
        for (int k0 = 0; k0 < n; k0 += KB) {
            float vg[KB], sgk[Q8 ? KB : 1];
#pragma unroll
            for (int i4 = 0; i4 < KB / 4; i4++) {
                const f32x4 v4 = *reinterpret_cast<const f32x4*>(col + k0 + 4 * i4);
                vg[4 * i4] = v4.x; vg[4 * i4 + 1] = v4.y; vg[4 * i4 + 2] = v4.z; vg[4 * i4 + 3] = v4.w;
                if constexpr (Q8) {
                    const f32x4 s4 = *reinterpret_cast<const f32x4*>(cs + k0 + 4 * i4);
                    sgk[4 * i4] = s4.x; sgk[4 * i4 + 1] = s4.y; sgk[4 * i4 + 2] = s4.z; sgk[4 * i4 + 3] = s4.w;
                }
            }
            auto term = [&](int k) {
                if constexpr (Q8) return vg[k] * sgk[k];  // (p_t * q_t, formed by the loaders) * s_t
                else return vg[k];                         // p_t * v_t, formed by the loaders
            };
            if (k0 + KB <= n) {
#pragma unroll
                for (int k = 0; k < KB; k++) acc = acc + term(k);
            } else {
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const float nacc = acc + term(k);
                    acc = k0 + k < n ? nacc : acc;
                }
            }
        }
    };
    for (int c = 0; c < nch; c += 2) {
        if (wave == 0) {
            sum_chunk(0, c);
        } else {
            if (c + 1 < nch) {
                store(lb, 1, c + 1);
                store_scales(sb, 1);
            }
            if (c + 3 < nch) {
                issue(lb, c + 3);
                issue_scales(sb, c + 3);
            }
        }
        __syncthreads();
        if (c + 1 >= nch) break;
        if (wave == 0) {
            sum_chunk(1, c + 1);
        } else {
            if (c + 2 < nch) {
                store(la, 0, c + 2);
                store_scales(sa, 0);
            }
            if (c + 4 < nch) {
                issue(la, c + 4);
                issue_scales(sa, c + 4);
            }
        }
        __syncthreads();
    }
    if (wave != 0) return;
    store_attn_out(a, h * HD + db * DB + d, acc, lane < 32);
}

// The library's zeroed arrival counters (one set per device, allocated on first
// use, never freed), for callers that pass none.  Each launch leaves them at
// zero again, so launches stream-ordered after one another may share them;
// launches that may overlap need counters of their own.
static constexpr int kLibCounters = 4096;
static unsigned* library_counters(int n_head) {
    static std::mutex mu;
    static unsigned* per_dev[64] = {};
    if (n_head > kLibCounters) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!per_dev[dev]) {
        unsigned* p = nullptr;
        if (hipMalloc((void**)&p, sizeof(unsigned) * kLibCounters) != hipSuccess) return nullptr;
        if (hipMemset(p, 0, sizeof(unsigned) * kLibCounters) != hipSuccess) { (void)hipFree(p); return nullptr; }
        per_dev[dev] = p;
    }
    return per_dev[dev];
}

// The two-launch split form (scores, then softmax and V sum) for `rows`
// query rows (grid rows; 1 for a decode step).
static hipError_t launch_split_two(const AttnArgs& a, int rows, hipStream_t stream) {
    const bool vt = a.vt_stride > 0;
    const int kvt = a.k_type, vtt = a.v_type;
    const int S = min(kSplitWgs, (a.max_ctx + kAttnKeys - 1) / kAttnKeys);
    const size_t smem_a = sizeof(float) * (kAttnV4Hdr + (size_t)kAttnKeys * (a.head_dim + 4));
    const size_t smem_b = sizeof(float) * ((size_t)(a.max_ctx + 31) / 32 * 32 + 8);
    const int nd = a.head_dim / 32;
    // kernel[hd 128][vt][cache type]
    void (*const pv[2][2][3])(AttnArgs) = {
        {{attention_pv_split<64, false, kKvF32>, attention_pv_split<64, false, kKvF16>,
          attention_pv_split<64, false, kKvQ8>},
         {attention_pv_split<64, true, kKvF32>, attention_pv_split<64, true, kKvF16>,
          attention_pv_split<64, true, kKvQ8>}},
        {{attention_pv_split<128, false, kKvF32>, attention_pv_split<128, false, kKvF16>,
          attention_pv_split<128, false, kKvQ8>},
         {attention_pv_split<128, true, kKvF32>, attention_pv_split<128, true, kKvF16>,
          attention_pv_split<128, true, kKvQ8>}}};
    void (*const sc[2][3])(AttnArgs) = {
        {attention_scores_split<64, kKvF32>, attention_scores_split<64, kKvF16>, attention_scores_split<64, kKvQ8>},
        {attention_scores_split<128, kKvF32>, attention_scores_split<128, kKvF16>,
         attention_scores_split<128, kKvQ8>}};
    auto pvk = pv[a.head_dim == 128][vt][vtt];
    size_t smem_pv = smem_b;
    const size_t pcap = (size_t)(a.max_ctx + 31) / 32 * 32;
    const size_t smem_lv = sizeof(float) * (pcap + 32 + 2 * 32 * kPvPitch + (vtt == kKvQ8 ? 2 * kPvChunk : 0));
    // (short caches keep the register ring: at a few hundred keys the
    // loader waves' barriers cost more than they save, 6.30 -> 6.55 us)
    const bool lv_used = vt && a.max_ctx > kPvLdsMinCtx && smem_lv <= kMaxLds && pv_lds_enabled();
    if (lv_used) {  // V staged in LDS
        void (*const lv[2][3])(AttnArgs) = {
            {attention_pv_lds<64, kKvF32>, attention_pv_lds<64, kKvF16>, attention_pv_lds<64, kKvQ8>},
            {attention_pv_lds<128, kKvF32>, attention_pv_lds<128, kKvF16>, attention_pv_lds<128, kKvQ8>}};
        pvk = lv[a.head_dim == 128][vtt];
        smem_pv = smem_lv;
    }
    const size_t smem_sl = sizeof(float) * (2 * ((size_t)(a.max_ctx + 31) / 32 * 32) + 32);
    if (!lv_used && vtt == kKvQ8 && smem_sl <= kMaxLds) {  // q8_0 scales beside the probabilities
        void (*const pvs[2][2])(AttnArgs) = {
            {attention_pv_split<64, false, kKvQ8, true>, attention_pv_split<64, true, kKvQ8, true>},
            {attention_pv_split<128, false, kKvQ8, true>, attention_pv_split<128, true, kKvQ8, true>}};
        pvk = pvs[a.head_dim == 128][vt];
        smem_pv = smem_sl;
    }
    const hipError_t e = allow_lds(pvk, smem_pv);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sc[a.head_dim == 128][kvt], dim3(a.n_head * S, rows), dim3(kThreads), smem_a, stream, a);
    hipLaunchKernelGGL(pvk, dim3(a.n_head * nd, rows), dim3(kThreads), smem_pv, stream, a);
    return hipGetLastError();
}

hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t stream) {
    if (!a.q || !a.cache_k || !a.cache_v || !a.out || a.n_head <= 0 || a.kv_heads <= 0 || a.head_dim <= 0 ||
        a.head_dim > 256 || (a.head_dim & 3) || (a.kv_stride & 3) || (a.head_stride & 3) || a.max_ctx <= 0)
        return hipErrorInvalidValue;
    // rows of one head must not overlap rows of the next: either interleaved
    // ([pos][kv_heads*hd]) or head-major ([kv_head][max_ctx][hd])
    const bool interleaved = a.head_stride == a.head_dim && a.kv_stride >= a.kv_heads * a.head_dim;
    const bool head_major = a.kv_stride == a.head_dim && a.head_stride >= a.max_ctx * a.head_dim;
    if (!interleaved && !head_major) return hipErrorInvalidValue;
    if (((uintptr_t)a.cache_k | (uintptr_t)a.cache_v) & 15) return hipErrorInvalidValue;
    if (a.fused && (!a.k || !a.v)) return hipErrorInvalidValue;
    if (a.q_out && (!a.q_scale || (a.head_dim & 31))) return hipErrorInvalidValue;
    if (!a.pos_dev && (a.pos_host < 0 || a.pos_host >= a.max_ctx)) return hipErrorInvalidValue;
    if (a.rope_cos && (!a.rope_sin || (a.head_dim & 1))) return hipErrorInvalidValue;
    const bool lds_scores = a.max_ctx <= kAttnLdsScores;
    if (!lds_scores && !a.scores) return hipErrorInvalidValue;
    const int mode = attention_path();
    const bool fast_hd = a.head_dim == 128 || a.head_dim == 64;
    const bool vt = a.vt_stride > 0;
    const bool split_ok = fast_hd && a.scores && (mode == kAttnPathSplit || mode == kAttnPathFused);
    if (vt && (!split_ok || (a.vt_stride & 3) || a.vt_stride < (a.max_ctx + 3) / 4 * 4))
        return hipErrorInvalidValue;  // the transposed V cache is read by the split kernels only
    if ((a.key_base || a.key_ring) && (!split_ok || a.fused || vt || a.key_base < 0 || a.key_ring < 0))
        return hipErrorInvalidValue;  // window / ring rows: row-major caches on the split kernels
    const int kt = a.k_type, vtt = a.v_type;  // cache element types of K and V
    if (kt < kKvF32 || kt > kKvQ8 || vtt < kKvF32 || vtt > kKvQ8) return hipErrorInvalidValue;
    if ((kt != kKvF32 || vtt != kKvF32) && !split_ok)
        return hipErrorInvalidValue;  // f16 / q8_0 caches are read by the split kernels only
    const bool any_q8 = kt == kKvQ8 || vtt == kKvQ8;
    if (kt == kKvQ8 && (!a.k_scale || (a.kv_stride & 15) || (a.head_stride & 15))) return hipErrorInvalidValue;
    if (vtt == kKvQ8 && (!a.v_scale || (!vt && ((a.kv_stride & 15) || (a.head_stride & 15))) ||
                         (vt && ((a.vt_stride & 15) || a.vt_stride < (a.max_ctx + 15) / 16 * 16))))
        return hipErrorInvalidValue;  // 16-byte int8 rows, (transposed V) 16-key groups of a column
    // q8_0 and mixed caches: the two-launch split form only
    if ((any_q8 || kt != vtt) && a.max_ctx > kSplitMaxCtx) return hipErrorInvalidValue;
    const bool f16 = kt == kKvF16;
    if (split_ok && !any_q8 && kt == vtt && (mode == kAttnPathFused || a.max_ctx > kSplitMaxCtx)) {
        AttnArgs f = a;
        if (!f.counters) f.counters = library_counters(a.n_head);
        if (!f.counters) return hipErrorInvalidValue;
        const int S = min(kSplitWgs, (a.max_ctx + kAttnKeys - 1) / kAttnKeys);
        const size_t smem_a = sizeof(float) * (kAttnV4Hdr + (size_t)kAttnKeys * (a.head_dim + 4));
        const size_t smem_p = sizeof(float) * ((size_t)(a.max_ctx + 31) / 32 * 32 + 8);
        const bool pg = smem_p > 64 * 1024;  // probabilities in place in the scores buffer
        const size_t smem = pg || smem_p < smem_a ? smem_a : smem_p;
        const dim3 grid(a.n_head * S);
        // kernel[hd 128][pg][vt][f16]
        void (*const kerns[2][2][2][2])(AttnArgs) = {
            {{{attention_split_fused<64, false, false, false>, attention_split_fused<64, false, false, true>},
              {attention_split_fused<64, false, true, false>, attention_split_fused<64, false, true, true>}},
             {{attention_split_fused<64, true, false, false>, attention_split_fused<64, true, false, true>},
              {attention_split_fused<64, true, true, false>, attention_split_fused<64, true, true, true>}}},
            {{{attention_split_fused<128, false, false, false>, attention_split_fused<128, false, false, true>},
              {attention_split_fused<128, false, true, false>, attention_split_fused<128, false, true, true>}},
             {{attention_split_fused<128, true, false, false>, attention_split_fused<128, true, false, true>},
              {attention_split_fused<128, true, true, false>, attention_split_fused<128, true, true, true>}}}};
        hipLaunchKernelGGL(kerns[a.head_dim == 128][pg][vt][f16], grid, dim3(kThreads), smem, stream, f);
        return hipGetLastError();
    }
    if (split_ok) return launch_split_two(a, 1, stream);
    if (fast_hd && mode != kAttnPathGeneral) {
        const size_t smem = sizeof(float) * (kAttnV4Hdr + (size_t)kAttnKeys * (a.head_dim + 4) +
                                             (lds_scores ? (a.max_ctx + 31) / 32 * 32 : 0));
        if (a.head_dim == 128)
            hipLaunchKernelGGL(attention_decode_v4<128>, dim3(a.n_head), dim3(kThreads), smem, stream, a);
        else
            hipLaunchKernelGGL(attention_decode_v4<64>, dim3(a.n_head), dim3(kThreads), smem, stream, a);
        return hipGetLastError();
    }
    const int kc = a.head_dim <= 128 ? kAttnKeys : (kThreads * 32) / a.head_dim;
    const size_t smem = sizeof(float) * (kAttnHdr + (size_t)kc * (a.head_dim + 1) + (lds_scores ? a.max_ctx : 0));
    hipLaunchKernelGGL(attention_decode_kernel, dim3(a.n_head), dim3(kThreads), smem, stream, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prompt rows, batched per kv head: the decode kernels' arithmetic for every
// (row, head), with each K chunk and V column loaded once for a block of
// kRowsQ (row, head) queries of one kv group instead of once per query.
// Query qi of block b is row b*RB + qi/G, head g*G + qi%G (G = n_head /
// kv_heads, RB = kRowsQ / G rows per block).
static constexpr int kRowsQ = 32;

// Scores: workgroup (kv head g, key chunk c, row block b) stages the chunk's
// 64 keys (widened to fp32) and the block's queries in LDS; wave w takes
// queries w, w+4, ..., lane k key t0+k: s = dot_isa(q, k) * scale, as
// scores_split_chunks computes it.
template <int HD, int KV>
__global__ __launch_bounds__(kThreads) void attention_scores_rows(AttnArgs a, int rows) {
    extern __shared__ __align__(16) float lds[];
    constexpr bool F16 = KV == kKvF16, Q8 = KV == kKvQ8;
    constexpr int kp = HD + 4, kc = kAttnKeys;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int G = a.n_head / a.kv_heads, RB = kRowsQ / G;
    const int g = blockIdx.x, c = blockIdx.y;
    const int r0 = (int)blockIdx.z * RB;
    const int rn = min(RB, rows - r0);
    const int pos0 = a.pos_host + r0, t0 = c * kc;
    if (rn <= 0 || t0 > pos0 + rn - 1) return;  // every row of the block ends before the chunk
    const int nk = min(kc, pos0 + rn - t0);      // keys up to the block's last position
    float* kt = lds;                             // [64 keys][kp]
    float* sq = lds + kc * kp;                   // [queries][HD]
    ChunkRegs ck;
    ChunkRegs16 ck16;
    ChunkRegs8 ck8;
    if constexpr (Q8)
        chunk_issue8_t<HD>(ck8, reinterpret_cast<const int8_t*>(a.cache_k) + (size_t)g * a.head_stride, a.kv_stride,
                           t0, nk, kp);
    else if constexpr (F16)
        chunk_issue16_t<HD>(ck16, reinterpret_cast<const uint16_t*>(a.cache_k) + (size_t)g * a.head_stride,
                            a.kv_stride, t0, nk, kp, -1);
    else
        chunk_issue_t<HD>(ck, a.cache_k + (size_t)g * a.head_stride, a.kv_stride, t0, nk, HD, kp, -1);
    const int nq = rn * G;
    for (int i = tid * 4; i < nq * HD; i += kThreads * 4) {
        const int qi = i / HD, d = i - qi * HD;
        const int ri = qi / G, hi = qi - ri * G;
        *reinterpret_cast<f32x4*>(sq + i) =
            *reinterpret_cast<const f32x4*>(a.q + (size_t)(r0 + ri) * a.q_row + (g * G + hi) * HD + d);
    }
    if constexpr (Q8) chunk_store8(ck8, kt);
    else if constexpr (F16) chunk_store16(ck16, kt, kp, nullptr, t0, nk, -1, HD);
    else chunk_store_v4(ck, kt, kp, nullptr, t0, nk, -1, HD);
    __syncthreads();
    const int t = t0 + lane;
    for (int qi = wave; qi < nq; qi += kThreads / 64) {
        const int ri = qi / G, hi = qi - ri * G;
        if (t > pos0 + ri) continue;
        float* sg = a.scores + (size_t)(r0 + ri) * a.scores_row + (size_t)(g * G + hi) * a.max_ctx;
        const float4* qv = reinterpret_cast<const float4*>(sq + qi * HD);
        const float4* kv = reinterpret_cast<const float4*>(kt + lane * kp);
        if constexpr (Q8) sg[t] = (dot_parity_v4<HD, kIsaScalar>(qv, kv) * a.k_scale[t]) * a.scale;
        else sg[t] = (F16 ? dot_parity_v4<HD, kIsaScalar>(qv, kv) : dot_v4_isa<HD>(qv, kv, a.isa)) * a.scale;
    }
}

// Softmax of one (row, head) per wave, in place in the scores buffer:
// head_softmax's values (max, fast_exp_scalar(x - max), the sum in key order,
// x *= 1/sum).  The exponentials of each 1024-key chunk are also staged in the
// wave's LDS, where lane 0 adds them in order (a dependent chain of adds from
// LDS instead of from memory); four softmaxes per workgroup.
static constexpr int kSoftmaxChunk = 1024;

__global__ __launch_bounds__(kThreads) void attention_softmax_rows(AttnArgs a, int rows) {
    __shared__ __align__(16) float buf[4][kSoftmaxChunk];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int i = (int)blockIdx.x * 4 + wave;
    if (i >= rows * a.n_head) return;
    const int r = i / a.n_head, h = i - r * a.n_head;
    const int n = a.pos_host + r + 1;
    float* sg = a.scores + (size_t)r * a.scores_row + (size_t)h * a.max_ctx;
    float m = -INFINITY;
    for (int t = lane; t < n; t += 64) m = fmaxf(m, sg[t]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float* b = buf[wave];
    float sum = 0.0f;  // lane 0's running sum
    for (int c0 = 0; c0 < n; c0 += kSoftmaxChunk) {
        const int len = min(kSoftmaxChunk, n - c0);
        for (int t = lane; t < len; t += 64) {
            const float e = fast_exp_scalar(sg[c0 + t] - m);
            sg[c0 + t] = e;
            b[t] = e;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) sum = ordered_sum_contig(b, len, sum);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    sum = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sum)));
    if (sum != 0.0f) {
        const float inv = 1.0f / sum;
        for (int t = lane; t < n; t += 64) sg[t] = sg[t] * inv;
    }
}

// The V sum, transposed cache: workgroup (kv head g, block b of kPvRowsQ
// queries); wave w holds columns 64*(w % CW) .. +63 of the head (CW = HD / 64
// column waves) and sums queries qp, qp + QW, ... (qp = w / CW, QW = 4 / CW),
// lane = column.  Per 64-key chunk a lane loads its column's keys once
// (widened to fp32) and applies them to each of its queries in key order,
// acc + p*v (q8_0: acc + (p*q)*s); the block's probabilities (and the keys'
// q8_0 scales) of the chunk are staged in LDS by the whole workgroup and read
// as broadcasts: the ordered sum of VColumn::sum for every (query, column).
static constexpr int kPvRowsQ = 16;

template <int HD, int KV>
__global__ __launch_bounds__(kThreads) void attention_pv_rows(AttnArgs a, int rows) {
    constexpr bool F16 = KV == kKvF16, Q8 = KV == kKvQ8;
    constexpr int CW = HD / 64, QW = 4 / CW, NQ = kPvRowsQ / QW;  // queries per wave
    constexpr int kc = 64, PP = kc + 4;                          // keys per chunk, staged pitch
    __shared__ __align__(16) float ps[kPvRowsQ * PP + kc];       // [query][key], then q8_0 scales
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.n_head / a.kv_heads, RB = kPvRowsQ / G;
    const int g = blockIdx.x;
    const int r0 = (int)blockIdx.y * RB;
    const int rn = min(RB, rows - r0);
    if (rn <= 0) return;
    const int pos0 = a.pos_host + r0;
    const int col = (wave % CW) * 64 + lane, qp = wave / CW;
    const size_t cidx = (size_t)(g * HD + col) * a.vt_stride;
    const float* vcol = a.cache_v + cidx;
    const uint16_t* vcol16 = reinterpret_cast<const uint16_t*>(a.cache_v) + cidx;
    const int8_t* vcol8 = reinterpret_cast<const int8_t*>(a.cache_v) + cidx;
    float acc[NQ];
#pragma unroll
    for (int j = 0; j < NQ; j++) acc[j] = 0.0f;
    const int last = pos0 + rn - 1;  // the block's last position
    const int nq = rn * G;
    for (int t0 = 0; t0 <= last; t0 += kc) {
        __syncthreads();  // the previous chunk's probabilities are read
        // stage: query qi's probabilities t0 .. t0+63 (up to its own position)
        for (int i = tid; i < nq * (kc / 4); i += kThreads) {
            const int qi = i / (kc / 4), k4 = i - qi * (kc / 4);
            const int ri = qi / G, hi = qi - ri * G;
            const int lim = pos0 + ri - t0;  // last key of this query in the chunk
            if (4 * k4 > lim) continue;
            const float* src = a.scores + (size_t)(r0 + ri) * a.scores_row + (size_t)(g * G + hi) * a.max_ctx + t0;
            f32x4 v4;
            v4.x = src[4 * k4];
            v4.y = 4 * k4 + 1 <= lim ? src[4 * k4 + 1] : 0.0f;
            v4.z = 4 * k4 + 2 <= lim ? src[4 * k4 + 2] : 0.0f;
            v4.w = 4 * k4 + 3 <= lim ? src[4 * k4 + 3] : 0.0f;
            *reinterpret_cast<f32x4*>(ps + qi * PP + 4 * k4) = v4;
        }
        if constexpr (Q8)
            if (tid < kc) ps[kPvRowsQ * PP + tid] = a.v_scale[min(t0 + tid, last)];
        float v[kc];
        // keys past `last` are read at the last whole group (never added)
        if constexpr (Q8) {
#pragma unroll
            for (int j = 0; j < kc / 16; j++) {
                const int tk = min(t0 + 16 * j, last & ~15);
                const u32x4 b = *reinterpret_cast<const u32x4*>(vcol8 + tk);
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    v[16 * j + 4 * w] = q8_byte_sdwa<0>(b[w]);
                    v[16 * j + 4 * w + 1] = q8_byte_sdwa<1>(b[w]);
                    v[16 * j + 4 * w + 2] = q8_byte_sdwa<2>(b[w]);
                    v[16 * j + 4 * w + 3] = q8_byte_sdwa<3>(b[w]);
                }
            }
        } else if constexpr (F16) {
#pragma unroll
            for (int j = 0; j < kc / 4; j++) {
                const u32x2 h = *reinterpret_cast<const u32x2*>(vcol16 + min(t0 + 4 * j, last & ~3));
                v[4 * j] = f16_cache_load((uint16_t)(h.x & 0xFFFFu));
                v[4 * j + 1] = f16_cache_load((uint16_t)(h.x >> 16));
                v[4 * j + 2] = f16_cache_load((uint16_t)(h.y & 0xFFFFu));
                v[4 * j + 3] = f16_cache_load((uint16_t)(h.y >> 16));
            }
        } else {
#pragma unroll
            for (int j = 0; j < kc / 4; j++) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(vcol + min(t0 + 4 * j, last & ~3));
                v[4 * j] = x.x;
                v[4 * j + 1] = x.y;
                v[4 * j + 2] = x.z;
                v[4 * j + 3] = x.w;
            }
        }
        __syncthreads();
        const float* sc = ps + kPvRowsQ * PP;
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const int qi = qp + QW * j;
            const int ri = qi / G;
            const int pos = pos0 + ri;
            if (ri >= rn || t0 > pos) continue;  // wave-uniform
            const float* pq = ps + qi * PP;
            float s = acc[j];
            auto term = [&](int k, float pk) { return Q8 ? (pk * v[k]) * sc[k] : pk * v[k]; };
            if (t0 + kc - 1 <= pos) {
#pragma unroll
                for (int k4 = 0; k4 < kc / 4; k4++) {
                    const f32x4 p4 = *reinterpret_cast<const f32x4*>(pq + 4 * k4);
                    s = s + term(4 * k4, p4.x);
                    s = s + term(4 * k4 + 1, p4.y);
                    s = s + term(4 * k4 + 2, p4.z);
                    s = s + term(4 * k4 + 3, p4.w);
                }
            } else {
#pragma unroll
                for (int k4 = 0; k4 < kc / 4; k4++) {
                    const f32x4 p4 = *reinterpret_cast<const f32x4*>(pq + 4 * k4);
                    const float pk[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        if (t0 + 4 * k4 + c <= pos) s = s + term(4 * k4 + c, pk[c]);
                }
            }
            acc[j] = s;
        }
    }
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        const int qi = qp + QW * j;
        const int ri = qi / G, hi = qi - ri * G;
        const bool live = ri < rn;
        AttnArgs o = a;  // the row's output pointers
        const size_t r = (size_t)(r0 + (live ? ri : 0));
        o.out = a.out + r * a.out_row;
        if (a.q_out) {
            o.q_out = a.q_out + r * a.out_row;
            o.q_scale = a.q_scale + r * (a.out_row / 32);
        }
        store_attn_out(o, (g * G + hi) * HD + col, acc[j], live);
    }
}

static hipError_t launch_rows_batched(const AttnArgs& a, int rows, hipStream_t stream) {
    const int G = a.n_head / a.kv_heads, RB = kRowsQ / G;
    const int nblk = (rows + RB - 1) / RB;
    const int RBv = kPvRowsQ / G, nblk_v = (rows + RBv - 1) / RBv;
    const int last = a.pos_host + rows - 1;
    const int nchunks = last / kAttnKeys + 1;
    const bool hd128 = a.head_dim == 128;
    void (*const sc[2][3])(AttnArgs, int) = {
        {attention_scores_rows<64, kKvF32>, attention_scores_rows<64, kKvF16>, attention_scores_rows<64, kKvQ8>},
        {attention_scores_rows<128, kKvF32>, attention_scores_rows<128, kKvF16>, attention_scores_rows<128, kKvQ8>}};
    void (*const pv[2][3])(AttnArgs, int) = {
        {attention_pv_rows<64, kKvF32>, attention_pv_rows<64, kKvF16>, attention_pv_rows<64, kKvQ8>},
        {attention_pv_rows<128, kKvF32>, attention_pv_rows<128, kKvF16>, attention_pv_rows<128, kKvQ8>}};
    const size_t smem = sizeof(float) * ((size_t)kAttnKeys * (a.head_dim + 4) + (size_t)kRowsQ * a.head_dim);
    hipLaunchKernelGGL(sc[hd128][a.k_type], dim3(a.kv_heads, nchunks, nblk), dim3(kThreads), smem, stream, a, rows);
    hipLaunchKernelGGL(attention_softmax_rows, dim3((rows * a.n_head + 3) / 4), dim3(kThreads), 0, stream, a, rows);
    hipLaunchKernelGGL(pv[hd128][a.v_type], dim3(a.kv_heads, nblk_v), dim3(kThreads), 0, stream, a, rows);
    return hipGetLastError();
}

hipError_t launch_attention_rows(const AttnArgs& a, int rows, hipStream_t stream) {
    if (rows < 1 || a.fused || a.pos_dev || a.pos_host < 0 || a.pos_host + rows > a.max_ctx ||
        (a.head_dim != 64 && a.head_dim != 128) || !a.scores || a.max_ctx > kSplitMaxCtx ||
        (rows > 1 && (a.q_row < a.n_head * a.head_dim || a.out_row < a.n_head * a.head_dim ||
                      a.scores_row < (size_t)a.n_head * a.max_ctx || (a.q_out && (a.out_row & 31)))))
        return hipErrorInvalidValue;
    const int mode = attention_path();
    if (mode != kAttnPathSplit && mode != kAttnPathFused) return hipErrorInvalidValue;
    if (!a.q || !a.cache_k || !a.cache_v || !a.out || a.n_head <= 0 || a.kv_heads <= 0 || (a.kv_stride & 3) ||
        (a.head_stride & 3) || (((uintptr_t)a.cache_k | (uintptr_t)a.cache_v) & 15) ||
        (a.q_out && !a.q_scale) || (a.rope_cos && !a.rope_sin))
        return hipErrorInvalidValue;
    if (a.k_type < kKvF32 || a.k_type > kKvQ8 || a.v_type < kKvF32 || a.v_type > kKvQ8) return hipErrorInvalidValue;
    if ((a.k_type == kKvQ8 && !a.k_scale) || (a.v_type == kKvQ8 && !a.v_scale)) return hipErrorInvalidValue;
    if (a.vt_stride > 0 && ((a.vt_stride & 3) || a.vt_stride < (a.max_ctx + 3) / 4 * 4)) return hipErrorInvalidValue;
    if (a.vt_stride > 0 && a.v_type == kKvQ8 && ((a.vt_stride & 15) || a.vt_stride < (a.max_ctx + 15) / 16 * 16))
        return hipErrorInvalidValue;
    if ((a.k_type == kKvQ8 || (a.v_type == kKvQ8 && a.vt_stride == 0)) && ((a.kv_stride & 15) || (a.head_stride & 15)))
        return hipErrorInvalidValue;
    // the batched form: transposed V, whole kv groups in a block of kRowsQ queries
    const int G = a.kv_heads > 0 ? a.n_head / a.kv_heads : 0;
    const bool batched = a.vt_stride > 0 && G > 0 && a.n_head == G * a.kv_heads && kRowsQ % G == 0 && kPvRowsQ % G == 0 &&
                         a.key_base == 0 && a.key_ring == 0;
    if (batched && !getenv("MANTLE_HIP_ROWS_PER_QUERY")) return launch_rows_batched(a, rows, stream);
    return launch_split_two(a, rows, stream);
}

// storeQ8's element (ops_runtime.go:158-168): q = int32(v*inv + 0.5), or
// int32(v*inv - 0.5) for v < 0, clamped to +-127.  Go's float32 -> int32 on
// amd64 (CVTTSS2SL) gives INT32_MIN for NaN and out-of-range values, which the
// clamp then takes to -127; the GPU conversion saturates, so that case is
// made explicit (it arises when 127 / maxAbs overflows to +Inf).
__device__ __forceinline__ int8_t q8_store_value(float v, float inv) {
    const float t = v * inv;
    const float r = v < 0.0f ? t - 0.5f : t + 0.5f;
    int q = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT32_MIN;
    q = q > 127 ? 127 : (q < -127 ? -127 : q);
    return (int8_t)q;
}

// One workgroup: the step's K and V rows (K prepared first when PREP: the
// per-head RMSNorm and RoPE of the fused attention step, prep_pair), each
// row's max |x| over all kv heads, its scale maxAbs / 127 and the int8 row
// (storeQ8, ops_runtime.go:132-168).  LDS: both rows, 4 wave stagings, 8
// reduction floats.
template <int PREP_HD>
__global__ __launch_bounds__(kThreads) void kv_append_q8_kernel(KvQ8Args a) {
    extern __shared__ __align__(16) float lds[];
    const int n = a.kv_heads * a.head_dim;
    float* sk = lds;
    float* sv = lds + n;
    float* wbuf = sv + n;
    float* red = wbuf + 4 * 128;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos_host) + (int)blockIdx.x;  // row blockIdx.x of `tokens`
    if (blockIdx.x > 0) {
        a.k += (size_t)blockIdx.x * a.tok_stride;
        a.v += (size_t)blockIdx.x * a.tok_stride;
    }
    if constexpr (PREP_HD > 0) {
        constexpr int HD = PREP_HD, half = HD / 2;
        const int li = lane < half ? lane : 0;
        const bool norm = a.k_norm != nullptr, rope = a.rope_cos != nullptr;
        for (int g = wave; g < a.kv_heads; g += kThreads / 64) {
            float x0 = a.k[g * HD + li], x1 = a.k[g * HD + li + half];
            const float g0 = norm ? a.k_norm[li] : 0.0f, g1 = norm ? a.k_norm[li + half] : 0.0f;
            const float cs = rope ? a.rope_cos[(size_t)pos * half + li] : 0.0f;
            const float sn = rope ? a.rope_sin[(size_t)pos * half + li] : 0.0f;
            prep_pair<HD>(x0, x1, g0, g1, cs, sn, norm, rope, a.eps, a.isa, wbuf + wave * 128);
            if (lane < half) {
                sk[g * HD + lane] = x0;
                sk[g * HD + lane + half] = x1;
            }
        }
    } else {
        for (int i = tid; i < n; i += kThreads) sk[i] = a.k[i];
    }
    for (int i = tid; i < n; i += kThreads) sv[i] = a.v[i];
    __syncthreads();
    float mk = 0.0f, mv = 0.0f;
    for (int i = tid; i < n; i += kThreads) {
        mk = fmaxf(mk, fabsf(sk[i]));
        mv = fmaxf(mv, fabsf(sv[i]));
    }
    for (int off = 32; off > 0; off >>= 1) {
        mk = fmaxf(mk, __shfl_down(mk, off, 64));
        mv = fmaxf(mv, __shfl_down(mv, off, 64));
    }
    if (lane == 0) {
        red[wave] = mk;
        red[4 + wave] = mv;
    }
    __syncthreads();
    const float max_k = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float max_v = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
    // a zero row: scale 0 and zeros (ops_runtime.go:147-153)
    const float inv_k = max_k == 0.0f ? 0.0f : 127.0f / max_k;
    const float inv_v = max_v == 0.0f ? 0.0f : 127.0f / max_v;
    for (int i = tid; i < n; i += kThreads) {
        const int g = i / a.head_dim, d = i - g * a.head_dim;
        const size_t row = (size_t)g * a.head_stride + (size_t)pos * a.row_stride + d;
        if (!a.skip_k) a.cache_k[row] = max_k == 0.0f ? (int8_t)0 : q8_store_value(sk[i], inv_k);
        if (!a.skip_v) {
            const int8_t qv = max_v == 0.0f ? (int8_t)0 : q8_store_value(sv[i], inv_v);
            if (a.vt_stride > 0) a.cache_v[(size_t)i * a.vt_stride + pos] = qv;
            else a.cache_v[row] = qv;
        }
    }
    if (tid == 0) {
        if (!a.skip_k) a.k_scale[pos] = max_k / 127.0f;
        if (!a.skip_v) a.v_scale[pos] = max_v / 127.0f;
    }
}

hipError_t launch_kv_append_q8(const KvQ8Args& a, hipStream_t stream) {
    if ((a.skip_k && a.skip_v) || !a.k || !a.v || (!a.skip_k && (!a.cache_k || !a.k_scale)) ||
        (!a.skip_v && (!a.cache_v || !a.v_scale)) || a.kv_heads <= 0 || a.head_dim <= 0 ||
        a.kv_heads * a.head_dim > kKvQ8MaxRow || a.head_stride < 0 || a.row_stride < 0 || a.vt_stride < 0)
        return hipErrorInvalidValue;
    if (!a.pos_dev && a.pos_host < 0) return hipErrorInvalidValue;
    if (a.prep && a.head_dim != 64 && a.head_dim != 128) return hipErrorInvalidValue;
    if (a.rope_cos && !a.rope_sin) return hipErrorInvalidValue;
    const int rows = a.tokens > 1 ? a.tokens : 1;
    if (rows > 1 && (a.pos_dev || a.tok_stride < a.kv_heads * a.head_dim)) return hipErrorInvalidValue;
    const size_t smem = sizeof(float) * (2 * (size_t)a.kv_heads * a.head_dim + 4 * 128 + 8);
    auto k = !a.prep ? kv_append_q8_kernel<0> : (a.head_dim == 128 ? kv_append_q8_kernel<128> : kv_append_q8_kernel<64>);
    hipLaunchKernelGGL(k, dim3(rows), dim3(kThreads), smem, stream, a);
    return hipGetLastError();
}

// Rows pos .. pos+rows-1 of a prompt: wave w of workgroup (b, r) prepares
// vector 4b+w of row r -- query heads first, then the kv heads' K, then their
// V -- with the decode prologue's arithmetic (prep_pair; the f16 cache's
// rounding), writing q to qo and the K / V rows to the f32 / f16 caches.
template <int HD>
__global__ __launch_bounds__(kThreads) void attention_prep_rows_kernel(AttnArgs a, int qkv_row, float* qo) {
    __shared__ __align__(16) float wbuf[4 * 128];
    constexpr int half = HD / 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = (int)blockIdx.y;
    const int pos = a.pos_host + r;
    const int vi = (int)blockIdx.x * 4 + wave;
    const int nq = a.n_head, nkv = a.kv_heads;
    if (vi >= nq + 2 * nkv) return;
    const int li = lane < half ? lane : 0;
    const int kind = vi < nq ? 0 : (vi < nq + nkv ? 1 : 2);  // q, k, v
    const int hh = kind == 0 ? vi : (kind == 1 ? vi - nq : vi - nq - nkv);
    const int ctype = kind == 1 ? a.k_type : a.v_type;
    if (kind > 0 && ctype == kKvQ8) return;  // launch_kv_append_q8 writes the q8_0 rows
    const float* src = (kind == 0 ? a.q : (kind == 1 ? a.k : a.v)) + (size_t)r * qkv_row + hh * HD;
    const float* nw = kind == 0 ? a.q_norm : (kind == 1 ? a.k_norm : nullptr);
    const bool norm = nw != nullptr, rope = kind < 2 && a.rope_cos != nullptr;
    float x0 = src[li], x1 = src[li + half];
    const float g0 = norm ? nw[li] : 0.0f, g1 = norm ? nw[li + half] : 0.0f;
    const float cs = rope ? a.rope_cos[(size_t)pos * half + li] : 0.0f;
    const float sn = rope ? a.rope_sin[(size_t)pos * half + li] : 0.0f;
    prep_pair<HD>(x0, x1, g0, g1, cs, sn, norm, rope, a.eps, a.isa, wbuf + wave * 128);
    if (lane >= half) return;
    if (kind == 0) {
        float* dst = qo + (size_t)r * a.out_row + hh * HD;
        dst[lane] = x0;
        dst[lane + half] = x1;
        return;
    }
    if (ctype == kKvF16) {
        uint16_t* c16 = reinterpret_cast<uint16_t*>(kind == 1 ? a.cache_k : a.cache_v);
        const uint16_t h0 = mantle_f32_to_f16_trunc(f16_cache_round(x0));
        const uint16_t h1 = mantle_f32_to_f16_trunc(f16_cache_round(x1));
        if (kind == 2 && a.vt_stride > 0) {
            uint16_t* col = c16 + (size_t)(hh * HD + lane) * a.vt_stride + pos;
            col[0] = h0;
            col[(size_t)half * a.vt_stride] = h1;
        } else {
            uint16_t* row = c16 + (size_t)hh * a.head_stride + (size_t)pos * a.kv_stride;
            row[lane] = h0;
            row[lane + half] = h1;
        }
    } else if (kind == 2 && a.vt_stride > 0) {
        float* col = a.cache_v + (size_t)(hh * HD + lane) * a.vt_stride + pos;
        col[0] = x0;
        col[(size_t)half * a.vt_stride] = x1;
    } else {
        float* row = (kind == 1 ? a.cache_k : a.cache_v) + (size_t)hh * a.head_stride + (size_t)pos * a.kv_stride;
        row[lane] = x0;
        row[lane + half] = x1;
    }
}

hipError_t launch_attention_prep_rows(const AttnArgs& a, int rows, int qkv_row, float* qo, hipStream_t stream) {
    if (rows < 1 || !a.q || !a.k || !a.v || !qo || !a.cache_k || !a.cache_v || a.pos_dev || a.pos_host < 0 ||
        a.pos_host + rows > a.max_ctx || (a.head_dim != 64 && a.head_dim != 128) || a.n_head <= 0 ||
        a.kv_heads <= 0 || a.out_row < a.n_head * a.head_dim || qkv_row <= 0 || (a.rope_cos && !a.rope_sin) ||
        a.key_base || a.key_ring)
        return hipErrorInvalidValue;
    const int nv = a.n_head + 2 * a.kv_heads;
    const dim3 grid((nv + 3) / 4, rows);
    if (a.head_dim == 128)
        hipLaunchKernelGGL(attention_prep_rows_kernel<128>, grid, dim3(kThreads), 0, stream, a, qkv_row, qo);
    else
        hipLaunchKernelGGL(attention_prep_rows_kernel<64>, grid, dim3(kThreads), 0, stream, a, qkv_row, qo);
    return hipGetLastError();
}

#ifdef MANTLE_PHASE_TRACE
MANTLE_PHASE_READER(phase_read_attention)
#endif

}  // namespace mantle
