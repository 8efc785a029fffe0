// gemv_bf16.hip -- dense bf16 GEMV with fp32 activations for raw-bf16 MCF
// weights (internal/backend/simd/matvec.go:406-979, matVecRangeBF16), bit-exact
// to each of Mantle's three CPU reduction orders.
//
// HBM-bound: 2 bytes per weight, nothing to reuse at batch 1.  The order the
// CPU fixes decides the lane layout, because a chain of dependent fp32 adds
// cannot be split across lanes:
//  * AVX-512 (matvec.go:738-834): 32 running sums per row (16 lanes x two
//    accumulators, element j feeds sum j mod 32).  Four lanes per row; lane q
//    owns sums 8q .. 8q+7 and loads the 8 bf16 of each 32-element step in one
//    16-byte load.  Sums 16+l join sum l across the quad, then the 16 are added
//    in order.
//  * AVX2 (matvec.go:513-610) and scalar (matvec.go:419-445): 8 running sums /
//    8-term groups per row, so one lane per row streams the whole row 16 bytes
//    at a time.
// x is staged once per workgroup in LDS.  Up to three matrices (Q, K, V) share
// one launch and one x.
#include <hip/hip_runtime.h>

#include "gemv.h"
#include "kernels.h"

namespace mantle {

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct Bf16Params {
    const uint16_t* w[3];
    float* y[3];
    int rows[3];
    int row_begin[4];  // first global row of each matrix
    int nmat, cols;
    const float* x;
    unsigned long long* key;  // kEpiArgmax: kArgmaxSlots keys
};

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

__device__ __forceinline__ void unpack8(const u32x4_t& v, float (&f)[8]) {
    f[0] = bf_lo(v.x); f[1] = bf_hi(v.x); f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
    f[4] = bf_lo(v.z); f[5] = bf_hi(v.z); f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

__device__ __forceinline__ float bf_at(const uint16_t* row, int j) { return __uint_as_float((uint32_t)row[j] << 16); }

// The matrix and local row of global row g (selects, not an indexed struct access).
__device__ __forceinline__ int mat_of(const Bf16Params& p, int g) {
    return (p.nmat > 1 && g >= p.row_begin[1]) + (p.nmat > 2 && g >= p.row_begin[2]);
}

template <int EPI>
__device__ __forceinline__ void bf16_epilogue(const Bf16Params& p, int g, float sum, unsigned long long& best) {
    const int k = mat_of(p, g);
    const int r = g - (k == 0 ? 0 : (k == 1 ? p.row_begin[1] : p.row_begin[2]));
    float* y = k == 0 ? p.y[0] : (k == 1 ? p.y[1] : p.y[2]);
    if (EPI == kEpiResAdd) {
        y[r] = y[r] + sum;  // runtime.go:278-289 addResidual after the GEMV
    } else {
        y[r] = sum;
        if (EPI == kEpiArgmax) {
            const unsigned long long kk = argmax_key(sum, r);
            best = kk > best ? kk : best;
        }
    }
}

template <int NW>
__device__ __forceinline__ void argmax_flush(const Bf16Params& p, unsigned long long best) {
    __shared__ unsigned long long red[NW];
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_down(best, off, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = red[0];
        for (int i = 1; i < NW; i++) m = red[i] > m ? red[i] : m;
        atomicMax(p.key + (blockIdx.x % kArgmaxSlots) * kArgmaxStride, m);
    }
}

// x -> LDS, issued in batches of 16 float4 per lane, every load of a batch
// before its first store (x is 16-byte aligned, cols a multiple of 8).
__device__ __forceinline__ void stage_x(const Bf16Params& p, float* sx, int nt) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4* x4 = reinterpret_cast<const f4*>(p.x);
    f4* s4 = reinterpret_cast<f4*>(sx);
    const int n4 = p.cols / 4;
    for (int i0 = 0; i0 < n4; i0 += 16 * nt) {
        f4 v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int i = i0 + u * nt + (int)threadIdx.x;
            v[u] = x4[i < n4 ? i : 0];
        }
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int i = i0 + u * nt + (int)threadIdx.x;
            if (i < n4) s4[i] = v[u];
        }
    }
    __syncthreads();
}

// AVX-512 order, four lanes per row, 16 rows per wave.  Weight loads run U
// steps (of 32 elements) ahead of their FMAs, double-buffered; the first U are
// issued before x is staged, so x's latency hides behind theirs.
constexpr int kAvx512Unroll = 16;

template <int EPI, int NW>
__global__ __launch_bounds__(NW * 64) void bf16_gemv_avx512(Bf16Params p) {
    extern __shared__ __align__(16) float sx[];
    constexpr int U = kAvx512Unroll;
    const int lane = threadIdx.x & 63, q = lane & 3;
    const int total = p.row_begin[p.nmat];
    const int g = (blockIdx.x * NW + (threadIdx.x >> 6)) * 16 + (lane >> 2);
    const bool live = g < total;
    const int gc = live ? g : total - 1;  // rows past the end re-read the last row, never stored
    const int k = mat_of(p, gc);
    const uint16_t* wbase = k == 0 ? p.w[0] : (k == 1 ? p.w[1] : p.w[2]);
    const int r = gc - (k == 0 ? 0 : (k == 1 ? p.row_begin[1] : p.row_begin[2]));
    const uint16_t* row = wbase + (size_t)r * p.cols;
    const u32x4_t* rv = reinterpret_cast<const u32x4_t*>(row) + q;  // step s: rv[4 s]
    const int c = p.cols;
    const int steps = c / 32;
    const int last = steps > 0 ? steps - 1 : 0;
    auto load = [&](u32x4_t (&v)[U], int s0) {
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(rv + 4 * (s0 + u <= last ? s0 + u : last));
    };
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    auto fmas = [&](const u32x4_t (&v)[U], int s0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (s0 + u < steps) {
                float wf[8];
                unpack8(v[u], wf);
                const float* xs = sx + 32 * (s0 + u) + 8 * q;
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = __builtin_fmaf(wf[e], xs[e], acc[e]);
            }
        }
    };
    // two buffers in alternation (a register copy would wait for its load)
    u32x4_t va[U], vb[U];
    load(va, 0);
    __builtin_amdgcn_sched_barrier(0);
    stage_x(p, sx, NW * 64);
    for (int s = 0; s < steps; s += 2 * U) {
        load(vb, s + U);  // clamped: past the row's end they re-read its last step
        __builtin_amdgcn_sched_barrier(0);
        fmas(va, s);
        if (s + U >= steps) break;
        load(va, s + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        fmas(vb, s + U);
    }
    int j = steps * 32;
    if (c - j >= 16) {  // a remaining 16-element chunk feeds sums 0..15 (lanes 0, 1)
        if (q < 2) {
            float wf[8];
            unpack8(*reinterpret_cast<const u32x4_t*>(row + j + 8 * q), wf);
            const float* xs = sx + j + 8 * q;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = __builtin_fmaf(wf[e], xs[e], acc[e]);
        }
        j += 16;
    }
    // acc.Add(acc_2): lanes 0, 1 take the sums of lanes 2, 3
    float cmb[8];
#pragma unroll
    for (int e = 0; e < 8; e++) cmb[e] = acc[e] + __shfl_xor(acc[e], 2, 64);
    float hi[8];
#pragma unroll
    for (int e = 0; e < 8; e++) hi[e] = __shfl_xor(cmb[e], 1, 64);
    unsigned long long best = 0;
    if (q == 0) {
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) sum += cmb[e];
#pragma unroll
        for (int e = 0; e < 8; e++) sum += hi[e];
        for (; j < c; j++) sum += bf_at(row, j) * sx[j];
        if (live) bf16_epilogue<EPI>(p, g, sum, best);
    }
    if (EPI == kEpiArgmax) argmax_flush<NW>(p, best);
}

// AVX2 (ISA 1) or scalar (ISA 0) order, one lane per row, loads 8 steps (of 8
// elements) ahead.
template <int ISA, int EPI, int NW>
__global__ __launch_bounds__(NW * 64) void bf16_gemv_lane_row(Bf16Params p) {
    extern __shared__ __align__(16) float sx[];
    constexpr int U = 8;
    const int total = p.row_begin[p.nmat];
    const int g = blockIdx.x * NW * 64 + threadIdx.x;
    const bool live = g < total;
    const int gc = live ? g : total - 1;
    const int k = mat_of(p, gc);
    const uint16_t* wbase = k == 0 ? p.w[0] : (k == 1 ? p.w[1] : p.w[2]);
    const int r = gc - (k == 0 ? 0 : (k == 1 ? p.row_begin[1] : p.row_begin[2]));
    const uint16_t* row = wbase + (size_t)r * p.cols;
    const u32x4_t* rv = reinterpret_cast<const u32x4_t*>(row);
    const int c = p.cols;
    const int steps = c / 8;
    const int last = steps > 0 ? steps - 1 : 0;
    auto load = [&](u32x4_t (&v)[U], int s0) {
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(rv + (s0 + u <= last ? s0 + u : last));
    };
    float sum = 0.0f;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    auto step8 = [&](const u32x4_t (&v)[U], int s0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (s0 + u < steps) {
                float wf[8];
                unpack8(v[u], wf);
                const float* xs = sx + 8 * (s0 + u);
                if (ISA == kIsaAvx2) {
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[e] = __builtin_fmaf(wf[e], xs[e], acc[e]);
                } else {  // sum += p0 + p1 + ... + p7 (products rounded, no FMA)
                    float gsum = wf[0] * xs[0];
#pragma unroll
                    for (int e = 1; e < 8; e++) gsum += wf[e] * xs[e];
                    sum += gsum;
                }
            }
        }
    };
    u32x4_t va[U], vb[U];
    load(va, 0);
    __builtin_amdgcn_sched_barrier(0);
    stage_x(p, sx, NW * 64);
    for (int s = 0; s < steps; s += 2 * U) {
        load(vb, s + U);
        __builtin_amdgcn_sched_barrier(0);
        step8(va, s);
        if (s + U >= steps) break;
        load(va, s + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        step8(vb, s + U);
    }
    if (ISA == kIsaAvx2) {
        float h = acc[0];
#pragma unroll
        for (int e = 1; e < 8; e++) h += acc[e];
        sum += h;
    }
    for (int j = steps * 8; j < c; j++) sum += bf_at(row, j) * sx[j];
    unsigned long long best = 0;
    if (live) bf16_epilogue<EPI>(p, g, sum, best);
    if (EPI == kEpiArgmax) argmax_flush<NW>(p, best);
}

template <int EPI>
hipError_t launch_bf16_epi(Bf16Params& p, int isa, hipStream_t stream) {
    const size_t smem = sizeof(float) * (size_t)p.cols;
    const int total = p.row_begin[p.nmat];
    if (isa == kIsaAvx512) {
        // one-wave workgroups of 16 rows: thousands of workgroups for every
        // Qwen3 matrix, spread over all CUs
        const int grid = (total + 15) / 16;
        hipLaunchKernelGGL((bf16_gemv_avx512<EPI, 1>), dim3(grid), dim3(64), smem, stream, p);
    } else {
        const int grid = (total + 63) / 64;
        if (isa == kIsaAvx2)
            hipLaunchKernelGGL((bf16_gemv_lane_row<kIsaAvx2, EPI, 1>), dim3(grid), dim3(64), smem, stream, p);
        else
            hipLaunchKernelGGL((bf16_gemv_lane_row<kIsaScalar, EPI, 1>), dim3(grid), dim3(64), smem, stream, p);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16_gemv(const uint16_t* const* w, float* const* y, const int* rows, int nmat, int cols,
                            const float* x, GemvEpi epi, unsigned long long* argmax_key, int isa,
                            hipStream_t stream) {
    if (!w || !y || !rows || nmat < 1 || nmat > 3 || cols <= 0 || !x || ((uintptr_t)x & 15))
        return hipErrorInvalidValue;
    if (cols % 8 || cols > kBf16MaxCols) return hipErrorInvalidValue;  // 16-byte row loads; x fits LDS
    if (epi != kEpiStore && epi != kEpiResAdd && epi != kEpiArgmax) return hipErrorInvalidValue;
    if (epi == kEpiArgmax && (!argmax_key || nmat != 1)) return hipErrorInvalidValue;
    if (isa != kIsaAvx512 && isa != kIsaAvx2 && isa != kIsaScalar) return hipErrorInvalidValue;
    Bf16Params p = {};
    p.nmat = nmat;
    p.cols = cols;
    p.x = x;
    p.key = argmax_key;
    int total = 0;
    for (int i = 0; i < nmat; i++) {
        if (!w[i] || !y[i] || rows[i] <= 0 || ((uintptr_t)w[i] & 15)) return hipErrorInvalidValue;
        if ((size_t)rows[i] * (size_t)cols > (size_t)1 << 31) return hipErrorInvalidValue;  // 32-bit row offsets
        p.w[i] = w[i];
        p.y[i] = y[i];
        p.rows[i] = rows[i];
        p.row_begin[i] = total;
        total += rows[i];
    }
    p.row_begin[nmat] = total;
    for (int i = nmat + 1; i < 4; i++) p.row_begin[i] = total;
    switch (epi) {
        case kEpiStore: return launch_bf16_epi<kEpiStore>(p, isa, stream);
        case kEpiResAdd: return launch_bf16_epi<kEpiResAdd>(p, isa, stream);
        default: return launch_bf16_epi<kEpiArgmax>(p, isa, stream);
    }
}

}  // namespace mantle
