// gemv_w4a32.hip -- the k4 GEMV on fp32 activations (W4A32), batch 1..8.
//
// The arithmetic of the CUDA backend's quant_matvec_k4_f32 kernel behind
// mantleCudaQuantMatVecK4F32 (internal/backend/cuda/native/softmax.cu:411-546,
// :1046-1072) and the CPU's non-AVX2 branch (internal/backend/simd/
// matvec_quant.go:291-293): y[b][r] = sum over blocks of s_w[r,blk] *
// (sum_i q[r,blk,i] * x[b][32 blk + i]) in fp32, checked within max-abs 1e-3 /
// rel 1e-2 (the summation order is free; W4A8 is the bit-exact CPU form).
//
// Eight lanes per row, lane j taking blocks j, j+8, ...: a row's lanes read 128
// contiguous bytes per load, and the lanes of one block index read the same
// LDS words of x (one transaction per distinct address), staged once per
// workgroup for all its row units.  Each lane turns its nibbles into bytes of
// 16 q ((w << 4) & 0xF0F0F0F0 for the even ones, w & 0xF0F0F0F0 for the odd
// ones) and widens each with one SDWA conversion; the 1/16 joins the block
// scale.  Per weight: one conversion and NB FMAs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"
#include "kernels.h"

namespace mantle {

static constexpr int kW32Lanes = 8;               // lanes per row
static constexpr int kW32Rows = 32;               // rows per unit of four-wave workgroups: 4 waves x 8 rows
static constexpr int kW32Group = 4;               // blocks per lane per load group

// Byte C of w, sign-extended, as fp32 (SDWA byte select): one instruction.
template <int C>
__device__ __forceinline__ float sbyte_f32(uint32_t w) {
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

// xs: LDS [NB][cols] fp32.  Workgroups of NW waves; unit u covers rows
// 8NW*R*u onwards, 8NW*R of them: eight lanes per
// row, lane j taking blocks j, j+8, ... so that a row's lanes read 128
// contiguous bytes per load and the lanes of one block index share x words.
template <int NB, int R, int NW>
__global__ __launch_bounds__(256) void k4_gemv_w4a32_rows(K4Mat m, int bpr, const float* __restrict__ x,
                                                          float* __restrict__ y, int units) {
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x;
    const int cols = bpr * 32;
    // stage x once: NB * cols floats (cols is a multiple of 32)
    constexpr int RPU = 8 * NW;  // rows per lane-group slab: NW waves x 8 rows
    for (int i = tid * 4; i < NB * cols; i += NW * 64 * 4)
        *reinterpret_cast<float4*>(xs + i) = *reinterpret_cast<const float4*>(x + i);
    __syncthreads();
    const int spr = (bpr + 7) / 8;
    const int j = tid & (kW32Lanes - 1);
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        // R rows per lane group (rows r0, r0 + 32, ...): each x word read from LDS serves R rows
        const int r0 = u * RPU * R + tid / kW32Lanes;
        const uint4* nib[R];
        const uint8_t* sub[R];
        const uint16_t* sup[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = r0 + r * RPU;
            const int rc = row < m.rows ? row : m.rows - 1;  // rows past the end re-read the last (not stored)
            nib[r] = reinterpret_cast<const uint4*>(m.nib) + (size_t)rc * bpr;
            sub[r] = m.sub + (size_t)rc * bpr;
            sup[r] = m.sup + (size_t)rc * spr;
        }
        float acc[R][NB];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[r][b] = 0.0f;
        for (int g0 = 0; g0 < bpr; g0 += kW32Lanes * kW32Group) {
            uint4 w[R][kW32Group];
            float sc[R][kW32Group];
#pragma unroll
            for (int k = 0; k < kW32Group; k++) {
                int blk = g0 + k * kW32Lanes + j;
                blk = blk < bpr ? blk : bpr - 1;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    w[r][k] = nib[r][blk];
                    sc[r][k] = k4_scale(sup[r][blk >> 3], sub[r][blk]) * 0.0625f;  // the nibble bytes hold 16 q
                }
            }
#pragma unroll
            for (int k = 0; k < kW32Group; k++) {
                const int blk = g0 + k * kW32Lanes + j;
                const float* xb = xs + (blk < bpr ? blk : bpr - 1) * 32;
                float bs[R][NB];
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int b = 0; b < NB; b++) bs[r][b] = 0.0f;
#pragma unroll
                for (int d = 0; d < 4; d++) {  // word d: elements 8d .. 8d+7
                    float q[R][8];
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const uint32_t wd = d == 0 ? w[r][k].x : (d == 1 ? w[r][k].y : (d == 2 ? w[r][k].z : w[r][k].w));
                        const uint32_t e = (wd << 4) & 0xF0F0F0F0u, o = wd & 0xF0F0F0F0u;
                        q[r][0] = sbyte_f32<0>(e); q[r][1] = sbyte_f32<0>(o);
                        q[r][2] = sbyte_f32<1>(e); q[r][3] = sbyte_f32<1>(o);
                        q[r][4] = sbyte_f32<2>(e); q[r][5] = sbyte_f32<2>(o);
                        q[r][6] = sbyte_f32<3>(e); q[r][7] = sbyte_f32<3>(o);
                    }
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const float4 xa = *reinterpret_cast<const float4*>(xb + b * cols + 8 * d);
                        const float4 xc = *reinterpret_cast<const float4*>(xb + b * cols + 8 * d + 4);
#pragma unroll
                        for (int r = 0; r < R; r++) {
                            float s = bs[r][b];
                            s = __builtin_fmaf(q[r][0], xa.x, s);
                            s = __builtin_fmaf(q[r][1], xa.y, s);
                            s = __builtin_fmaf(q[r][2], xa.z, s);
                            s = __builtin_fmaf(q[r][3], xa.w, s);
                            s = __builtin_fmaf(q[r][4], xc.x, s);
                            s = __builtin_fmaf(q[r][5], xc.y, s);
                            s = __builtin_fmaf(q[r][6], xc.z, s);
                            s = __builtin_fmaf(q[r][7], xc.w, s);
                            bs[r][b] = s;
                        }
                    }
                }
                const bool live = blk < bpr;  // a re-read block adds nothing
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[r][b] = __builtin_fmaf(live ? sc[r][k] : 0.0f, bs[r][b], acc[r][b]);
            }
        }
        // each row's eight partial sums (any order: tolerance-checked arithmetic)
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float v = acc[r][b];
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                v += __shfl_xor(v, 4, 64);
                acc[r][b] = v;
            }
            const int row = r0 + r * RPU;
            if (j == 0 && row < m.rows) {
#pragma unroll
                for (int b = 0; b < NB; b++) y[(size_t)b * m.rows + row] = acc[r][b];
            }
        }
    }
}

template <int NB, int R, int NW = 4>
static hipError_t launch_rows_r(const K4Mat& m, int bpr, const float* x, float* y, hipStream_t stream) {
    auto kern = k4_gemv_w4a32_rows<NB, R, NW>;
    const size_t smem = sizeof(float) * (size_t)NB * bpr * 32;
    static bool lds_ok = false;
    if (smem > 64 * 1024 && !lds_ok) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return hipErrorInvalidValue;
        lds_ok = true;
    }
    const int units = (m.rows + 8 * NW * R - 1) / (8 * NW * R);
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // a few resident workgroups per CU, each staging x once for several units
    const int cap = 32 / NW * cus;
    const int grid = units < cap ? units : cap;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), smem, stream, m, bpr, x, y, units);
    return hipGetLastError();
}

// Wider batches hold two rows per lane group so that each x word read from LDS
// serves both.  So does batch 1-2 on matrices of more than eight workgroups
// per CU (the logits: 151936x1024 at batch 1 27.1 -> 25.5 us); smaller ones
// keep one row, which spreads their few rows over more waves (3072x1024 at
// batch 1: 4.8 us with one row, 8.7 with two).
template <int NB>
static hipError_t launch_rows(const K4Mat& m, int bpr, const float* x, float* y, hipStream_t stream) {
    if constexpr (NB >= 3) {
        return launch_rows_r<NB, 2>(m, bpr, x, y, stream);
    } else {
        int cus = 256, dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if ((m.rows + kW32Rows - 1) / kW32Rows >= 8 * cus) return launch_rows_r<NB, 2>(m, bpr, x, y, stream);
        // wide rows with fewer 32-row units than CUs (1024x3072): one-wave
        // workgroups of 8 rows spread them over four times as many CUs
        // (10.3 -> 9.3 us; the 1024-column shapes measured no faster)
        if (bpr >= 64 && (m.rows + kW32Rows - 1) / kW32Rows < cus) return launch_rows_r<NB, 1, 1>(m, bpr, x, y, stream);
        return launch_rows_r<NB, 1>(m, bpr, x, y, stream);
    }
}

// Whole rows of 32-weight blocks with x staged in at most 160 KiB of LDS;
// *used false otherwise (the caller takes the tile kernel).
hipError_t k4_gemv_w4a32_lane(const K4Mat& m, int cols, const float* x, float* y, int batch, hipStream_t stream,
                              bool* used) {
    *used = false;
    const int bpr = (cols + 31) / 32;
    if (cols != bpr * 32 || (size_t)batch * cols * sizeof(float) > 160 * 1024 || ((uintptr_t)x & 15)) return hipSuccess;
    *used = true;
    switch (batch) {
        case 1: return launch_rows<1>(m, bpr, x, y, stream);
        case 2: return launch_rows<2>(m, bpr, x, y, stream);
        case 3: return launch_rows<3>(m, bpr, x, y, stream);
        case 4: return launch_rows<4>(m, bpr, x, y, stream);
        case 5: return launch_rows<5>(m, bpr, x, y, stream);
        case 6: return launch_rows<6>(m, bpr, x, y, stream);
        case 7: return launch_rows<7>(m, bpr, x, y, stream);
        case 8: return launch_rows<8>(m, bpr, x, y, stream);
        default: *used = false; return hipSuccess;
    }
}

}  // namespace mantle
