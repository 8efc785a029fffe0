// gemv.h -- k4 GEMV launch parameters and host-side helpers shared by the
// tile kernel (kernels.hip) and the lane-chain kernel (gemv_lane_*.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "kernels.h"
#include "quant_device.h"

namespace mantle {

struct GemvParams {
    K4Mat mats[3];
    float* outs[3];
    int wg_begin[4];  // first tile of each matrix
    int ntiles;
    int nmat;
    int cols, bpr, spr, rpw, batch;
    const int8_t* qx;
    const float* xs;
    const float* x;       // W4A32 / in-kernel-quantised fp32 input [batch][cols]
    const float* norm_w;  // RMSNorm gains applied before quantisation (nullable)
    float eps;
    int isa;
    unsigned long long* key;
    int8_t* q_out;   // kEpiSiluMul: output also quantised (32-row units) ...
    float* q_scale;  // ... with these block scales
};


// kModeW4A8: activation already quantised (qx/xs); kModeW4A32: fp32 activation
// used as is; kModeW4A8Fused: every workgroup quantises the fp32 activation
// itself (after RMSNorm when norm_w is set) while its weight loads are in flight.
// Selects instead of a dynamic index into the by-value kernel argument: an
// indexed p.mats[k] would make the compiler copy the whole struct to scratch.
__device__ __forceinline__ K4Mat pick_mat(const GemvParams& p, int k) {
    return k == 0 ? p.mats[0] : (k == 1 ? p.mats[1] : p.mats[2]);
}
__device__ __forceinline__ float* pick_out(const GemvParams& p, int k) {
    return k == 0 ? p.outs[0] : (k == 1 ? p.outs[1] : p.outs[2]);
}

enum GemvMode : int { kModeW4A8 = 0, kModeW4A32 = 1, kModeW4A8Fused = 2 };
// Lane-kernel prologue: activation pre-quantised (qx/xs), quantised in the
// kernel, or RMSNorm then quantised in the kernel.
enum LanePro : int { kProQx = 0, kProQuant = 1, kProNorm = 2 };

// 64-bit key whose maximum over (v, idx) pairs is argmaxHost's answer
// (runtime_greedy.go:70-82: best = x[0], then x[i] > best): order-preserving
// value bits, then -idx so the first maximum wins.  Strict '>' also makes -0
// equal to +0 (mapped to +0 here) and never lets a NaN win: a NaN at index 0
// is kept forever (the largest key), any other NaN takes key 0, below every
// number (the smallest numeric key, -inf, is 0x007FFFFF...).
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return idx == 0 ? ~0ull : 0ull;
    if (u == 0x80000000u) u = 0u;
    uint32_t s = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)s << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// Workgroups of kernel `fn` (with `smem` bytes of LDS) that fit on the whole
// device at once; cached per kernel instance and LDS size class.
template <typename K>
static int resident_wgs(K fn, size_t smem) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn), kThreads, smem) !=
            hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    return per_cu * cus;
}

static inline bool lane_gemv_disabled() {
    static bool v = [] {
        const char* e = getenv("MANTLE_HIP_GEMV_TILES");
        return e && atoi(e) != 0;
    }();
    return v;
}

static inline int lane_small_rows() {
    static int v = [] {
        const char* e = getenv("MANTLE_HIP_GEMV_SMALL_ROWS");
        return e ? atoi(e) : 16384;
    }();
    return v;
}

// Matrices of at least this many blocks take the large-matrix launch (one
// unit per multi-wave workgroup) even with few rows: measured on Qwen3-4B's
// 6144 x 2560 QKV, 11.4 -> 7.6 us.
static inline int64_t lane_large_blocks() {
    static int64_t v = [] {
        const char* e = getenv("MANTLE_HIP_GEMV_LARGE_BLOCKS");
        return e ? (int64_t)atoll(e) : (int64_t)262144;
    }();
    return v;
}

static inline int gemv_max_wgs() {
    static int v = [] {
        const char* e = getenv("MANTLE_HIP_GEMV_MAX_WGS");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Lane-chain GEMV entry points, one translation unit each (they compile in
// parallel).  `pro` is a LanePro; *used is false when the lane kernel has no
// instance for the shape and the caller must use the tile kernel.
hipError_t lane_gemv_store(GemvParams& p, int pro, hipStream_t stream, bool* used);              // gemv_lane_store.hip
hipError_t lane_gemv_fused(GemvParams& p, GemvEpi epi, int pro, hipStream_t stream, bool* used); // gemv_lane_fused.hip
hipError_t lane_gemv_batch8(GemvParams& p, int pro, hipStream_t stream, bool* used);             // gemv_lane_b8.hip
// W4A32 with one lane per row (gemv_w4a32.hip); *used false when x does not fit LDS.
hipError_t k4_gemv_w4a32_mfma_launch(const K4Mat& m, int cols, const float* x, float* y, int batch,
                                     hipStream_t stream, bool* used);  // gemm_w4a32.hip
hipError_t k4_gemv_w4a32_lane(const K4Mat& m, int cols, const float* x, float* y, int batch, hipStream_t stream,
                              bool* used);

}  // namespace mantle
