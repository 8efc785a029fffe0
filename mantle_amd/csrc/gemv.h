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
    L2Prefetch pf;   // the next GEMV's weights (pf.nmat == 0: none)
};

// Issue this workgroup's share of the prefetch (at most PF loads per thread,
// results in v, to be consumed at the kernel's end so the loads stay in
// flight meanwhile).  The workgroups of XCD class c = b mod 8 fetch the
// lines of the consumer units that run on workgroups of the same class.
template <int PF, int NT>
__device__ __forceinline__ void l2_prefetch_issue(const L2Prefetch& pf, uint32_t (&v)[PF]) {
#pragma unroll
    for (int s = 0; s < PF; s++) v[s] = 0;
    if (pf.nmat == 0) return;
    const int b = (int)blockIdx.x, G = (int)gridDim.x, c = b & 7;
    if (c >= pf.grid) return;
    const int nc = (G - c + 7) >> 3, k = b >> 3;
    const int nwc = (pf.grid - c + 7) >> 3;  // consumer workgroups of class c
    const float inv_nwc = 1.0f / (float)nwc;
    const int total = nwc * pf.per * pf.nsub * pf.lines;
    const int tid = (int)threadIdx.x;
#pragma unroll
    for (int s = 0; s < PF; s++) {
        const int f0 = (k + s * nc) * NT;
        if (f0 + (tid & ~63) >= total) break;  // wave-uniform
        int f = f0 + tid;
        bool ok = f < total;
        f = ok ? f : 0;
        int t = (int)((float)f * pf.inv_lines);
        int l = f - t * pf.lines;
        if (l < 0) { t--; l += pf.lines; } else if (l >= pf.lines) { t++; l -= pf.lines; }
        const int m = pf.nsub == 2 ? (t & 1) : 0;
        const int t2 = pf.nsub == 2 ? (t >> 1) : t;
        int i = (int)((float)t2 * inv_nwc);
        int w = t2 - i * nwc;
        if (w < 0) { i--; w += nwc; } else if (w >= nwc) { i++; w -= nwc; }
        const int u = c + 8 * w + i * pf.grid;
        ok = ok && u < pf.units;
        int ms = m, first = 0;
        if (pf.nsub == 1) {
            if (pf.nmat > 1 && u >= pf.wg_begin[1]) { ms = 1; first = pf.wg_begin[1]; }
            if (pf.nmat > 2 && u >= pf.wg_begin[2]) { ms = 2; first = pf.wg_begin[2]; }
        }
        const K4Mat M = ms == 0 ? pf.mats[0] : (ms == 1 ? pf.mats[1] : pf.mats[2]);
        const int row0 = (u - first) * pf.rpu;
        const uint8_t* a;
        if (l < pf.nib_lines) {
            ok = ok && row0 + (l * 8) / pf.bpr < M.rows;
            a = M.nib + ((size_t)row0 * pf.bpr * 16 + (size_t)l * 128);
        } else if (l == pf.nib_lines) {
            a = M.sub + (size_t)row0 * pf.bpr;
        } else {
            a = reinterpret_cast<const uint8_t*>(M.sup + (size_t)row0 * (pf.bpr / 8));
        }
        ok = ok && row0 < M.rows;
        a = ok ? a : pf.mats[0].nib;
        v[s] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(a) & ~(uintptr_t)3);
    }
}

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

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    uint32_t u = __float_as_uint(v);
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

}  // namespace mantle
