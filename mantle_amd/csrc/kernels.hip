// kernels.hip -- hand-written gfx950 kernels for Mantle's k4 decode path.
//
// Design (CDNA4, 64-wide waves, 256-thread workgroups):
//  * k4 GEMV: every lane owns whole 32-weight blocks.  A block's 16 nibble
//    bytes are one 128-bit load and consecutive lanes read consecutive blocks,
//    so a wave streams 1 KiB of contiguous HBM per load instruction.  The
//    activation is quantised to int8 once per vector (Mantle's W4A8 CPU
//    arithmetic) and staged in LDS; the block dot is 8 v_dot4_i32_i8 on the
//    nibbles shifted into the high half of each byte (exact), and the per-block
//    fp32 terms go to LDS so that one lane per row can add them in block
//    order -- the order Mantle's CPU loop uses, which makes the result
//    bit-identical to it.
//  * Epilogues fold the residual add, SiLU(gate)*up and the greedy argmax into
//    the GEMV, so the decode step has no separate elementwise launches.
//  * Decode attention fuses per-head q/k RMSNorm, RoPE, the KV append and the
//    softmax-weighted V sum in one launch per layer.
//
// Compiled with -ffp-contract=off: every fused multiply-add is explicit.
#include <hip/hip_fp16.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <array>
#include <mutex>
#include <vector>

#include "gemv.h"
#include "phase_trace.h"
#include "quant_device.h"

namespace mantle {

__global__ __launch_bounds__(kThreads) void quantize_vec_kernel(const float* __restrict__ x, const float* __restrict__ weight,
                                                                  float eps, int n, int isa, int8_t* __restrict__ qx,
                                                                  float* __restrict__ xs, float* __restrict__ norm_out) {
    extern __shared__ __align__(16) float vals[];  // ceil32(n) + 17
    const int row = blockIdx.x;
    const int np = (n + 31) & ~31;
    wg_quantize_vec(x + (size_t)row * n, weight, eps, n, isa, vals, vals + np, qx + (size_t)row * np,
                    xs + (size_t)row * (np / 32), norm_out ? norm_out + (size_t)row * n : nullptr);
}

hipError_t launch_quantize_vec(const float* x, const float* weight, float eps, int n, int batch, int isa,
                               int8_t* qx, float* xs, float* norm_out, hipStream_t stream) {
    if (!x || !qx || !xs || n <= 0 || batch <= 0) return hipErrorInvalidValue;
    const size_t smem = sizeof(float) * ((size_t)(n + 31) / 32 * 32 + 17);
    if (smem > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_vec_kernel, dim3(batch), dim3(kThreads), smem, stream, x, weight, eps, n, isa, qx,
                       xs, norm_out);
    return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                           const float* __restrict__ weight, float eps, int n, int isa) {
    __shared__ float red[17];
    const int row = blockIdx.x;
    x += (size_t)row * n;
    out += (size_t)row * n;
    float sumsq = wg_sumsq_parity(x, n, isa, red);
    float scale = rms_scale(sumsq, n, eps);
    for (int i = threadIdx.x; i < n; i += kThreads) out[i] = (x[i] * scale) * weight[i];
}

// Rows of a multiple of 64 values, up to 16 per thread (n <= 4096): the row is
// loaded once as float4 by every thread, staged transposed in LDS for the
// parity lanes (float4 runs), and scaled from registers.
static constexpr int kRowsMaxPer = 4;  // float4 per thread
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                                const float* __restrict__ weight, float eps, int n,
                                                                int isa) {
    extern __shared__ __align__(16) float tv[];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)row * n);
    const float4* w4 = reinterpret_cast<const float4*>(weight);
    float4* o4 = reinterpret_cast<float4*>(out + (size_t)row * n);
    const int n4 = n >> 2, P = rms_stage_pitch(n);
    float4 v[kRowsMaxPer], g[kRowsMaxPer];
#pragma unroll
    for (int r = 0; r < kRowsMaxPer; r++) {
        const int c = tid + r * kThreads;
        const int cc = c < n4 ? c : 0;  // unconditional loads; the surplus is not used
        v[r] = x4[cc];
        g[r] = w4[cc];
    }
#pragma unroll
    for (int r = 0; r < kRowsMaxPer; r++) {
        const int c = tid + r * kThreads;
        if (c < n4) {  // value i = 4c + e goes to staged row i % 16, column i / 16
            const int i = 4 * c;
            tv[((i + 0) & 15) * P + ((i + 0) >> 4)] = v[r].x;
            tv[((i + 1) & 15) * P + ((i + 1) >> 4)] = v[r].y;
            tv[((i + 2) & 15) * P + ((i + 2) >> 4)] = v[r].z;
            tv[((i + 3) & 15) * P + ((i + 3) >> 4)] = v[r].w;
        }
    }
    __syncthreads();
    const float scale = wg_rms_scale_rt(tv, n, eps, isa, tv + 16 * P);
#pragma unroll
    for (int r = 0; r < kRowsMaxPer; r++) {
        const int c = tid + r * kThreads;
        if (c < n4)
            o4[c] = make_float4((v[r].x * scale) * g[r].x, (v[r].y * scale) * g[r].y, (v[r].z * scale) * g[r].z,
                                (v[r].w * scale) * g[r].w);
    }
}

hipError_t launch_rmsnorm(float* out, const float* x, const float* weight, float eps, int n, int rows, int isa,
                          hipStream_t stream) {
    if (!out || !x || !weight || n <= 0 || rows <= 0) return hipErrorInvalidValue;
    if (n % 64 == 0 && n <= kRowsMaxPer * 4 * kThreads && !(((uintptr_t)out | (uintptr_t)x | (uintptr_t)weight) & 15)) {
        const size_t smem = sizeof(float) * (16 * (size_t)rms_stage_pitch(n) + 4);
        hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(kThreads), smem, stream, out, x, weight, eps, n, isa);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, stream, out, x, weight, eps, n, isa);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k4 GEMV

int64_t k4_payload_size(int64_t rows, int64_t cols) {
    int64_t bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    int64_t sub_off = (rows * spr * 2 + 63) & ~(int64_t)63;
    int64_t data_off = (sub_off + rows * bpr + 63) & ~(int64_t)63;
    return data_off + rows * bpr * 16;
}

K4Mat k4_mat_from_payload(const uint8_t* payload, int rows, int cols) {
    int64_t bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    int64_t sub_off = ((int64_t)rows * spr * 2 + 63) & ~(int64_t)63;
    int64_t data_off = (sub_off + (int64_t)rows * bpr + 63) & ~(int64_t)63;
    K4Mat m;
    m.sup = reinterpret_cast<const uint16_t*>(payload);
    m.sub = payload + sub_off;
    m.nib = payload + data_off;
    m.rows = rows;
    return m;
}

template <int MODE, int EPI>
__global__ __launch_bounds__(kThreads) void k4_gemv_kernel(GemvParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int bpr = p.bpr;
    const int B = p.batch;
    const int tid = threadIdx.x;
    constexpr bool kInt8 = MODE != kModeW4A32;
    const int qbytes = kInt8 ? B * bpr * 32 : 0;
    int8_t* sq = reinterpret_cast<int8_t*>(smem);
    float* sxs = reinterpret_cast<float*>(smem + qbytes);
    // terms[b * tp + row]: one fp32 term per (32-weight block, output row).  Rows
    // are contiguous so the ordered row sums read conflict-free; the odd pitch
    // keeps the writers (consecutive lanes = consecutive blocks) on distinct banks.
    // The fused prologue uses the same region as its fp32 staging buffer first.
    float* terms = sxs + (kInt8 ? B * bpr : 0);
    constexpr int nsub = EPI == kEpiSiluMul ? 2 : 1;
    const int tp = (nsub * p.rpw * B) | 1;
    const int per_sub = p.rpw * bpr;
    const int npairs = nsub * per_sub;  // <= kThreads * kMaxPairs: one load pass per tile

    // A workgroup walks tiles blockIdx.x, +gridDim.x, ...; tile t covers rows
    // [row0, row0 + rpw) of matrix s (of both matrices for the SiLU pair).
    auto tile_rows = [&](int tile, int& ms, int& row0) {
        ms = 0;
        int first = 0;
        if (EPI != kEpiSiluMul) {
            if (p.nmat > 1 && tile >= p.wg_begin[1]) { ms = 1; first = p.wg_begin[1]; }
            if (p.nmat > 2 && tile >= p.wg_begin[2]) { ms = 2; first = p.wg_begin[2]; }
        }
        row0 = (tile - first) * p.rpw;
    };

    // One tile's worth of in-flight weight registers.  Two of them let a
    // workgroup keep the next tile's loads in flight while it computes one.
    struct TileRegs {
        uint4 w[kMaxPairs];
        uint32_t wsc[kMaxPairs];  // f16 super-scale bits | u6 byte << 16
        int meta[kMaxPairs];      // term row << 16 | block, or -1
        int tile, ms, row0;
        float resid;              // residual operand of this lane's row (kEpiResAdd)
    };
    // Issue this lane's 128-bit nibble loads (one 32-weight block each) for a
    // tile; the scale bytes are decoded only when used, so nothing here waits.
    auto load_tile = [&](TileRegs& R, int tile) {
        R.tile = tile;
        tile_rows(tile, R.ms, R.row0);
        const int ms = R.ms, row0 = R.row0;
#pragma unroll
        for (int j = 0; j < kMaxPairs; j++) {
            const int pi = j * kThreads + tid;
            R.wsc[j] = 0;
            R.w[j] = make_uint4(0, 0, 0, 0);
            R.meta[j] = -1;
            if (pi < npairs) {
                const int k = nsub == 2 ? pi / per_sub : 0;
                const int rem = pi - k * per_sub;
                const int r = rem / bpr;
                const int b = rem - r * bpr;
                R.meta[j] = (((k * p.rpw + r) * B) << 16) | b;
                const K4Mat M = pick_mat(p, nsub == 2 ? k : ms);
                const int grow = row0 + r;
                if (grow < M.rows) {
                    const size_t blk = (size_t)grow * bpr + b;
                    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(M.nib) + blk);
                    R.w[j] = make_uint4(v.x, v.y, v.z, v.w);
                    R.wsc[j] = (uint32_t)M.sup[(size_t)grow * p.spr + (b >> 3)] | ((uint32_t)M.sub[blk] << 16);
                }
            }
        }
        R.resid = 0.0f;
        if (EPI == kEpiResAdd && tid < p.rpw && row0 + tid < p.mats[0].rows) R.resid = p.outs[0][row0 + tid];
    };
    auto compute_tile = [&](const TileRegs& R) {
#pragma unroll
        for (int j = 0; j < kMaxPairs; j++) {
            if (R.meta[j] < 0) continue;
            const int b = R.meta[j] & 0xFFFF;
            const float swj = k4_scale((uint16_t)(R.wsc[j] & 0xFFFFu), (uint8_t)(R.wsc[j] >> 16));
            float* tcol = terms + b * tp + (R.meta[j] >> 16);
            for (int bi = 0; bi < B; bi++) {
                float term = 0.0f;
                if (kInt8) {
                    const float xsv = sxs[bi * bpr + b];
                    if (swj != 0.0f && xsv != 0.0f) {
                        const int8_t* xb = sq + (bi * bpr + b) * 32;
                        const uint4 xe = *reinterpret_cast<const uint4*>(xb);
                        const uint4 xo = *reinterpret_cast<const uint4*>(xb + 16);
                        term = (float)k4_block_dot(R.w[j], xe, xo) * (swj * xsv);
                    }
                } else {
                    if (swj != 0.0f) {
                        const float* xb = p.x + (size_t)bi * p.cols + b * 32;
                        const int n = min(32, p.cols - b * 32);
                        const uint32_t wd[4] = {R.w[j].x, R.w[j].y, R.w[j].z, R.w[j].w};
                        float d = 0.0f;
                        for (int e = 0; e < n; e++) d = __builtin_fmaf((float)k4_nib(wd[e >> 3], e & 7), xb[e], d);
                        term = swj * d;
                    }
                }
                tcol[bi] = term;
            }
        }
    };
    unsigned long long best = 0;
    // Ordered row sums of one tile's terms and the epilogue.
    auto finish_tile = [&](const TileRegs& R) {
        const int row0 = R.row0;
        if (EPI == kEpiSiluMul) {
            if (tid < p.rpw) {
                const int grow = row0 + tid;
                if (grow < p.mats[0].rows) {
                    const float g = ordered_sum(terms + tid, tp, bpr);
                    const float u = ordered_sum(terms + p.rpw + tid, tp, bpr);
                    p.outs[0][grow] = fast_silu_vec(g) * u;
                }
            }
        } else {
            const int rows = pick_mat(p, R.ms).rows;
            float* out = pick_out(p, R.ms);
            for (int t = tid; t < p.rpw * B; t += kThreads) {
                const int r = t / B;
                const int bi = t - r * B;
                const int grow = row0 + r;
                if (grow >= rows) continue;
                const float sum = ordered_sum(terms + t, tp, bpr);
                if (EPI == kEpiResAdd) {
                    out[grow] = R.resid + sum;
                } else {
                    out[(size_t)bi * rows + grow] = sum;
                    if (EPI == kEpiArgmax) {
                        const unsigned long long k = argmax_key(sum, grow);
                        best = k > best ? k : best;
                    }
                }
            }
        }
    };

    const int G = (int)gridDim.x;
    TileRegs A, Bq;
    PHASE_SLOT();
    PHASE(0);
    load_tile(A, blockIdx.x);
    const bool two = (int)blockIdx.x + G < p.ntiles;
    if (two) load_tile(Bq, blockIdx.x + G);
    PHASE(1);
    if (MODE == kModeW4A8) {
        for (int i = tid * 16; i < qbytes; i += kThreads * 16)
            *reinterpret_cast<uint4*>(sq + i) = *reinterpret_cast<const uint4*>(p.qx + i);
        for (int i = tid; i < B * bpr; i += kThreads) sxs[i] = p.xs[i];
        __syncthreads();
    } else if (MODE == kModeW4A8Fused) {
        const int np = bpr * 32;
        for (int bi = 0; bi < B; bi++)
            wg_quantize_vec(p.x + (size_t)bi * p.cols, p.norm_w, p.eps, p.cols, p.isa, terms, terms + np, sq + bi * np,
                            sxs + bi * bpr, nullptr);
    }
    PHASE(2);
    // Consume `cur`, refill it with the tile two steps ahead, finish the tile.
    auto step = [&](TileRegs& cur) -> bool {
        compute_tile(cur);
        __syncthreads();
        const TileRegs done_meta = cur;  // tile identity and residual for the epilogue
        const int ahead = cur.tile + 2 * G;
        if (ahead < p.ntiles) load_tile(cur, ahead);
        else cur.tile = -1;
        PHASE(3);
        finish_tile(done_meta);
        PHASE(4);
        __syncthreads();
        return true;
    };
    step(A);
    if (two) {
        while (true) {
            step(Bq);
            if (A.tile < 0) break;
            step(A);
            if (Bq.tile < 0) break;
        }
    }
    if (EPI == kEpiArgmax) {
        __shared__ unsigned long long red[kThreads / 64];
        for (int off = 32; off > 0; off >>= 1) {
            unsigned long long o = __shfl_down(best, off, 64);
            best = o > best ? o : best;
        }
        if ((tid & 63) == 0) red[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            unsigned long long m = red[0];
            for (int i = 1; i < kThreads / 64; i++) m = red[i] > m ? red[i] : m;
            atomicMax(p.key + (blockIdx.x % kArgmaxSlots) * kArgmaxStride, m);
        }
    }
}

// Rows per tile: the fewest rows that still give one tile per resident
// workgroup (small matrices are latency-bound: spread them out), capped by the
// 256 lanes x 8 blocks a single load pass covers and by the LDS budget.
static int choose_rpw(int total_rows, int bpr, int nsub, int batch, size_t fixed_smem, size_t smem_cap, int slots) {
    int rmax = (kThreads * kMaxPairs) / (bpr * nsub);
    if (rmax < 1) rmax = 1;
    while (rmax > 1 && fixed_smem + (size_t)((nsub * rmax * batch) | 1) * bpr * 4 > smem_cap) rmax--;
    int rpw = (total_rows + slots - 1) / slots;
    if (rpw < 1) rpw = 1;
    return rpw < rmax ? rpw : rmax;
}

template <int MODE, int EPI>
static hipError_t launch_gemv_epi(GemvParams& p, hipStream_t stream) {
    constexpr int nsub = EPI == kEpiSiluMul ? 2 : 1;
    if (nsub * p.bpr > kThreads * kMaxPairs) return hipErrorInvalidValue;  // cols > 65536 (per matrix)
    auto kern = k4_gemv_kernel<MODE, EPI>;
    int total_rows = 0;
    for (int i = 0; i < p.nmat; i++) total_rows += p.mats[i].rows;
    if (EPI == kEpiSiluMul) total_rows = p.mats[0].rows;
    const size_t fixed = MODE != kModeW4A32 ? (size_t)p.batch * p.bpr * 36 : 0;
    const size_t cap = 64 * 1024;
    const size_t stage = MODE == kModeW4A8Fused && p.norm_w ? ((size_t)p.bpr * 32 + 17) * 4 : 17 * 4;
    // residency measured at the largest LDS footprint this launch can have
    int slots = resident_wgs(kern, fixed + (stage > 16 * 1024 ? stage : 16 * 1024));
    if (gemv_max_wgs() > 0) slots = gemv_max_wgs();
    p.rpw = choose_rpw(total_rows, p.bpr, nsub, p.batch, fixed, cap, slots);
    size_t work = (size_t)((nsub * p.rpw * p.batch) | 1) * p.bpr * 4;
    work = work > stage ? work : stage;
    const size_t smem = fixed + work;
    if (smem > cap) return hipErrorInvalidValue;
    int ntiles = 0;
    if (EPI == kEpiSiluMul) {
        p.wg_begin[0] = 0;
        ntiles = (p.mats[0].rows + p.rpw - 1) / p.rpw;
    } else {
        for (int i = 0; i < p.nmat; i++) {
            p.wg_begin[i] = ntiles;
            ntiles += (p.mats[i].rows + p.rpw - 1) / p.rpw;
        }
    }
    p.wg_begin[p.nmat] = ntiles;
    p.ntiles = ntiles;
    // At most one resident wave of workgroups; the tiles are dealt out evenly.
    const int per = (ntiles + slots - 1) / slots;
    const int grid = (ntiles + per - 1) / per;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), smem, stream, p);
    return hipGetLastError();
}

// Lane-chain kernel for the shapes and prologue / epilogue pairs it is
// instantiated for, else the tile kernel.  In-kernel quantisation reads x (and
// the gains) as float4: both must be 16-byte aligned.
static hipError_t dispatch_lane_gemv(GemvParams& p, GemvEpi epi, hipStream_t stream, bool* used) {
    *used = false;
    if (lane_gemv_disabled() || p.cols != p.bpr * 32) return hipSuccess;
    // 8-lane rows read their u6 bytes and f16 supers as u32 words
    for (int i = 0; i < p.nmat; i++)
        if (((uintptr_t)p.mats[i].sub | (uintptr_t)p.mats[i].sup) & 3) return hipSuccess;
    int pro = kProQx;
    if (!p.qx) {
        if (((uintptr_t)p.x | (uintptr_t)p.norm_w) & 15) return hipSuccess;
        pro = p.norm_w ? kProNorm : kProQuant;
    }
    if (p.batch == 1) {
        if (epi == kEpiStore) return lane_gemv_store(p, pro, stream, used);
        return lane_gemv_fused(p, epi, pro, stream, used);
    }
    if (p.batch == 8 && epi == kEpiStore) return lane_gemv_batch8(p, pro, stream, used);
    return hipSuccess;
}


template <int MODE>
static hipError_t launch_gemv(GemvParams& p, GemvEpi epi, hipStream_t stream) {
    switch (epi) {
        case kEpiStore: return launch_gemv_epi<MODE, kEpiStore>(p, stream);
        case kEpiResAdd: return launch_gemv_epi<MODE, kEpiResAdd>(p, stream);
        case kEpiSiluMul: return launch_gemv_epi<MODE, kEpiSiluMul>(p, stream);
        case kEpiArgmax: return launch_gemv_epi<MODE, kEpiArgmax>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

// Largest batch whose int8 activations, scales and one row's partial sums
// fit the tile kernel's 64 KiB of LDS; wider batches run as several launches
// over consecutive activation rows (the columns of a batch are independent).
static int tile_batch_fit(int bpr, size_t stage) {
    int b = 8;
    while (b > 1) {
        const size_t work = (size_t)(b | 1) * bpr * 4;
        if ((size_t)b * bpr * 36 + (work > stage ? work : stage) <= 64 * 1024) break;
        b--;
    }
    return b;
}

hipError_t launch_k4_gemv_w4a8(const K4Mat* mats, float* const* outs, int nmat, int cols, const int8_t* qx,
                               const float* xs, int batch, GemvEpi epi, unsigned long long* argmax_key,
                               hipStream_t stream) {
    if (!mats || !outs || nmat < 1 || nmat > 3 || cols <= 0 || !qx || !xs || batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    if (epi == kEpiSiluMul && (nmat != 2 || mats[0].rows != mats[1].rows || batch != 1)) return hipErrorInvalidValue;
    if ((epi == kEpiResAdd || epi == kEpiArgmax) && batch != 1) return hipErrorInvalidValue;
    if (epi == kEpiArgmax && (!argmax_key || nmat != 1)) return hipErrorInvalidValue;
    GemvParams p = {};
    for (int i = 0; i < nmat; i++) {
        if (!mats[i].nib || !mats[i].sub || !mats[i].sup || mats[i].rows <= 0 || !outs[i]) return hipErrorInvalidValue;
        p.mats[i] = mats[i];
        p.outs[i] = outs[i];
    }
    p.nmat = nmat;
    p.cols = cols;
    p.bpr = (cols + 31) / 32;
    p.spr = (p.bpr + 7) / 8;
    p.batch = batch;
    p.qx = qx;
    p.xs = xs;
    p.key = argmax_key;
    // batches of a tall matrix (the lm_head): the block dots on int8 matrix
    // cores (bit-identical); the lane GEMV's DPP dot chains bound it there
    if (batch >= 2 && nmat == 1 && (epi == kEpiStore || epi == kEpiResAdd) && p.bpr % 8 == 0 &&
        mats[0].rows >= 16384 && ((uintptr_t)qx & 15) == 0)
        return launch_k4_gemm_w4a8(mats[0], cols, qx, xs, batch, outs[0], mats[0].rows, epi, stream);
    bool used = false;
    hipError_t e = dispatch_lane_gemv(p, epi, stream, &used);
    if (used) return e;
    const int fit = tile_batch_fit(p.bpr, 17 * 4);
    if (batch > fit) {  // store epilogue only (batch > 1)
        for (int b0 = 0; b0 < batch; b0 += fit) {
            float* o[3];
            for (int i = 0; i < nmat; i++) o[i] = outs[i] + (size_t)b0 * mats[i].rows;
            const int nb = batch - b0 < fit ? batch - b0 : fit;
            e = launch_k4_gemv_w4a8(mats, o, nmat, cols, qx + (size_t)b0 * p.bpr * 32, xs + (size_t)b0 * p.bpr, nb,
                                    epi, argmax_key, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    return launch_gemv<kModeW4A8>(p, epi, stream);
}

hipError_t launch_k4_gemv_w4a8_fused(const K4Mat* mats, float* const* outs, int nmat, int cols, const float* x,
                                     const float* norm_w, float eps, int isa, int batch, GemvEpi epi,
                                     unsigned long long* argmax_key, hipStream_t stream, int8_t* q_out,
                                     float* q_scale) {
    if (!mats || !outs || nmat < 1 || nmat > 3 || cols <= 0 || !x || batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    if (epi == kEpiSiluMul && (nmat != 2 || mats[0].rows != mats[1].rows || batch != 1)) return hipErrorInvalidValue;
    if ((epi == kEpiResAdd || epi == kEpiArgmax) && batch != 1) return hipErrorInvalidValue;
    if (epi == kEpiArgmax && (!argmax_key || nmat != 1)) return hipErrorInvalidValue;
    if ((q_out || q_scale) && (epi != kEpiSiluMul || !q_out || !q_scale)) return hipErrorInvalidValue;
    GemvParams p = {};
    for (int i = 0; i < nmat; i++) {
        if (!mats[i].nib || !mats[i].sub || !mats[i].sup || mats[i].rows <= 0 || !outs[i]) return hipErrorInvalidValue;
        p.mats[i] = mats[i];
        p.outs[i] = outs[i];
    }
    p.nmat = nmat;
    p.cols = cols;
    p.bpr = (cols + 31) / 32;
    p.spr = (p.bpr + 7) / 8;
    p.batch = batch;
    p.x = x;
    p.norm_w = norm_w;
    p.eps = eps;
    p.isa = isa;
    p.key = argmax_key;
    p.q_out = q_out;
    p.q_scale = q_scale;
    bool used = false;
    hipError_t e = dispatch_lane_gemv(p, epi, stream, &used);
    if (used) return e;
    const int fit = tile_batch_fit(p.bpr, norm_w ? ((size_t)p.bpr * 32 + 17) * 4 : 17 * 4);
    if (batch > fit) {  // store epilogue only (batch > 1)
        for (int b0 = 0; b0 < batch; b0 += fit) {
            float* o[3];
            for (int i = 0; i < nmat; i++) o[i] = outs[i] + (size_t)b0 * mats[i].rows;
            const int nb = batch - b0 < fit ? batch - b0 : fit;
            e = launch_k4_gemv_w4a8_fused(mats, o, nmat, cols, x + (size_t)b0 * cols, norm_w, eps, isa, nb, epi,
                                          argmax_key, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    e = launch_gemv<kModeW4A8Fused>(p, epi, stream);
    if (e != hipSuccess || !q_out) return e;
    // the tile kernel has no quantising epilogue: a separate quantiser launch
    return launch_quantize_vec(outs[0], nullptr, 0.0f, mats[0].rows, 1, isa, q_out, q_scale, nullptr, stream);
}

// ---------------------------------------------------------------------------
// The W4A8 GEMV's activation staging (int8 blocks + block scales) for callers
// that cannot allocate: a fixed library array per device instead of caller
// scratch.  In host code `scratch` names a host-side stand-in, never its
// device address: that comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static void* scratch_ptr() {
    static std::mutex mu;
    static void* per_dev[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!per_dev[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        per_dev[dev] = p;
    }
    return per_dev[dev];
}

hipError_t launch_k4_gemv_w4a8_noalloc(const K4Mat& m, int cols, const float* x, float* y, int batch, int isa,
                                       hipStream_t stream) {
    const int bpr = (cols + 31) / 32;
    if (cols <= 0 || batch < 1 || batch > kNoAllocMaxBatch || bpr > kNoAllocMaxBlocks) {
        fprintf(stderr, "mantle_hip: no-alloc W4A8 GEMV takes at most %d columns and batch %d (got %d, %d)\n",
                kNoAllocMaxBlocks * 32, kNoAllocMaxBatch, cols, batch);
        return hipErrorInvalidValue;
    }
    unsigned char* base = static_cast<unsigned char*>(scratch_ptr());
    if (!base) return hipErrorInvalidSymbol;
    int8_t* qx = reinterpret_cast<int8_t*>(base);
    float* xs = reinterpret_cast<float*>(base + (size_t)kNoAllocMaxBatch * kNoAllocMaxBlocks * 32);
    // every byte of qx / xs the GEMV reads is written by the quantiser first
    hipError_t e = launch_quantize_vec(x, nullptr, 0.0f, cols, batch, isa, qx, xs, nullptr, stream);
    if (e != hipSuccess) return e;
    float* outs[1] = {y};
    return launch_k4_gemv_w4a8(&m, outs, 1, cols, qx, xs, batch, kEpiStore, nullptr, stream);
}

hipError_t launch_k4_gemv_w4a32(const K4Mat& m, int cols, const float* x, float* y, int batch, hipStream_t stream) {
    if (!m.nib || !m.sub || !m.sup || m.rows <= 0 || cols <= 0 || !x || !y || batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    GemvParams p = {};
    p.mats[0] = m;
    p.outs[0] = y;
    p.nmat = 1;
    p.cols = cols;
    p.bpr = (cols + 31) / 32;
    p.spr = (p.bpr + 7) / 8;
    p.batch = batch;
    p.x = x;
    if (!lane_gemv_disabled()) {
        bool used = false;
        hipError_t e = hipSuccess;
        // batches: the block dots on f16 matrix cores (x as two f16 parts)
        if (batch >= 2 && !getenv("MANTLE_HIP_W4A32_LANE")) e = k4_gemv_w4a32_mfma_launch(m, cols, x, y, batch, stream, &used);
        if (used) return e;
        e = k4_gemv_w4a32_lane(m, cols, x, y, batch, stream, &used);
        if (used) return e;
    }
    return launch_gemv<kModeW4A32>(p, kEpiStore, stream);
}

// ---------------------------------------------------------------------------
// Token embedding (rowToQuant, internal/backend/core/quant_stub.go:51-85) and step bookkeeping.

__global__ __launch_bounds__(kThreads) void embed_kernel(K4Mat emb, int cols, const int* __restrict__ prompt,
                                                         DecodeState* st, float* __restrict__ x) {
    const int pos = st->pos;
    int tok = pos < st->n_prompt ? prompt[pos] : st->next_tok;
    if (tok < 0 || tok >= emb.rows) tok = 0;  // host validates ids; never index outside the table
    const int bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const int b = c >> 5, e = c & 31;
        const size_t blk = (size_t)tok * bpr + b;
        const float sc = k4_scale(emb.sup[(size_t)tok * spr + (b >> 3)], emb.sub[blk]);
        const uint32_t word = reinterpret_cast<const uint32_t*>(emb.nib + blk * 16)[e >> 3];
        x[c] = sc == 0.0f ? 0.0f : (float)k4_nib(word, e & 7) * sc;
    }
    for (int i = threadIdx.x; i < kArgmaxSlots; i += kThreads) st->argmax_keys[i * kArgmaxStride] = 0ull;
}

// Embedding row of a raw-bf16 table (bf16 -> f32 is exact: bits << 16).
__global__ __launch_bounds__(kThreads) void embed_bf16_kernel(const uint16_t* __restrict__ emb, int vocab, int cols,
                                                              const int* __restrict__ prompt, DecodeState* st,
                                                              float* __restrict__ x) {
    const int pos = st->pos;
    int tok = pos < st->n_prompt ? prompt[pos] : st->next_tok;
    if (tok < 0 || tok >= vocab) tok = 0;
    const uint16_t* row = emb + (size_t)tok * cols;
    for (int c = threadIdx.x; c < cols; c += kThreads) x[c] = __uint_as_float((uint32_t)row[c] << 16);
    for (int i = threadIdx.x; i < kArgmaxSlots; i += kThreads) st->argmax_keys[i * kArgmaxStride] = 0ull;
}

hipError_t launch_embed_bf16(const uint16_t* emb, int vocab, int cols, const int* prompt, DecodeState* st, float* x,
                             hipStream_t stream) {
    if (!emb || !prompt || !st || !x || cols <= 0 || vocab <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_bf16_kernel, dim3(1), dim3(kThreads), 0, stream, emb, vocab, cols, prompt, st, x);
    return hipGetLastError();
}

hipError_t launch_embed(const K4Mat& emb, int cols, const int* prompt, DecodeState* st, float* x,
                        hipStream_t stream) {
    if (!emb.nib || !prompt || !st || !x || cols <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(kThreads), 0, stream, emb, cols, prompt, st, x);
    return hipGetLastError();
}

// Embedding rows of `rows` prompt tokens (tokens[r] -> x + r*cols), each as
// embed_kernel dequantises it.
__global__ __launch_bounds__(kThreads) void embed_rows_kernel(K4Mat emb, int cols, const int* __restrict__ tokens,
                                                              float* __restrict__ x) {
    const int r = blockIdx.x;
    int tok = tokens[r];
    if (tok < 0 || tok >= emb.rows) tok = 0;
    const int bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    float* xr = x + (size_t)r * cols;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const int b = c >> 5, e = c & 31;
        const size_t blk = (size_t)tok * bpr + b;
        const float sc = k4_scale(emb.sup[(size_t)tok * spr + (b >> 3)], emb.sub[blk]);
        const uint32_t word = reinterpret_cast<const uint32_t*>(emb.nib + blk * 16)[e >> 3];
        xr[c] = sc == 0.0f ? 0.0f : (float)k4_nib(word, e & 7) * sc;
    }
}

hipError_t launch_embed_rows(const K4Mat& emb, int cols, const int* tokens, int rows, float* x, hipStream_t stream) {
    if (!emb.nib || !tokens || !x || cols <= 0 || rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(rows), dim3(kThreads), 0, stream, emb, cols, tokens, x);
    return hipGetLastError();
}

// A step's bookkeeping before its final GEMV runs outside the decode step:
// the position and cleared argmax slots.
__global__ void set_step_kernel(DecodeState* st, int pos) {
    if (threadIdx.x == 0) st->pos = pos;
    for (int i = threadIdx.x; i < kArgmaxSlots; i += blockDim.x) st->argmax_keys[i * kArgmaxStride] = 0ull;
}

hipError_t launch_set_step(DecodeState* st, int pos, hipStream_t stream) {
    if (!st || pos < 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(64), 0, stream, st, pos);
    return hipGetLastError();
}

// One wave: the max over the argmax slots, then the step bookkeeping.
__global__ __launch_bounds__(64) void finish_step_kernel(DecodeState* st, int* out_tokens) {
    const int lane = threadIdx.x;
    unsigned long long key = lane < kArgmaxSlots ? st->argmax_keys[lane * kArgmaxStride] : 0ull;
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_down(key, off, 64);
        key = o > key ? o : key;
    }
    if (lane != 0) return;
    const int idx = key == 0ull ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    st->next_tok = idx;
    out_tokens[st->pos] = idx;
    st->pos = st->pos + 1;
}

hipError_t launch_finish_step(DecodeState* st, int* out_tokens, hipStream_t stream) {
    if (!st || !out_tokens) return hipErrorInvalidValue;
    hipLaunchKernelGGL(finish_step_kernel, dim3(1), dim3(64), 0, stream, st, out_tokens);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Standalone ops

__global__ void dequant_k4_kernel(K4Mat m, int cols, float* out32, uint16_t* out16) {
    const int bpr = (cols + 31) / 32, spr = (bpr + 7) / 8;
    const size_t total = (size_t)m.rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i - (size_t)r * cols);
        const int b = c >> 5, e = c & 31;
        const size_t blk = (size_t)r * bpr + b;
        const float sc = k4_scale(m.sup[(size_t)r * spr + (b >> 3)], m.sub[blk]);
        const uint32_t word = reinterpret_cast<const uint32_t*>(m.nib + blk * 16)[e >> 3];
        const float v = sc == 0.0f ? 0.0f : (float)k4_nib(word, e & 7) * sc;
        if (out32) out32[i] = v;
        if (out16) out16[i] = __half_as_ushort(__float2half_rn(v));
    }
}

hipError_t launch_dequant_k4(const K4Mat& m, int cols, float* out32, uint16_t* out16, hipStream_t stream) {
    if (!m.nib || !m.sub || !m.sup || m.rows <= 0 || cols <= 0 || (!out32 && !out16)) return hipErrorInvalidValue;
    size_t total = (size_t)m.rows * cols;
    int grid = (int)((total + kThreads - 1) / kThreads);
    if (grid > 65535) grid = 65535;
    hipLaunchKernelGGL(dequant_k4_kernel, dim3(grid), dim3(kThreads), 0, stream, m, cols, out32, out16);
    return hipGetLastError();
}

// ffn.go:72-90: act = fastSiluVec(gate) * up for 8-wide chunks, scalar Silu tail.
__global__ void silu_mul_kernel(const float* gate, const float* up, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int vec_end = n & ~7;
    if (i < vec_end) {
        out[i] = fast_silu_vec(gate[i]) * up[i];
    } else {
        const float g = gate[i];
        float sig = g > 10.0f ? 1.0f : (g < -10.0f ? 0.0f : 1.0f / (1.0f + fast_exp_scalar(-g)));
        out[i] = (g * sig) * up[i];
    }
}

hipError_t launch_silu_mul(const float* gate, const float* up, float* out, int n, hipStream_t stream) {
    if (!gate || !up || !out || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, stream, gate, up, out, n);
    return hipGetLastError();
}

__global__ void add_kernel(float* dst, const float* src, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = dst[i] + src[i];
}

hipError_t launch_add(float* dst, const float* src, int n, hipStream_t stream) {
    if (!dst || !src || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, stream, dst, src, n);
    return hipGetLastError();
}

// argmaxHost (runtime_greedy.go:70-82): strict '>' keeps the first maximum.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* x, int n, int* out_idx) {
    __shared__ unsigned long long red[kThreads / 64];
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        unsigned long long k = argmax_key(x[i], i);
        best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_down(best, off, 64);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = red[0];
        for (int i = 1; i < kThreads / 64; i++) m = red[i] > m ? red[i] : m;
        *out_idx = (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
    }
}

hipError_t launch_argmax(const float* x, int n, int* out_idx, hipStream_t stream) {
    if (!x || !out_idx || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kThreads), 0, stream, x, n, out_idx);
    return hipGetLastError();
}

// Softmax rows (ops.go:83-106) -- one workgroup per row, ordered sum.
__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(float* data, int cols) {
    __shared__ float smax[kThreads / 64];
    __shared__ float ssum;
    float* x = data + (size_t)blockIdx.x * cols;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < cols; i += kThreads) m = fmaxf(m, x[i]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_down(m, off, 64));
    if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = m;
    __syncthreads();
    float maxv = smax[0];
    for (int i = 1; i < kThreads / 64; i++) maxv = fmaxf(maxv, smax[i]);
    for (int i = threadIdx.x; i < cols; i += kThreads) x[i] = fast_exp_scalar(x[i] - maxv);
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < cols; i++) s += x[i];
        ssum = s;
    }
    __syncthreads();
    if (ssum == 0.0f) return;
    const float inv = 1.0f / ssum;
    for (int i = threadIdx.x; i < cols; i += kThreads) x[i] = x[i] * inv;
}

hipError_t launch_softmax_rows(float* data, int rows, int cols, hipStream_t stream) {
    if (!data || rows <= 0 || cols <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3(rows), dim3(kThreads), 0, stream, data, cols);
    return hipGetLastError();
}

__global__ void rope_table_kernel(float* x, const float* c, const float* s, int head_dim, int half) {
    float* lo = x + (size_t)blockIdx.x * head_dim;
    float* hi = lo + half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float x0 = lo[i], x1 = hi[i];
        lo[i] = x0 * c[i] - x1 * s[i];
        hi[i] = __builtin_fmaf(x0, s[i], x1 * c[i]);
    }
}

hipError_t launch_rope_table(float* x, const float* cosv, const float* sinv, int head_dim, int half, int n_heads,
                             hipStream_t stream) {
    if (!x || !cosv || !sinv || head_dim <= 0 || half <= 0 || half * 2 > head_dim || n_heads <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_table_kernel, dim3(n_heads), dim3(128), 0, stream, x, cosv, sinv, head_dim, half);
    return hipGetLastError();
}

// RoPE from inverse frequencies: float64 (Mantle's CPU invFreq []float64,
// internal/backend/simd/loader.go:1604-1612) or float32 (the CUDA backend's
// pre-uploaded table, internal/backend/cuda/native/attn_fused.cu:51-58);
// either way the angle pos * invFreq[i] and its cos / sin are evaluated in
// f64 as applyRoPE does (ops_avx512.go:146-160), then the CPU's pair update.
template <typename F>
__global__ void rope_freq_kernel(float* x, const F* inv_freq, int pos, float attn_scale, int head_dim, int half) {
    float* lo = x + (size_t)blockIdx.x * head_dim;
    float* hi = lo + half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const double ang = (double)pos * (double)inv_freq[i];
        float c = (float)cos(ang), s = (float)sin(ang);
        if (attn_scale != 1.0f) {
            c = c * attn_scale;
            s = s * attn_scale;
        }
        float x0 = lo[i], x1 = hi[i];
        lo[i] = x0 * c - x1 * s;
        hi[i] = __builtin_fmaf(x0, s, x1 * c);
    }
}

template <typename F>
static hipError_t launch_rope_freq(float* x, const F* inv_freq, int pos, float attn_scale, int head_dim, int half,
                                   int n_heads, hipStream_t stream) {
    if (!x || !inv_freq || head_dim <= 0 || half <= 0 || half * 2 > head_dim || n_heads <= 0 || pos < 0)
        return hipErrorInvalidValue;
    if (attn_scale == 0.0f) attn_scale = 1.0f;
    hipLaunchKernelGGL(rope_freq_kernel<F>, dim3(n_heads), dim3(128), 0, stream, x, inv_freq, pos, attn_scale,
                       head_dim, half);
    return hipGetLastError();
}

hipError_t launch_rope_f64(float* x, const double* inv_freq, int pos, float attn_scale, int head_dim, int half,
                           int n_heads, hipStream_t stream) {
    return launch_rope_freq(x, inv_freq, pos, attn_scale, head_dim, half, n_heads, stream);
}

hipError_t launch_rope_f32(float* x, const float* inv_freq, int pos, float attn_scale, int head_dim, int half,
                           int n_heads, hipStream_t stream) {
    return launch_rope_freq(x, inv_freq, pos, attn_scale, head_dim, half, n_heads, stream);
}

__global__ void store_kv_row_kernel(float* cache, const float* src, int cache_pos, int kv_stride) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kv_stride; i += gridDim.x * blockDim.x)
        cache[(size_t)cache_pos * kv_stride + i] = src[i];
}

// StoreKV into an f16 cache (ops_runtime.go:112-131, Float32ToFloat16Slice):
// Mantle's truncating conversion.
__global__ void store_kv_row_f16_kernel(uint16_t* cache, const float* src, int cache_pos, int kv_stride) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kv_stride; i += gridDim.x * blockDim.x)
        cache[(size_t)cache_pos * kv_stride + i] = mantle_f32_to_f16_trunc(src[i]);
}

hipError_t launch_store_kv_row_f16(uint16_t* cache, const float* src, int cache_pos, int kv_stride,
                                   hipStream_t stream) {
    if (!cache || !src || cache_pos < 0 || kv_stride <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(store_kv_row_f16_kernel, dim3((kv_stride + kThreads - 1) / kThreads), dim3(kThreads), 0, stream,
                       cache, src, cache_pos, kv_stride);
    return hipGetLastError();
}

hipError_t launch_store_kv_row(float* cache, const float* src, int cache_pos, int kv_stride, hipStream_t stream) {
    if (!cache || !src || cache_pos < 0 || kv_stride <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(store_kv_row_kernel, dim3((kv_stride + kThreads - 1) / kThreads), dim3(kThreads), 0, stream,
                       cache, src, cache_pos, kv_stride);
    return hipGetLastError();
}

}  // namespace mantle

#ifdef MANTLE_PHASE_TRACE
namespace mantle {
MANTLE_PHASE_READER(phase_read_kernels)
int phase_read_lane_store(unsigned long long*, int, unsigned*);
int phase_read_lane_fused(unsigned long long*, int, unsigned*);
int phase_read_lane_b8(unsigned long long*, int, unsigned*);
int phase_read_attention(unsigned long long*, int, unsigned*);
}  // namespace mantle
// All translation units' stamps, ordered by launch start.
extern "C" int mantleHipDebugPhaseTrace(unsigned long long* out, int max_slots, unsigned* n) {
    int (*readers[])(unsigned long long*, int, unsigned*) = {mantle::phase_read_kernels, mantle::phase_read_lane_store,
                                                             mantle::phase_read_lane_fused, mantle::phase_read_lane_b8,
                                                             mantle::phase_read_attention};
    std::vector<std::array<unsigned long long, 8>> rows;
    for (auto rd : readers) {
        std::vector<unsigned long long> buf((size_t)8192 * 8);
        unsigned k = 0;
        int e = rd(buf.data(), 8192, &k);
        if (e) return e;
        for (unsigned i = 0; i < k && i < 8192; i++) {
            std::array<unsigned long long, 8> r;
            for (int c = 0; c < 8; c++) r[c] = buf[i * 8 + c];
            rows.push_back(r);
        }
    }
    std::sort(rows.begin(), rows.end(), [](const auto& a, const auto& b) { return a[0] < b[0]; });
    const size_t m = rows.size() < (size_t)max_slots ? rows.size() : (size_t)max_slots;
    for (size_t i = 0; i < m; i++)
        for (int c = 0; c < 8; c++) out[i * 8 + c] = rows[i][c];
    *n = (unsigned)m;
    return 0;
}
#endif
