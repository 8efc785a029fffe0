// gemv_lane.h -- the lane-chain k4 GEMV kernel template and its launchers;
// instantiated by gemv_lane_store.hip, gemv_lane_fused.hip and gemv_lane_b8.hip.
#pragma once

#include "gemv.h"
#include "phase_trace.h"
#include "quant_device.h"

namespace mantle {

// ---------------------------------------------------------------------------
// k4 GEMV, lane-chain form (rows whose block count is 8 * BPL).
//
// Eight lanes own one output row; lane j holds blocks [j*BPL, (j+1)*BPL) of
// it in registers (BPL 128-bit nibble loads; the 8 lanes of a row cover its
// bytes contiguously).  The CPU's ordered block sum ((t0 + t1) + t2) + ... is
// kept exactly: lane j adds its own terms in order after receiving the running
// sum of lane j-1 through a DPP row_shr:1 move -- seven hand-offs, no LDS and
// no barrier.  A 256-lane workgroup covers 32 rows per unit and keeps two
// units of weight loads in flight while it computes.

__device__ __forceinline__ float dpp_shr1(float v) {  // lane i <- lane i-1 (within 16; lane 0 of a row gets 0)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_shl7(float v) {  // lane i <- lane i+7 (within 16): j=0 <- j=7 of its group
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x107, 0xF, 0xF, true));
}
template <int K>
__device__ __forceinline__ float dpp_shr(float v) {  // lane i <- lane i-K within its row of 16 (K = 1..15)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + K, 0xF, 0xF, true));
}

// Gather the 8 lanes' value of one row group into lane j == 7: lane 7 receives
// lane jj's value through a DPP row_shr:(7-jj) move.
template <int JJ>
__device__ __forceinline__ float from_lane(float v) {
    if constexpr (JJ == 7) return v;
    else return dpp_shr<7 - JJ>(v);
}

// Lane j of a row's 8 lanes owns blocks j, j+8, j+16, ... (BPL of them): each
// load instruction of the 8 lanes reads 128 contiguous bytes of the row.  The
// CPU's ordered block sum walks the lanes cyclically: block b is added by lane
// b % 8 to the running sum it receives from lane (b-1) % 8 (DPP row_shr:1, and
// row_shl:7 for the wrap from lane 7 to lane 0).
template <int EPI, int BPL, int NB, int NW, int PRO>
__global__ __launch_bounds__(NW * 64) void k4_gemv_lane_kernel(GemvParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = NW * 64;
    constexpr int NSUB = EPI == kEpiSiluMul ? 2 : 1;
    constexpr int RPU = 8 * NW;  // rows per unit
    constexpr int NQ = BPL / 4;  // u32 words of u6 bytes per lane (bytes j*BPL .. j*BPL+BPL-1 of the row)
    constexpr int NS = BPL / 2;  // u32 words of f16 super-scales per row (BPL supers)
    const int bpr = 8 * BPL;
    int8_t* sq = reinterpret_cast<int8_t*>(smem);
    float* sxs = reinterpret_cast<float*>(smem + NB * bpr * 32);
    float* work = sxs + NB * bpr;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int j = lane & 7;
    const int gbase = lane & ~7;                    // first lane of this row's group
    const int rsub = (tid >> 6) * 8 + (lane >> 3);  // row within the unit

    struct Unit {
        uint4 w[NSUB][BPL];    // nibbles of blocks j, j+8, ...
        uint32_t sub[NSUB][NQ];
        uint32_t sup[NSUB][NS];
        int unit, ms, row;
        float resid;
    };
    auto load_unit = [&](Unit& R, int unit) {
        R.unit = unit;
        int ms = 0, first = 0;
        if (EPI != kEpiSiluMul) {
            if (p.nmat > 1 && unit >= p.wg_begin[1]) { ms = 1; first = p.wg_begin[1]; }
            if (p.nmat > 2 && unit >= p.wg_begin[2]) { ms = 2; first = p.wg_begin[2]; }
        }
        R.ms = ms;
        const int row = (unit - first) * RPU + rsub;
        R.row = row;
#pragma unroll
        for (int k = 0; k < NSUB; k++) {
            const K4Mat M = pick_mat(p, NSUB == 2 ? k : ms);
            const bool ok = row < M.rows;
            const size_t r0 = (size_t)row * bpr;
#pragma unroll
            for (int q = 0; q < BPL; q++) {
                u32x4 v = {0, 0, 0, 0};
                if (ok) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(M.nib) + r0 + j + 8 * q);
                R.w[k][q] = make_uint4(v.x, v.y, v.z, v.w);
            }
            const uint32_t* sw = reinterpret_cast<const uint32_t*>(M.sub + r0 + j * BPL);
            const uint32_t* su = reinterpret_cast<const uint32_t*>(M.sup + (size_t)row * BPL);
#pragma unroll
            for (int m = 0; m < NQ; m++) R.sub[k][m] = ok ? sw[m] : 0u;
#pragma unroll
            for (int m = 0; m < NS; m++) R.sup[k][m] = ok ? su[m] : 0u;
        }
        R.resid = 0.0f;
        if (EPI == kEpiResAdd && j == 7 && row < p.mats[0].rows) R.resid = p.outs[0][row];
    };
    // u6 byte of block b = j + 8q: held by lane b / BPL of the group, word (b % BPL) / 4.
    auto sub_byte = [&](const Unit& R, int k, int q) -> uint32_t {
        const int b = j + 8 * q;
        const int src = gbase + b / BPL;
        const int wi = (b % BPL) >> 2;
        uint32_t got = 0;
#pragma unroll
        for (int m = 0; m < NQ; m++) {
            const uint32_t v = (uint32_t)__shfl((int)R.sub[k][m], src, 64);
            got = m == wi ? v : got;
        }
        return (got >> (8 * (b & 3))) & 0xFFu;
    };
    // Ordered row sum of matrix k, batch column bi; valid in lane j == 7.
    auto row_sum = [&](const Unit& R, int k, int bi) -> float {
        float t[BPL];
#pragma unroll
        for (int q = 0; q < BPL; q++) {
            const int b = j + 8 * q;
            const uint32_t supw = R.sup[k][q >> 1];
            const float sw = k4_scale((uint16_t)((q & 1) ? (supw >> 16) : (supw & 0xFFFFu)), (uint8_t)sub_byte(R, k, q));
            const float xsv = sxs[bi * bpr + b];
            float term = 0.0f;
            if (sw != 0.0f && xsv != 0.0f) {
                const int8_t* xb = sq + (bi * bpr + b) * 32;
                const uint4 xe = *reinterpret_cast<const uint4*>(xb);
                const uint4 xo = *reinterpret_cast<const uint4*>(xb + 16);
                term = (float)k4_block_dot(R.w[k][q], xe, xo) * (sw * xsv);
            }
            t[q] = term;
        }
        // Block b = jj + 8q lives in lane jj: lane 7 gathers them and adds in block order.
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < BPL; q++) {
            s = s + from_lane<0>(t[q]);
            s = s + from_lane<1>(t[q]);
            s = s + from_lane<2>(t[q]);
            s = s + from_lane<3>(t[q]);
            s = s + from_lane<4>(t[q]);
            s = s + from_lane<5>(t[q]);
            s = s + from_lane<6>(t[q]);
            s = s + from_lane<7>(t[q]);
        }
        return s;
    };

    const int G = (int)gridDim.x;
    Unit A, Bq;
    PHASE_SLOT();
    PHASE(0);
    // Activation loads first: they must not queue behind the weight stream.
    // Every trip's loads are issued here, so the prologue waits for HBM once.
    constexpr int HALVES = 16 * BPL;  // 16-value halves of one activation row
    constexpr int TRIPS = (HALVES + NT - 1) / NT;
    constexpr int QV = (NB * BPL * 256 / 16 + NT - 1) / NT;  // 16-byte pieces of qx per lane
    float pv[PRO == kProQx ? 1 : TRIPS][16], pg[PRO == kProNorm ? TRIPS : 1][16];
    uint4 qpre[PRO == kProQx ? QV : 1];
    if constexpr (PRO == kProQx) {
#pragma unroll
        for (int r = 0; r < QV; r++) {
            const int i = (tid + r * NT) * 16;
            if (i < NB * bpr * 32) qpre[r] = *reinterpret_cast<const uint4*>(p.qx + i);
        }
    } else if constexpr (NB == 1) {
#pragma unroll
        for (int t = 0; t < TRIPS; t++) {
            const int hh = tid + t * NT;
            if (HALVES % NT == 0 || hh < HALVES) {
                const float4* x4 = reinterpret_cast<const float4*>(p.x + hh * 16);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float4 u = x4[k];
                    pv[t][4 * k] = u.x; pv[t][4 * k + 1] = u.y; pv[t][4 * k + 2] = u.z; pv[t][4 * k + 3] = u.w;
                }
                if constexpr (PRO == kProNorm) {
                    const float4* g4 = reinterpret_cast<const float4*>(p.norm_w + hh * 16);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const float4 u = g4[k];
                        pg[t][4 * k] = u.x; pg[t][4 * k + 1] = u.y; pg[t][4 * k + 2] = u.z; pg[t][4 * k + 3] = u.w;
                    }
                }
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // activation loads stay ahead of the weight stream
    load_unit(A, blockIdx.x);
    const bool two = (int)blockIdx.x + G < p.ntiles;
    if (two) load_unit(Bq, blockIdx.x + G);
    if constexpr (PRO == kProQx) {
#pragma unroll
        for (int r = 0; r < QV; r++) {
            const int i = (tid + r * NT) * 16;
            if (i < NB * bpr * 32) *reinterpret_cast<uint4*>(sq + i) = qpre[r];
        }
        for (int i = tid; i < NB * bpr; i += NT) sxs[i] = p.xs[i];
        __syncthreads();
    } else if constexpr (NB == 1) {
        PHASE_AFTER(1, pv[0][0]);
        float scale = 1.0f;
        if constexpr (PRO == kProNorm) {
            constexpr int NCOL = BPL * 256;
#pragma unroll
            for (int t = 0; t < TRIPS; t++) {
                const int hh = tid + t * NT;
                if (HALVES % NT == 0 || hh < HALVES) rms_stage_half(work, rms_stage_pitch(NCOL), hh, pv[t]);
            }
            __syncthreads();
            scale = wg_rms_scale_t<NCOL, NW>(work, p.eps, p.isa, work + 16 * rms_stage_pitch(NCOL));
            PHASE(2);
        }
#pragma unroll
        for (int t = 0; t < TRIPS; t++) {
            const int hh = tid + t * NT;
            const bool live = HALVES % NT == 0 || hh < HALVES;
            if constexpr (PRO == kProNorm) {
#pragma unroll
                for (int k = 0; k < 16; k++) pv[t][k] = (pv[t][k] * scale) * pg[t][k];
            }
            quantize_half16(pv[t], live, hh, sq, sxs);
        }
        __syncthreads();
    } else {
        for (int bi = 0; bi < NB; bi++)
            wg_quantize_vec<NT>(p.x + (size_t)bi * p.cols, PRO == kProNorm ? p.norm_w : nullptr, p.eps, p.cols, p.isa,
                                work, work + bpr * 32, sq + bi * bpr * 32, sxs + bi * bpr, nullptr);
    }
    PHASE(3);
    unsigned long long best = 0;
    int nstep = 0;
    auto step = [&](Unit& cur) {
        float res[NSUB][NB];
#pragma unroll
        for (int k = 0; k < NSUB; k++)
#pragma unroll
            for (int bi = 0; bi < NB; bi++) res[k][bi] = row_sum(cur, k, bi);
        const int row = cur.row, ms = cur.ms;
        const float resid = cur.resid;
        const int ahead = cur.unit + 2 * G;
        if (ahead < p.ntiles) load_unit(cur, ahead);  // refill while the results are written
        else cur.unit = -1;
        nstep++;
        if (nstep == 1) PHASE(4);
        if (j != 7) return;
        if (EPI == kEpiSiluMul) {
            if (row < p.mats[0].rows) p.outs[0][row] = fast_silu_vec(res[0][0]) * res[1][0];
        } else {
            const int rows = pick_mat(p, ms).rows;
            if (row >= rows) return;
            float* out = pick_out(p, ms);
            if (EPI == kEpiResAdd) {
                out[row] = resid + res[0][0];
            } else {
#pragma unroll
                for (int bi = 0; bi < NB; bi++) out[(size_t)bi * rows + row] = res[0][bi];
                if (EPI == kEpiArgmax) {
                    const unsigned long long key = argmax_key(res[0][0], row);
                    best = key > best ? key : best;
                }
            }
        }
    };
    step(A);
    if (two) {
        while (true) {
            step(Bq);
            if (A.unit < 0) break;
            step(A);
            if (Bq.unit < 0) break;
        }
    }
    PHASE(5);
    if (EPI == kEpiArgmax) {
        __shared__ unsigned long long red[NW];
        for (int off = 32; off > 0; off >>= 1) {
            unsigned long long o = __shfl_down(best, off, 64);
            best = o > best ? o : best;
        }
        if ((tid & 63) == 0) red[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            unsigned long long m = red[0];
            for (int i = 1; i < NW; i++) m = red[i] > m ? red[i] : m;
            atomicMax(p.key, m);
        }
    }
}

template <int EPI, int BPL, int NB, int NW, int PRO>
static hipError_t launch_lane_gemv(GemvParams& p, hipStream_t stream) {
    auto kern = k4_gemv_lane_kernel<EPI, BPL, NB, NW, PRO>;
    constexpr int RPU = 8 * NW;
    const size_t stage = PRO == kProNorm ? ((size_t)16 * rms_stage_pitch(p.bpr * 32) + 4) * 4 : 17 * 4;
    const size_t smem = (size_t)NB * p.bpr * 36 + stage;
    if (smem > 64 * 1024) return hipErrorInvalidValue;
    int units = 0;
    if (EPI == kEpiSiluMul) {
        p.wg_begin[0] = 0;
        units = (p.mats[0].rows + RPU - 1) / RPU;
    } else {
        for (int i = 0; i < p.nmat; i++) {
            p.wg_begin[i] = units;
            units += (p.mats[i].rows + RPU - 1) / RPU;
        }
    }
    p.wg_begin[p.nmat] = units;
    p.ntiles = units;
    p.rpw = RPU;
    int slots = resident_wgs(kern, smem);
    if (gemv_max_wgs() > 0) slots = gemv_max_wgs();
    const int per = (units + slots - 1) / slots;
    const int grid = (units + per - 1) / per;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), smem, stream, p);
    return hipGetLastError();
}

// Small matrices (latency-bound): one-wave workgroups, 8 rows each, so many
// CUs share the few MB.  Large ones: four-wave workgroups streaming many units.
template <int EPI, int BPL, int NB, int PRO>
static hipError_t launch_lane_gemv_sized(GemvParams& p, hipStream_t stream) {
    int rows = 0;
    for (int i = 0; i < p.nmat; i++) rows += p.mats[i].rows;
    if (rows <= lane_small_rows()) return launch_lane_gemv<EPI, BPL, NB, 1, PRO>(p, stream);
    return launch_lane_gemv<EPI, BPL, NB, 4, PRO>(p, stream);
}

template <int EPI, int NB, int PRO>
static hipError_t try_lane_gemv(GemvParams& p, hipStream_t stream, bool* used) {
    *used = true;
    switch (p.bpr) {
        case 32: return launch_lane_gemv_sized<EPI, 4, NB, PRO>(p, stream);
        case 64: return launch_lane_gemv_sized<EPI, 8, NB, PRO>(p, stream);
        case 96: return launch_lane_gemv_sized<EPI, 12, NB, PRO>(p, stream);
        default: *used = false; return hipSuccess;
    }
}

}  // namespace mantle
