// gemv_lane.h -- the lane-chain k4 GEMV kernel template and its launchers;
// instantiated by gemv_lane_store.hip, gemv_lane_fused.hip and gemv_lane_b8.hip.
#pragma once

#include "gemv.h"
#include "phase_trace.h"
#include "quant_device.h"

namespace mantle {

// ---------------------------------------------------------------------------
// k4 GEMV, lane-group form.
//
// LPR lanes (8 or 16) own one output row; lane j holds blocks j, j+LPR,
// j+2*LPR, ... (BPL of them) in registers, so each load instruction of a row's
// lanes reads LPR*16 contiguous nibble bytes.  The CPU's ordered block sum
// ((t0 + t1) + t2) + ... is kept exactly: the row's last lane gathers every
// term through DPP row_shr moves (all LPR lanes sit in one 16-lane DPP row)
// and adds them in block order -- no LDS, no barrier.  Eight lanes per row
// keep the load count per row low for large matrices; sixteen halve the loads
// each wave must issue, which is what bounds the latency of small ones.

template <int K>
__device__ __forceinline__ float dpp_shr(float v) {  // lane i <- lane i-K within its row of 16 (K = 1..15)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + K, 0xF, 0xF, true));
}

// Lane LPR-1 of a row group receives lane JJ's value (DPP row_shr:(LPR-1-JJ)).
template <int JJ, int LPR>
__device__ __forceinline__ float from_lane(float v) {
    if constexpr (JJ == LPR - 1) return v;
    else return dpp_shr<LPR - 1 - JJ>(v);
}

template <int LPR, int JJ = 0>
__device__ __forceinline__ float gather_add(float s, float t) {
    if constexpr (JJ == LPR) return s;
    else return gather_add<LPR, JJ + 1>(s + from_lane<JJ, LPR>(t), t);
}

// gather_add for NB independent sums at once: the chains interleave, so each
// DPP add's latency is hidden behind the other columns' adds.
#ifndef MANTLE_BATCH_GROUP
#define MANTLE_BATCH_GROUP 4
#endif
static constexpr int kBatchGroup = MANTLE_BATCH_GROUP;  // batch columns summed together
template <int LPR, int NB, int JJ = 0>
__device__ __forceinline__ void gather_add_n(float (&s)[NB], const float (&t)[NB]) {
    if constexpr (JJ < LPR) {
#pragma unroll
        for (int bi = 0; bi < NB; bi++) s[bi] = s[bi] + from_lane<JJ, LPR>(t[bi]);
        gather_add_n<LPR, NB, JJ + 1>(s, t);
    }
}

// Rows wider than a lane's registers hold (BPLT > BPL blocks per lane) are
// processed in NCHK pieces of BPL blocks per lane, in block order: piece c
// covers blocks LPR*BPL*c .. LPR*BPL*(c+1)-1, so the last lane's running sum
// continues the CPU's ordered sum from one piece to the next.  Blocks past the
// row in the last piece re-read the row's last block and add exactly 0.
template <int EPI, int LPR, int BPL, int NB, int NW, int PRO, int D, int BPLT_ = 0>
__global__ __launch_bounds__(NW * 64) void k4_gemv_lane_kernel(GemvParams p) {
    static_assert(LPR == 8 || LPR == 16, "8 or 16 lanes per row");
    constexpr int BPLT = BPLT_ ? BPLT_ : BPL;              // blocks per lane over the whole row
    constexpr int NCHK = (BPLT + BPL - 1) / BPL;           // pieces per row
    constexpr bool CHUNKED = NCHK > 1;
    static_assert(!CHUNKED || NB == 1, "pieced rows at batch 1 only");
    static_assert(!CHUNKED || D == 2, "pieces of a row are double-buffered");
    // 8-lane whole rows take their u6 bytes and supers as u32 words
    constexpr bool WORDS = LPR == 8 && !CHUNKED;
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = NW * 64;
    constexpr int NSUB = EPI == kEpiSiluMul ? 2 : 1;
    constexpr int RPW = 64 / LPR;   // rows per wave
    constexpr int RPU = RPW * NW;   // rows per unit
    constexpr int BPR = LPR * BPLT;  // blocks per row
    // WORDS: the u6 bytes of a row arrive as u32 words (lane j: bytes j*BPL ..
    // j*BPL+BPL-1) and the f16 supers as words; otherwise one byte / half each.
    constexpr int NQ = WORDS ? BPL / 4 : BPL;
    constexpr int NS = WORDS ? BPL / 2 : BPL;
    static_assert(!WORDS || BPL % 4 == 0, "8-lane rows take 4k blocks per lane");
    const int bpr = BPR;
    int8_t* sq = reinterpret_cast<int8_t*>(smem);
    float* sxs = reinterpret_cast<float*>(smem + NB * bpr * 32);
    float* work = sxs + NB * bpr;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int j = lane % LPR;
    const int gbase = lane - j;                          // first lane of this row's group
    const int rsub = (tid >> 6) * RPW + lane / LPR;      // row within the unit

    struct Unit {
        uint4 w[NSUB][BPL];  // nibbles of blocks j, j+LPR, ...
        uint32_t sub[NSUB][NQ];
        uint32_t sup[NSUB][NS];
        int unit, ms, row, piece, chunk;
        float resid;
    };
    const int G = (int)gridDim.x;
    // Piece i of this workgroup: unit blockIdx.x + (i / NCHK) * G, chunk i % NCHK.
    auto unit_of = [&](int i) { return (int)blockIdx.x + (NCHK == 1 ? i : i / NCHK) * G; };
    auto load_unit = [&](Unit& R, int piece) {
        const int unit = unit_of(piece);
        const int chunk = NCHK == 1 ? 0 : piece % NCHK;
        R.piece = piece;
        R.chunk = chunk;
        R.unit = unit;
        int ms = 0, first = 0;
        if (EPI != kEpiSiluMul) {
            if (p.nmat > 1 && unit >= p.wg_begin[1]) { ms = 1; first = p.wg_begin[1]; }
            if (p.nmat > 2 && unit >= p.wg_begin[2]) { ms = 2; first = p.wg_begin[2]; }
        }
        R.ms = ms;
        const int row = (unit - first) * RPU + rsub;
        R.row = row;
        // Loads are unconditional: a row past the matrix re-reads its last row
        // (never stored), so no branch or wait sits between the loads.  Offsets
        // are 32-bit from a uniform base (SGPR base + VGPR offset + immediate).
#pragma unroll
        for (int k = 0; k < NSUB; k++) {
            const K4Mat M = pick_mat(p, NSUB == 2 ? k : ms);
            const uint32_t rc = (uint32_t)(row < M.rows ? row : M.rows - 1);
            if constexpr (CHUNKED) {
                const unsigned char* nb = reinterpret_cast<const unsigned char*>(M.nib);
#pragma unroll
                for (int q = 0; q < BPL; q++) {
                    const int qg = chunk * BPL + q;
                    const uint32_t b = (uint32_t)(j + LPR * (qg < BPLT ? qg : BPLT - 1));
                    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nb + (rc * BPR + b) * 16u));
                    R.w[k][q] = make_uint4(v.x, v.y, v.z, v.w);
                    R.sub[k][q] = M.sub[rc * BPR + b];
                    R.sup[k][q] = M.sup[rc * (BPR / 8) + (b >> 3)];
                }
                continue;
            }
            const unsigned char* nb = reinterpret_cast<const unsigned char*>(M.nib) + (rc * BPR + j) * 16u;
#pragma unroll
            for (int q = 0; q < BPL; q++) {
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nb + q * LPR * 16));
                R.w[k][q] = make_uint4(v.x, v.y, v.z, v.w);
            }
            if constexpr (WORDS) {
                const uint32_t* sw = reinterpret_cast<const uint32_t*>(M.sub + rc * BPR + j * BPL);
                const uint32_t* su = reinterpret_cast<const uint32_t*>(M.sup + rc * BPL);
#pragma unroll
                for (int m = 0; m < NQ; m++) R.sub[k][m] = sw[m];
#pragma unroll
                for (int m = 0; m < NS; m++) R.sup[k][m] = su[m];
            } else {
                // block b = j + 16q: u6 byte b, super (b / 8) = 2q + j / 8 of the row's bpr / 8
                const uint8_t* sb = M.sub + rc * BPR + j;
                const uint16_t* sp = M.sup + rc * (BPR / 8) + (j >> 3);
#pragma unroll
                for (int q = 0; q < BPL; q++) R.sub[k][q] = sb[16 * q];
#pragma unroll
                for (int q = 0; q < BPL; q++) R.sup[k][q] = sp[2 * q];
            }
        }
        R.resid = 0.0f;
        if constexpr (EPI == kEpiResAdd) {
            const int rows0 = p.mats[0].rows;
            R.resid = p.outs[0][row < rows0 ? row : rows0 - 1];
        }
    };
    // LPR 8: u6 byte of block b = j + 8q is held by lane b / BPL of the group, word (b % BPL) / 4.
    auto sub_byte = [&](const Unit& R, int k, int q) -> uint32_t {
        if constexpr (!WORDS) {
            return R.sub[k][q];
        } else {
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
        }
    };
    auto super_half = [&](const Unit& R, int k, int q) -> uint16_t {
        if constexpr (!WORDS) {
            return (uint16_t)R.sup[k][q];
        } else {
            const uint32_t supw = R.sup[k][q >> 1];
            return (uint16_t)((q & 1) ? (supw >> 16) : (supw & 0xFFFFu));
        }
    };
    // Ordered row sum of matrix k, batch column bi; valid in lane j == LPR-1.
    // The weight block scales of matrix k (shared by every batch column).
    auto block_scales = [&](const Unit& R, int k, float (&sw)[BPL]) {
#pragma unroll
        for (int q = 0; q < BPL; q++) sw[q] = k4_scale(super_half(R, k, q), (uint8_t)sub_byte(R, k, q));
    };
    // s0: the running sum of the row's earlier pieces (0 for the first).
    auto row_sum = [&](const Unit& R, int k, int bi, const float (&swk)[BPL], float s0) -> float {
        float t[BPL];
#pragma unroll
        for (int q = 0; q < BPL; q++) {
            const int qg = R.chunk * BPL + q;
            const bool live = !CHUNKED || BPLT % BPL == 0 || qg < BPLT;
            const int b = j + LPR * (live ? qg : BPLT - 1);
            const float sw = swk[q];
            const float xsv = sxs[bi * bpr + b];
            float term = 0.0f;
            if (live && sw != 0.0f && xsv != 0.0f) {
                const int8_t* xb = sq + (bi * bpr + b) * 32;
                const uint4 xe = *reinterpret_cast<const uint4*>(xb);
                const uint4 xo = *reinterpret_cast<const uint4*>(xb + 16);
                term = (float)k4_block_dot(R.w[k][q], xe, xo) * (sw * xsv);
            }
            t[q] = term;
        }
        // Block b = jj + LPR*q lives in lane jj: the last lane adds them in block order.
        float s = s0;
#pragma unroll
        for (int q = 0; q < BPL; q++) s = gather_add<LPR>(s, t[q]);
        return s;
    };
    // All NB batch columns of matrix k: per block the terms of every column,
    // then the ordered sums of the columns interleaved (same order per column).
    auto row_sums = [&](const Unit& R, int k, const float (&swk)[BPL], float (&res)[NB]) {
        // columns in groups of CG: a group's terms, then its CG ordered sums
        // interleaved; one group at a time bounds the live DPP results
        constexpr int CG = NB % kBatchGroup == 0 ? kBatchGroup : 1;
#pragma unroll
        for (int b0 = 0; b0 < NB; b0 += CG) {
            float t[BPL][CG];
#pragma unroll
            for (int q = 0; q < BPL; q++) {
                const int b = j + LPR * q;
#pragma unroll
                for (int c = 0; c < CG; c++) {
                    const int bi = b0 + c;
                    const float xsv = sxs[bi * bpr + b];
                    float term = 0.0f;
                    if (swk[q] != 0.0f && xsv != 0.0f) {
                        const int8_t* xb = sq + (bi * bpr + b) * 32;
                        const uint4 xe = *reinterpret_cast<const uint4*>(xb);
                        const uint4 xo = *reinterpret_cast<const uint4*>(xb + 16);
                        term = (float)k4_block_dot(R.w[k][q], xe, xo) * (swk[q] * xsv);
                    }
                    t[q][c] = term;
                }
            }
            float acc[CG];
#pragma unroll
            for (int c = 0; c < CG; c++) acc[c] = 0.0f;
#pragma unroll
            for (int q = 0; q < BPL; q++) gather_add_n<LPR, CG>(acc, t[q]);
#pragma unroll
            for (int c = 0; c < CG; c++) {
                // materialise the sum here: left alone, the adds sink into the
                // last lane's store branch and keep every DPP result live until then
                asm volatile("" : "+v"(acc[c]));
                res[b0 + c] = acc[c];
            }
        }
    };

    static_assert(D == 1 || D == 2, "one or two units in flight");
    Unit A, Bq;  // D == 2: the workgroup's even pieces in A, odd ones in Bq
    PHASE_SLOT();
    PHASE(0);
    // Activation loads first: they must not queue behind the weight stream.
    // Every trip's loads are issued here, so the prologue waits for HBM once.
    // The fp32 row is spread over the workgroup in pieces of VPT consecutive
    // values (VPT = 16 / 8 / 4 / 2: every thread busy where the row allows),
    // so a multi-wave workgroup shares the RMSNorm and quantisation work.
    constexpr int NCOLS = BPR * 32;
    constexpr int VPT0 = NCOLS / NT;
    constexpr int VPT = VPT0 >= 16 ? 16 : (VPT0 >= 8 ? 8 : (VPT0 >= 4 ? 4 : 2));
    constexpr int PIECES = NCOLS / VPT;
    constexpr int TRIPS = (PIECES + NT - 1) / NT;
    constexpr int QV = (NB * BPR * 2 + NT - 1) / NT;  // 16-byte pieces of qx per lane
    float pv[PRO == kProQx ? 1 : TRIPS][VPT], pg[PRO == kProNorm ? TRIPS : 1][VPT];
    constexpr int XV = (NB * BPR + NT - 1) / NT;  // block scales per lane
    u32x4 qpre[PRO == kProQx ? QV : 1];
    float xpre[PRO == kProQx ? XV : 1];
    if constexpr (PRO == kProQx) {
        // unconditional (clamped) loads; the surplus is not stored
#pragma unroll
        for (int r = 0; r < QV; r++) {
            const int i = (tid + r * NT) * 16;
            qpre[r] = *reinterpret_cast<const u32x4*>(p.qx + (i < NB * BPR * 32 ? i : 0));
        }
#pragma unroll
        for (int r = 0; r < XV; r++) {
            const int i = tid + r * NT;
            xpre[r] = p.xs[i < NB * BPR ? i : 0];
        }
    } else if constexpr (NB == 1) {
#pragma unroll
        for (int t = 0; t < TRIPS; t++) {
            // unconditional: threads past the row re-read piece 0 (not used)
            const int pc = PIECES % NT == 0 || tid + t * NT < PIECES ? tid + t * NT : 0;
            load_piece<VPT>(p.x + pc * VPT, pv[t]);
            if constexpr (PRO == kProNorm) load_piece<VPT>(p.norm_w + pc * VPT, pg[t]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // activation loads stay ahead of the weight stream
    load_unit(A, 0);
    const bool two = D == 2 && unit_of(1) < p.ntiles;
    if (two) load_unit(Bq, 1);
    PHASE(1);
    if constexpr (PRO == kProQx) {
        PHASE_AFTER(2, qpre[0].x);
#pragma unroll
        for (int r = 0; r < QV; r++) {
            const int i = (tid + r * NT) * 16;
            if (i < NB * bpr * 32) *reinterpret_cast<u32x4*>(sq + i) = qpre[r];
        }
#pragma unroll
        for (int r = 0; r < XV; r++) {
            const int i = tid + r * NT;
            if (i < NB * bpr) sxs[i] = xpre[r];
        }
        __syncthreads();
    } else if constexpr (NB == 1) {
        PHASE_AFTER(2, pv[0][0]);
        float scale = 1.0f;
        if constexpr (PRO == kProNorm) {
#pragma unroll
            for (int t = 0; t < TRIPS; t++) {
                const int pc = tid + t * NT;
                if (PIECES % NT == 0 || pc < PIECES) rms_stage_piece<VPT>(work, rms_stage_pitch(NCOLS), pc, pv[t]);
            }
            __syncthreads();
            scale = wg_rms_scale_t<NCOLS, NW>(work, p.eps, p.isa, work + 16 * rms_stage_pitch(NCOLS));
            PHASE(6);
        }
#pragma unroll
        for (int t = 0; t < TRIPS; t++) {
            const int pc = tid + t * NT;
            const bool live = PIECES % NT == 0 || pc < PIECES;
            if constexpr (PRO == kProNorm) {
#pragma unroll
                for (int k = 0; k < VPT; k++) pv[t][k] = (pv[t][k] * scale) * pg[t][k];
            }
            quantize_piece<VPT>(pv[t], live, pc, sq, sxs);
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
    float carry[NSUB] = {};  // running sums of the current row's earlier pieces
    auto step = [&](Unit& cur) {
        float res[NSUB][NB];
#pragma unroll
        for (int k = 0; k < NSUB; k++) {
            float swk[BPL];
            block_scales(cur, k, swk);
            if constexpr (NB == 1) res[k][0] = row_sum(cur, k, 0, swk, CHUNKED ? carry[k] : 0.0f);
            else row_sums(cur, k, swk, res[k]);
        }
        const int row = cur.row, ms = cur.ms, unit = cur.unit;
        const bool last = !CHUNKED || cur.chunk == NCHK - 1;
        const float resid = cur.resid;
        const int ahead = cur.piece + D;
        if (unit_of(ahead) < p.ntiles) load_unit(cur, ahead);  // refill while the results are written
        else cur.unit = -1;
        if constexpr (CHUNKED) {
#pragma unroll
            for (int k = 0; k < NSUB; k++) carry[k] = last ? 0.0f : res[k][0];
            if (!last) return;
        }
        nstep++;
        if (nstep == 1) PHASE(4);
        if constexpr (EPI == kEpiSiluMul) {
            const int rows = p.mats[0].rows;
            float y = 0.0f;
            if (j == LPR - 1 && row < rows) {
                y = fast_silu_vec(res[0][0]) * res[1][0];
                p.outs[0][row] = y;
            }
            if constexpr (RPU == 32) {
                // A unit is 32 consecutive rows: exactly one int8 block of the
                // next GEMV's activation, quantised here instead of by every
                // workgroup of that GEMV.
                if (p.q_out) {
                    float* slot = work;  // the prologue's staging is no longer read
                    if (j == LPR - 1) slot[rsub] = y;
                    __syncthreads();
                    if (tid < 32) {
                        float sc;
                        const int32_t q = quant_lane32(slot[tid], &sc);
                        // rows past the matrix hold y = 0: their bytes are 0
                        p.q_out[unit * 32 + qx_perm(tid)] = (int8_t)q;
                        if (tid == 0) p.q_scale[unit] = sc;
                    }
                    __syncthreads();
                }
            }
        } else {
            if (j != LPR - 1) return;
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
    if constexpr (D == 1) {
        step(A);
        while (A.unit >= 0) step(A);
    } else {
        step(A);
        if (two) {
            while (true) {
                step(Bq);
                if (A.unit < 0) break;
                step(A);
                if (Bq.unit < 0) break;
            }
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
            atomicMax(p.key + (blockIdx.x % kArgmaxSlots) * kArgmaxStride, m);
        }
    }
}

template <int EPI, int LPR, int BPL, int NB, int NW, int PRO, int D = 2, int BPLT = 0>
static hipError_t launch_lane_gemv(GemvParams& p, hipStream_t stream) {
    auto kern = k4_gemv_lane_kernel<EPI, LPR, BPL, NB, NW, PRO, D, BPLT>;
    constexpr int RPU = (64 / LPR) * NW;
    const size_t stage = PRO == kProNorm ? ((size_t)16 * rms_stage_pitch(p.bpr * 32) + 4) * 4 : 40 * 4;
    const size_t smem = (size_t)NB * p.bpr * 36 + stage;
    if (smem > 64 * 1024) return hipErrorInvalidValue;
    if (EPI == kEpiSiluMul && p.q_out && RPU != 32) return hipErrorInvalidValue;  // quantises 32-row units
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
    // D == 1: one unit per workgroup (the dispatcher keeps the CUs full);
    // D > 1: at most one resident wave of workgroups, units dealt out evenly
    // (pieced rows: one unit per workgroup, its pieces double-buffered)
    int slots = D == 1 || BPLT > BPL ? units : resident_wgs(kern, smem);
    if (gemv_max_wgs() > 0) slots = gemv_max_wgs();
    const int per = (units + slots - 1) / slots;
    const int grid = (units + per - 1) / per;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), smem, stream, p);
    return hipGetLastError();
}

// Blocks per lane of one piece of a row that spans BPLT blocks per lane: whole
// rows up to MAXC blocks per lane, else the fewest pieces of at most MAXC.
template <int BPLT, int MAXC>
constexpr int piece_bpl() {
    constexpr int n = (BPLT + MAXC - 1) / MAXC;
    return (BPLT + n - 1) / n;
}

// Large matrices (the logits): four-wave workgroups of one 32-row unit each,
// as many as there are units; 8 lanes per row where the row fits 8 lanes'
// registers.  Measured on the logits shape, this beats a resident grid that
// streams several units per workgroup (ring depth 1-4, 8 or 16 lanes per row,
// 2-8 waves): the dispatcher refills CUs as workgroups finish, and the
// per-workgroup prologue overlaps other loads.
// Small ones are latency-bound, and what bounds them is the loads each wave
// must issue before its data starts to arrive: 16 lanes per row and
// one-wave workgroups of 4 rows spread them over every CU.  The quantising
// SiLU epilogue needs 32-row units: 16 lanes per row in eight-wave workgroups.
// Rows of more than 6 blocks per lane (4 for gate and up) go in double-buffered pieces.
template <int EPI, int BPR, int NB, int PRO>
static hipError_t launch_lane_gemv_sized(GemvParams& p, hipStream_t stream) {
    static_assert(BPR % 16 == 0, "16-lane rows need a multiple of 16 blocks");
    constexpr int T16 = BPR / 16;             // blocks per lane at 16 lanes per row
    // two matrices' blocks per lane (gate and up) with the SiLU epilogue: at most 4
    constexpr int C16 = piece_bpl<T16, EPI == kEpiSiluMul ? 4 : 6>();
    constexpr bool L8 = BPR % 32 == 0 && BPR / 8 <= 8;  // whole 8-lane rows (u6 words: 4k blocks per lane)
    constexpr int T8 = BPR / 8;
    int rows = 0;
    for (int i = 0; i < p.nmat; i++) rows += p.mats[i].rows;
    const bool q32 = EPI == kEpiSiluMul && p.q_out;
    const bool large = rows > lane_small_rows() || (int64_t)rows * BPR >= lane_large_blocks();
    if constexpr (BPR >= 80) {
        // wide gate/up rows with the quantising SiLU epilogue: 32-row units of
        // four waves at 8 lanes per row, in pieces; two such workgroups fit a
        // CU, so the 4B/8B unit counts (304, 384) run in a single round
        // (pieces of up to 5 blocks per lane: the 4B rows in two pieces of 5
        // measured 15.9 -> 15.3 us against three of 4, 4, 2; 16 lanes per row
        // in eight-wave workgroups: 18.9 us)
        if (q32) return launch_lane_gemv<EPI, 8, piece_bpl<T8, 5>(), NB, 4, PRO, 2, T8>(p, stream);
    }
    // (16-lane rows make 16-row units at four waves: the quantising SiLU
    // epilogue takes the eight-wave instance below)
    if (large && (L8 || !q32)) {
        if constexpr (L8) {
            // with the RMSNorm prologue (the decode step's logits): resident
            // workgroups streaming several units each, so each runs the
            // prologue once (0.6B decode 1205 -> 1207 tok/s)
            if (PRO == kProNorm) return launch_lane_gemv<EPI, 8, BPR / 8, NB, 4, PRO, 2>(p, stream);
            return launch_lane_gemv<EPI, 8, BPR / 8, NB, 4, PRO, 1>(p, stream);
        }
        else if constexpr (C16 == T16) return launch_lane_gemv<EPI, 16, T16, NB, 4, PRO, 1>(p, stream);
        else return launch_lane_gemv<EPI, 16, C16, NB, 4, PRO, 2, T16>(p, stream);
    }
    if constexpr (C16 == T16) {
        if (q32) return launch_lane_gemv<EPI, 16, T16, NB, 8, PRO>(p, stream);
        // an in-kernel RMSNorm / quantisation prologue is shared by four waves
        return launch_lane_gemv<EPI, 16, T16, NB, PRO == kProQx ? 1 : 4, PRO>(p, stream);
    } else {
        if (q32) return launch_lane_gemv<EPI, 16, C16, NB, 8, PRO, 2, T16>(p, stream);
        return launch_lane_gemv<EPI, 16, C16, NB, 1, PRO, 2, T16>(p, stream);
    }
}

template <int EPI, int NB, int PRO>
static hipError_t try_lane_gemv(GemvParams& p, hipStream_t stream, bool* used) {
    *used = true;
    switch (p.bpr) {
        // Qwen3 0.6B (1024 / 2048 / 3072 columns), 4B (2560 / 4096 / 9728), 8B (4096 / 12288)
        case 32: return launch_lane_gemv_sized<EPI, 32, NB, PRO>(p, stream);
        case 64: return launch_lane_gemv_sized<EPI, 64, NB, PRO>(p, stream);
        case 80: return launch_lane_gemv_sized<EPI, 80, NB, PRO>(p, stream);
        case 96: return launch_lane_gemv_sized<EPI, 96, NB, PRO>(p, stream);
        case 128: return launch_lane_gemv_sized<EPI, 128, NB, PRO>(p, stream);
        case 304: return launch_lane_gemv_sized<EPI, 304, NB, PRO>(p, stream);
        case 384: return launch_lane_gemv_sized<EPI, 384, NB, PRO>(p, stream);
        default: *used = false; return hipSuccess;
    }
}

}  // namespace mantle
