// gemm_w4a8.hip -- the k4 W4A8 product over many activation vectors on int8
// MFMA (v_mfma_i32_16x16x32_i8): the batched GEMV (config 2 at batch 8) and the
// projections of a whole prompt (batched prefill).
//
// Arithmetic: exactly the CPU path's (matVecRangeQuantCached,
// internal/backend/simd/matvec_quant.go:256-296) for every (row, vector):
// y = sum over blocks b, in order, of float32(dot_b) * (s_w[r,b] * s_x[b]),
// where dot_b is the exact int32 dot of the block's 32 k4 weights with the
// vector's 32 int8 activations, and a block with a zero scale is skipped.  The
// matrix core gives exact integer dots; each lane then applies its block's
// terms to its own running sums, in block order: the same roundings as the CPU
// loop, bit for bit.  The weights enter as bytes of 16 q (nibble masks, as the
// lane GEMV does); the dot is then 16 * dot_b and >> 4 is exact.
//
// MFMA operand layout (16x16x32 i8): lane l holds A[row l%16][k 8(l/16)..+7]
// and B[k 8(l/16)..+7][column l%16]; the result D[row 4(l/16)+i][column l%16]
// in its register i.  The k order inside a block is free as long as A and B
// agree: the low dword of a lane's operands holds elements 8g+{0,2,4,6}, the
// high dword 8g+{1,3,5,7} -- the even / odd nibble masks of weight word g, and
// dwords g and 4+g of the permuted int8 activation block (the layout
// quantize_vec writes).
//
// Wide form (n > 8): column = activation vector, one MFMA per block and 16x16
// tile.  Pair form (n <= 8): columns 0-7 are the 8 vectors at block b, columns
// 8-15 the same vectors at block b+1; k groups 0-1 carry block b and 2-3 block
// b+1, with zeros in B where column and k group disagree, so two MFMAs (the two
// halves of the blocks, summed in the integer accumulator) give 16 rows x 8
// vectors x 2 blocks of dots with no idle column.  The odd block's term moves
// to the even column's lane by DPP, which adds it after the even one.
//
// Tiling: four waves per workgroup; wave (wr, wt) owns WR 16-row tiles x WT
// 16-column tiles.  Chunks of 8 blocks (128 weight bytes per row, 256
// activation bytes per vector) are staged in LDS, the next chunk's global loads
// in flight while the current one is multiplied; the weight block scales of
// the chunk are computed once per (row, block) while staging.  A chunk whose
// scales are all finite drops the skip test: a zero scale then gives a term of
// +-0, which leaves the running sum unchanged, as the skip does.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "device_common.h"
#include "gemv.h"

namespace mantle {

typedef int v4i32 __attribute__((ext_vector_type(4)));
static constexpr int kGemmKC = 8;  // blocks per chunk

struct GemmArgs {
    K4Mat w;
    int bpr;
    const int8_t* qx;  // [n][bpr*32] permuted int8 activations
    const float* xs;   // [n][bpr] their block scales
    float* y;          // y[v * ldy + row]
    int n, ldy;
    int epi;           // kEpiStore or kEpiResAdd (y += sum)
    // wide form, several matrices on the same activations in one launch: row
    // tiles [tile_end[m-1], tile_end[m]) of the grid are matrix ws[m] into ys[m]
    int nmat;
    K4Mat ws[3];
    float* ys[3];
    int tile_end[3];
};

__device__ __forceinline__ float dpp_from_upper8(float v) {  // lane i <- lane i+8 within its row of 16
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true));
}

__device__ __forceinline__ bool finite_f(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

// The int8 MFMA sees each weight as 16q, so its block dot d is 16 * dot.  The
// fast path takes d as is against s_w / 16: k4_scale16_hw is the block scale
// f16(super) * u6/32 divided by 16 (u6 / 512: the product of the f16 super and
// u6 stays exact in fp32 and is at least 2^-23, so no rounding either way).
// The super decodes through the hardware conversion: this file is built with
// f16 denormals flushed, so a subnormal super becomes +-0 as Mantle's decode
// makes it (NaN payloads may differ; NaN stays NaN).  For an activation scale
// s_x that is 0 or within [2^-100, 2^100], (s_w/16)*s_x is (s_w*s_x)/16 exactly
// (no underflow or overflow), and float(d) * that equals float(dot) *
// (s_w*s_x) (d = 16*dot is exact in fp32): the same bits as the CPU's term with
// one instruction (the shift) fewer.  Other scales take the exact form
// float(d >> 4) * ((16*(s_w/16)) * s_x) on the kernels' zero-test path.
__device__ __forceinline__ float k4_scale16_hw(uint16_t sup_bits, uint8_t sub) {
    const float sup = __half2float(__ushort_as_half(sup_bits));
    const uint32_t u6 = sub & 0x3Fu;
    if (sup == 0.0f || u6 == 0) return 0.0f;
    return sup * ((float)u6 * 0.001953125f);
}
__device__ __forceinline__ bool fast_xscale(float sx) {
    const float m = fabsf(sx);
    return sx == 0.0f || (m >= 0x1p-100f && m <= 0x1p100f);
}

template <int WR, int WT, int NWR, int NWT, bool PAIR>
__global__ __launch_bounds__(256) void k4_gemm_w4a8_mfma(GemmArgs a) {
    static_assert(NWR * NWT == 4, "four waves");
    static_assert(!PAIR || (WT == 1 && NWT == 1), "the pair form has one 16-column tile");
    constexpr int TR = NWR * WR * 16;            // rows per workgroup
    constexpr int TT = PAIR ? 8 : NWT * WT * 16;  // vectors per workgroup
    constexpr int WN_ITEMS = TR * 8 / 256;       // 16-byte weight pieces per thread per chunk
    constexpr int XQ_ITEMS = (TT * 16 + 255) / 256;
    constexpr int SW_ITEMS = (TR * kGemmKC + 255) / 256;
    constexpr int XS_ITEMS = (TT * kGemmKC + 255) / 256;
    static_assert(WN_ITEMS >= 1, "tile too small for the cooperative loads");
    // row / vector pitches padded by 16 bytes: the 16 lanes of one k group read
    // 16 different rows (vectors) and land in distinct banks
    constexpr int WP = 36, XP = 68;
    constexpr int XQ_WORDS = TT * XP + (PAIR ? 72 : 0);  // the pair form's zero operand at the end
    __shared__ __align__(16) uint32_t wn[TR * WP];       // [row][8 blocks x 16 bytes + pad]
    __shared__ __align__(16) uint32_t xq[XQ_WORDS];      // [vector][8 blocks x 32 bytes + pad]
    __shared__ __align__(16) float swT[kGemmKC * TR];    // [block][row]
    __shared__ __align__(16) float xsT[kGemmKC * TT];    // [block][vector]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tile = (int)blockIdx.x;
    K4Mat W = a.w;  // this workgroup's matrix and output (locals: the arguments stay in registers)
    float* Y = a.y;
    if (!PAIR && a.nmat > 1) {
        const int m = tile < a.tile_end[0] ? 0 : (tile < a.tile_end[1] ? 1 : 2);
        tile -= m == 0 ? 0 : (m == 1 ? a.tile_end[0] : a.tile_end[1]);
        W = m == 0 ? a.ws[0] : (m == 1 ? a.ws[1] : a.ws[2]);
        Y = m == 0 ? a.ys[0] : (m == 1 ? a.ys[1] : a.ys[2]);
    }
    const int row0 = tile * TR, v0 = (int)blockIdx.y * TT;
    const int wr0 = (wave / NWT) * WR * 16, wt0 = (wave % NWT) * WT * 16;
    const int rows = W.rows, bpr = a.bpr, spr = (bpr + 7) / 8;
    const int kq = lane >> 4, l16 = lane & 15;
    if constexpr (PAIR) {
        if (tid < 72) xq[TT * XP + tid] = 0u;
    }

    // staging registers of one chunk
    uint32_t rw[WN_ITEMS][4], rx[XQ_ITEMS][4];
    uint32_t rsub[SW_ITEMS];
    uint16_t rsup[SW_ITEMS];
    float rxs[XS_ITEMS];
    auto load_chunk = [&](int b0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < WN_ITEMS; i++) {
            const int it = tid + 256 * i, r = it >> 3, part = it & 7;
            const int gr = row0 + r < rows ? row0 + r : rows - 1;
            const uint4 u = reinterpret_cast<const uint4*>(W.nib)[(size_t)gr * bpr + b0 + part];
            rw[i][0] = u.x; rw[i][1] = u.y; rw[i][2] = u.z; rw[i][3] = u.w;
        }
#pragma unroll
        for (int i = 0; i < XQ_ITEMS; i++) {
            const int it = tid + 256 * i, v = (it >> 4) < TT ? it >> 4 : TT - 1, part = it & 15;
            const int gv = v0 + v < a.n ? v0 + v : a.n - 1;
            const uint4 u = reinterpret_cast<const uint4*>(a.qx + (size_t)gv * bpr * 32 + (size_t)b0 * 32)[part];
            rx[i][0] = u.x; rx[i][1] = u.y; rx[i][2] = u.z; rx[i][3] = u.w;
        }
#pragma unroll
        for (int i = 0; i < SW_ITEMS; i++) {
            const int it = tid + 256 * i;
            const int r = it / kGemmKC < TR ? it / kGemmKC : 0, blk = it % kGemmKC;
            const int gr = row0 + r < rows ? row0 + r : rows - 1;
            rsub[i] = W.sub[(size_t)gr * bpr + b0 + blk];
            rsup[i] = W.sup[(size_t)gr * spr + ((b0 + blk) >> 3)];
        }
#pragma unroll
        for (int i = 0; i < XS_ITEMS; i++) {
            const int it = tid + 256 * i;
            const int v = it / kGemmKC < TT ? it / kGemmKC : 0, blk = it % kGemmKC;
            const int gv = v0 + v < a.n ? v0 + v : a.n - 1;
            rxs[i] = a.xs[(size_t)gv * bpr + b0 + blk];
        }
    };
    // stores the staged chunk; true if one of its scales is not finite
    auto store_chunk = [&]() __attribute__((always_inline)) -> bool {
        bool odd = false;
#pragma unroll
        for (int i = 0; i < WN_ITEMS; i++) {
            const int it = tid + 256 * i;
            *reinterpret_cast<uint4*>(wn + (it >> 3) * WP + (it & 7) * 4) = make_uint4(rw[i][0], rw[i][1], rw[i][2], rw[i][3]);
        }
#pragma unroll
        for (int i = 0; i < XQ_ITEMS; i++) {
            const int it = tid + 256 * i;
            if (TT * 16 % 256 == 0 || it < TT * 16) *reinterpret_cast<uint4*>(xq + (it >> 4) * XP + (it & 15) * 4) = make_uint4(rx[i][0], rx[i][1], rx[i][2], rx[i][3]);
        }
#pragma unroll
        for (int i = 0; i < SW_ITEMS; i++) {
            const int it = tid + 256 * i;
            if (TR * kGemmKC % 256 == 0 || it < TR * kGemmKC) {
                const float s = k4_scale16_hw(rsup[i], (uint8_t)rsub[i]);
                swT[(it % kGemmKC) * TR + it / kGemmKC] = s;
                odd |= !finite_f(s);
            }
        }
#pragma unroll
        for (int i = 0; i < XS_ITEMS; i++) {
            const int it = tid + 256 * i;
            if (TT * kGemmKC % 256 == 0 || it < TT * kGemmKC) {
                xsT[(it % kGemmKC) * TT + it / kGemmKC] = rxs[i];
                odd |= !finite_f(rxs[i]) || !fast_xscale(rxs[i]);
            }
        }
        return odd;
    };

    float acc[WR][WT][4];
#pragma unroll
    for (int rt = 0; rt < WR; rt++)
#pragma unroll
        for (int tt = 0; tt < WT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[rt][tt][i] = 0.0f;

    // pair form: this lane's column is (vector c & 7, block parity c >> 3); its
    // k group carries parity kq >> 1; B is zero where the two differ
    const int par = l16 >> 3;
    const uint32_t* xbase;
    if constexpr (PAIR)
        xbase = (kq >> 1) == par ? xq + (l16 & 7) * XP + par * 8 + (kq & 1) : xq + TT * XP;
    else
        xbase = xq + (wt0 + l16) * XP + kq;

    // The chunk in LDS, with (SKIP) or without the zero-scale test.
    auto chunk_math = [&](auto skip_tag) __attribute__((always_inline)) {
        constexpr bool SKIP = decltype(skip_tag)::value;
        // The MFMAs of a group of blocks are issued together into separate
        // results, then their terms applied: the matrix core's latency overlaps
        // the previous results' arithmetic instead of stalling each step.
        if constexpr (!PAIR) {
            constexpr int G = 2;  // blocks per group
#pragma unroll
            for (int b0 = 0; b0 < kGemmKC; b0 += G) {
                v4i32 d[G][WR][WT];
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const int b = b0 + g;
                    long av[WR], bv[WT];
#pragma unroll
                    for (int rt = 0; rt < WR; rt++) {
                        const uint32_t w = wn[(wr0 + rt * 16 + l16) * WP + b * 4 + kq];
                        const uint32_t e = (w << 4) & 0xF0F0F0F0u, o = w & 0xF0F0F0F0u;  // 16 q, even / odd nibbles
                        av[rt] = (long)((uint64_t)e | ((uint64_t)o << 32));
                    }
#pragma unroll
                    for (int tt = 0; tt < WT; tt++) {
                        const uint32_t* xb = xbase + tt * 16 * XP + b * 8;
                        bv[tt] = (long)((uint64_t)xb[0] | ((uint64_t)xb[4] << 32));
                    }
#pragma unroll
                    for (int rt = 0; rt < WR; rt++)
#pragma unroll
                        for (int tt = 0; tt < WT; tt++) {
                            const v4i32 zero = {0, 0, 0, 0};
                            d[g][rt][tt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[rt], bv[tt], zero, 0, 0, 0);
                        }
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const int b = b0 + g;
#pragma unroll
                    for (int rt = 0; rt < WR; rt++) {
                        const float4 sw4 = *reinterpret_cast<const float4*>(&swT[b * TR + wr0 + rt * 16 + 4 * kq]);
                        const float sw[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
#pragma unroll
                        for (int tt = 0; tt < WT; tt++) {
                            const float sx = xsT[b * TT + wt0 + tt * 16 + l16];
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                float term;
                                if constexpr (SKIP) {
                                    term = (float)(d[g][rt][tt][i] >> 4) * ((16.0f * sw[i]) * sx);
                                    term = sw[i] != 0.0f && sx != 0.0f ? term : 0.0f;
                                } else {
                                    term = (float)d[g][rt][tt][i] * (sw[i] * sx);
                                }
                                acc[rt][tt][i] = acc[rt][tt][i] + term;
                            }
                        }
                    }
                }
            }
        } else {
            constexpr int NPAIR = kGemmKC / 2;
            v4i32 d[NPAIR][WR];
#pragma unroll
            for (int pr = 0; pr < NPAIR; pr++) {  // blocks 2pr (columns 0-7) and 2pr+1 (columns 8-15)
                const int b = 2 * pr;
                long av[WR][2], bv[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {  // half h: elements 16h .. 16h+15 of each block
#pragma unroll
                    for (int rt = 0; rt < WR; rt++) {
                        const uint32_t w = wn[(wr0 + rt * 16 + l16) * WP + (b + (kq >> 1)) * 4 + 2 * h + (kq & 1)];
                        const uint32_t e = (w << 4) & 0xF0F0F0F0u, o = w & 0xF0F0F0F0u;
                        av[rt][h] = (long)((uint64_t)e | ((uint64_t)o << 32));
                    }
                    const uint32_t* xb = xbase + b * 8 + 2 * h;
                    bv[h] = (long)((uint64_t)xb[0] | ((uint64_t)xb[4] << 32));
                }
#pragma unroll
                for (int rt = 0; rt < WR; rt++) {
                    const v4i32 zero = {0, 0, 0, 0};
                    d[pr][rt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[rt][0], bv[0], zero, 0, 0, 0);
                    d[pr][rt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[rt][1], bv[1], d[pr][rt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int pr = 0; pr < NPAIR; pr++) {
                const int b = 2 * pr;
                const float sx = xsT[(b + par) * TT + (l16 & 7)];
#pragma unroll
                for (int rt = 0; rt < WR; rt++) {
                    const float4 sw4 = *reinterpret_cast<const float4*>(&swT[(b + par) * TR + wr0 + rt * 16 + 4 * kq]);
                    const float sw[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float term;
                        if constexpr (SKIP) {
                            term = (float)(d[pr][rt][i] >> 4) * ((16.0f * sw[i]) * sx);
                            term = sw[i] != 0.0f && sx != 0.0f ? term : 0.0f;
                        } else {
                            term = (float)d[pr][rt][i] * (sw[i] * sx);
                        }
                        // block b's term, then block b+1's from the lane 8 columns up
                        const float up = dpp_from_upper8(term);
                        acc[rt][0][i] = acc[rt][0][i] + term;
                        acc[rt][0][i] = acc[rt][0][i] + up;
                    }
                }
            }
        }
    };

    const int nch = bpr / kGemmKC;
    load_chunk(0);
    for (int c = 0; c < nch; c++) {
        __syncthreads();  // the previous chunk's readers are done
        const bool odd = store_chunk();
        const bool any_odd = __syncthreads_or(odd);
        load_chunk((c + 1 < nch ? c + 1 : c) * kGemmKC);  // in flight while this chunk is multiplied (the last re-reads itself)
        if (any_odd)
            chunk_math(std::true_type{});
        else
            chunk_math(std::false_type{});
    }
#pragma unroll
    for (int rt = 0; rt < WR; rt++)
#pragma unroll
        for (int tt = 0; tt < WT; tt++) {
            const int col = PAIR ? l16 : wt0 + tt * 16 + l16;
            const int v = v0 + col;
            if ((PAIR && l16 >= 8) || v >= a.n) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = row0 + wr0 + rt * 16 + 4 * kq + i;
                if (r >= rows) continue;
                float* dst = Y + (size_t)v * a.ldy + r;
                *dst = a.epi == kEpiResAdd ? *dst + acc[rt][tt][i] : acc[rt][tt][i];
            }
        }
}

// Batched GEMV (n <= 8) in the pair form with the weights read straight into
// registers: every wave owns its own rows, so staging them in LDS would buy no
// reuse.  Lane (row l%16, k group kq) loads, for block quad Q, the whole block
// 4Q + kq of its row (16 bytes); its word w is the lane's A operand of the
// quad's MFMAs w (one per half).  B for column c (vector c%8, parity c/8) and
// half h is that word's activations (permuted dwords w and 4+w of block
// 4Q + kq) where kq == 2h + c/8, else zero: half h yields the block dots of
// blocks 4Q + 2h (columns 0-7) and 4Q + 2h + 1 (columns 8-15), the pair 2Q + h.  The 8 activation
// vectors and their block scales sit in LDS for the whole row; the weight block
// scales of each group of 8 blocks are computed by the lanes that loaded the
// row (blocks 2kq, 2kq+1) and pass through a wave-private LDS tile into the
// result layout (rows 4kq..4kq+3).  Groups of 8 blocks stream through a ring
// of D register slots, D-1 groups ahead of the arithmetic.
template <int NG, int RT, int D>
__global__ __launch_bounds__(256) void k4_gemv8_w4a8_mfma(GemmArgs a) {
    constexpr int BPR = NG * kGemmKC;
    constexpr int COLS = BPR * 32;
    constexpr int XPW = BPR * 8 + 39;  // words per staged vector: an odd pitch spreads the 8 vectors over the banks
    extern __shared__ __align__(16) uint32_t gsm[];
    uint32_t* xq = gsm;                                              // [8][XPW]
    float* xsT = reinterpret_cast<float*>(gsm + 8 * XPW);            // [BPR][8]
    float* swW = xsT + BPR * 8;                                      // [4 waves][RT][8 blocks][16 rows]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = lane >> 4, l16 = lane & 15;
    const int rows = a.w.rows, n = a.n;
    // Row tiles of RT*16 rows go to the waves in turn (wave w of workgroup b
    // takes tiles 4b+w, 4b+w + 4*grid, ...); the group stream runs on across
    // tile boundaries, so the next tile's first groups load during this one's
    // last.  D divides NG, so group g of any tile uses slot g % D.
    const int ntiles = (rows + RT * 16 - 1) / (RT * 16);
    const int tstride = (int)gridDim.x * 4;
    uint4 wbuf[D][RT][2];
    uint32_t sbuf[D][RT];
    uint32_t hbuf[D][RT];
    auto issue = [&](int tile, int g, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int r0 = tile * RT * 16 + rt * 16 + l16;
            const int r = r0 < rows ? r0 : rows - 1;
            const uint4* wp = reinterpret_cast<const uint4*>(a.w.nib + (size_t)r * BPR * 16) + kq;
            const uint8_t* sp = a.w.sub + (size_t)r * BPR + 2 * kq;
#pragma unroll
            for (int qq = 0; qq < 2; qq++) wbuf[slot][rt][qq] = wp[4 * (2 * g + qq)];
            sbuf[slot][rt] = (uint32_t)sp[kGemmKC * g] | ((uint32_t)sp[kGemmKC * g + 1] << 8);
            hbuf[slot][rt] = a.w.sup[(size_t)r * NG + g];
        }
    };
    int tile = (int)blockIdx.x * 4 + wave;
    if (tile < ntiles) {
#pragma unroll
        for (int g = 0; g < D - 1; g++) issue(tile, g, g);
    }

    // The activations: every load issued before the first store (a loop of
    // load-store pairs would wait out the memory latency once per trip).
    constexpr int XV = BPR * 8 / 4;                 // uint4 per vector
    constexpr int XI = (8 * XV + 255) / 256;        // uint4 per thread
    constexpr int SI = (BPR * 8 + 255) / 256;       // scales per thread
    uint4 xr[XI];
    float sr[SI];
#pragma unroll
    for (int k = 0; k < XI; k++) {
        const int i = tid + 256 * k;
        const int v = i / XV < 8 ? i / XV : 7, q = i % XV;
        const int gv = v < n ? v : n - 1;
        xr[k] = reinterpret_cast<const uint4*>(a.qx + (size_t)gv * COLS)[q];
    }
#pragma unroll
    for (int k = 0; k < SI; k++) {
        const int i = (tid + 256 * k) < BPR * 8 ? tid + 256 * k : 0;
        const int b = i >> 3, v = i & 7;
        sr[k] = a.xs[(size_t)(v < n ? v : n - 1) * BPR + b];
    }
    bool odd = false;
#pragma unroll
    for (int k = 0; k < XI; k++) {
        const int i = tid + 256 * k;
        if (8 * XV % 256 == 0 || i < 8 * XV) {
            uint32_t* dst = xq + (i / XV) * XPW + 4 * (i % XV);
            dst[0] = xr[k].x;
            dst[1] = xr[k].y;
            dst[2] = xr[k].z;
            dst[3] = xr[k].w;
        }
    }
#pragma unroll
    for (int k = 0; k < SI; k++) {
        const int i = tid + 256 * k;
        if (BPR * 8 % 256 == 0 || i < BPR * 8) {
            xsT[i] = sr[k];
            odd |= !finite_f(sr[k]) || !fast_xscale(sr[k]);
        }
    }
    const bool odd_x = __syncthreads_or(odd);

    const int par = l16 >> 3, vec = l16 & 7;
    const uint64_t bmask0 = kq == par ? ~0ull : 0ull, bmask1 = kq == 2 + par ? ~0ull : 0ull;
    const uint32_t* xrow = xq + vec * XPW + kq * 8;
    float* sww = swW + wave * RT * 128;

    for (; tile < ntiles; tile += tstride) {
        const int next = tile + tstride;
        float acc[RT][4];
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[rt][i] = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int ga = g + D - 1;  // the group loaded now
            if (ga < NG)
                issue(tile, ga, ga % D);
            else if (next < ntiles)
                issue(next, ga - NG, ga % D);
            const int slot = g % D;
            bool bad = false;
    #pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const float s0 = k4_scale16_hw((uint16_t)hbuf[slot][rt], (uint8_t)sbuf[slot][rt]);
                const float s1 = k4_scale16_hw((uint16_t)hbuf[slot][rt], (uint8_t)(sbuf[slot][rt] >> 8));
                sww[rt * 128 + (2 * kq) * 16 + l16] = s0;
                sww[rt * 128 + (2 * kq + 1) * 16 + l16] = s1;
                bad |= !finite_f(s0) || !finite_f(s1);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            v4i32 d[4][RT];  // pair jj = 2 qq + h
    #pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int Q = 2 * g + qq;
    #pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const v4i32 zero = {0, 0, 0, 0};
                    d[2 * qq][rt] = zero;
                    d[2 * qq + 1][rt] = zero;
                }
    #pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint64_t xv = (uint64_t)xrow[32 * Q + w] | ((uint64_t)xrow[32 * Q + w + 4] << 32);
                    const long b0 = (long)(xv & bmask0), b1 = (long)(xv & bmask1);
    #pragma unroll
                    for (int rt = 0; rt < RT; rt++) {
                        const uint4 wq = wbuf[slot][rt][qq];
                        const uint32_t ww = w == 0 ? wq.x : (w == 1 ? wq.y : (w == 2 ? wq.z : wq.w));
                        const long aw = (long)((uint64_t)((ww << 4) & 0xF0F0F0F0u) | ((uint64_t)(ww & 0xF0F0F0F0u) << 32));
                        d[2 * qq][rt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, b0, d[2 * qq][rt], 0, 0, 0);
                        d[2 * qq + 1][rt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, b1, d[2 * qq + 1][rt], 0, 0, 0);
                    }
                }
            }
            auto terms = [&](auto skip_tag) __attribute__((always_inline)) {
                constexpr bool SKIP = decltype(skip_tag)::value;
    #pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float sx = xsT[(kGemmKC * g + 2 * jj + par) * 8 + vec];
    #pragma unroll
                    for (int rt = 0; rt < RT; rt++) {
                        const float4 sw4 = *reinterpret_cast<const float4*>(&sww[rt * 128 + (2 * jj + par) * 16 + 4 * kq]);
                        const float sw[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
    #pragma unroll
                        for (int i = 0; i < 4; i++) {
                            float term;
                            if constexpr (SKIP) {
                                term = (float)(d[jj][rt][i] >> 4) * ((16.0f * sw[i]) * sx);
                                term = sw[i] != 0.0f && sx != 0.0f ? term : 0.0f;
                            } else {
                                term = (float)d[jj][rt][i] * (sw[i] * sx);
                            }
                            const float up = dpp_from_upper8(term);
                            acc[rt][i] = acc[rt][i] + term;
                            acc[rt][i] = acc[rt][i] + up;
                        }
                    }
                }
            };
            if (odd_x || __any(bad))
                terms(std::true_type{});
            else
                terms(std::false_type{});
            // the next group's scales overwrite this tile
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        if (l16 < 8 && vec < n) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = tile * RT * 16 + rt * 16 + 4 * kq + i;
                    if (r >= rows) continue;
                    float* dst = a.y + (size_t)vec * a.ldy + r;
                    *dst = a.epi == kEpiResAdd ? *dst + acc[rt][i] : acc[rt][i];
                }
        }
    }
}

template <int NG, int RT>
static void launch_gemv8_rt(const GemmArgs& a, hipStream_t stream) {
    constexpr int D = NG % 4 == 0 ? 4 : (NG % 3 == 0 ? 3 : (NG % 2 == 0 ? 2 : 1));
    constexpr int BPR = NG * kGemmKC;
    const size_t smem = sizeof(uint32_t) * (8 * (BPR * 8 + 39) + BPR * 8 + 4 * RT * 128);
    const int ntiles = (a.w.rows + RT * 16 - 1) / (RT * 16);
    constexpr int per_cu = 3;  // workgroups per CU; each stages the activations once
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int want = (ntiles + 3) / 4;
    const int grid = want < per_cu * cus ? want : per_cu * cus;
    hipLaunchKernelGGL((k4_gemv8_w4a8_mfma<NG, RT, D>), dim3(grid), dim3(256), smem, stream, a);
}

template <int NG>
static void launch_gemv8(const GemmArgs& a, hipStream_t stream) {
    launch_gemv8_rt<NG, 1>(a, stream);
}

hipError_t launch_k4_gemm_w4a8_multi(const K4Mat* mats, float* const* ys, int nmat, int cols, const int8_t* qx,
                                     const float* xs, int n, int ldy, GemvEpi epi, hipStream_t stream);

// y[v][row] (+)= W x_v for n activation vectors already quantised (qx / xs as
// quantize_vec writes them), on int8 MFMA.  Blocks per row a multiple of 8.
hipError_t launch_k4_gemm_w4a8(const K4Mat& w, int cols, const int8_t* qx, const float* xs, int n, float* y, int ldy,
                               GemvEpi epi, hipStream_t stream) {
    const int bpr = (cols + 31) / 32;
    if (!w.nib || !w.sub || !w.sup || w.rows <= 0 || cols != bpr * 32 || bpr % kGemmKC || !qx || !xs || !y ||
        n <= 0 || ldy < w.rows || (epi != kEpiStore && epi != kEpiResAdd))
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.w = w;
    a.bpr = bpr;
    a.qx = qx;
    a.xs = xs;
    a.y = y;
    a.n = n;
    a.ldy = ldy;
    a.epi = epi;
    const bool aligned = ((uintptr_t)qx & 15) == 0;
    if (n <= 8 && aligned && bpr <= 16 * kGemmKC) {  // a batched GEMV, weights straight to registers
        switch (bpr / kGemmKC) {
            case 1: launch_gemv8<1>(a, stream); break;
            case 2: launch_gemv8<2>(a, stream); break;
            case 3: launch_gemv8<3>(a, stream); break;
            case 4: launch_gemv8<4>(a, stream); break;
            case 5: launch_gemv8<5>(a, stream); break;
            case 6: launch_gemv8<6>(a, stream); break;
            case 7: launch_gemv8<7>(a, stream); break;
            case 8: launch_gemv8<8>(a, stream); break;
            case 9: launch_gemv8<9>(a, stream); break;
            case 10: launch_gemv8<10>(a, stream); break;
            case 11: launch_gemv8<11>(a, stream); break;
            case 12: launch_gemv8<12>(a, stream); break;
            case 13: launch_gemv8<13>(a, stream); break;
            case 14: launch_gemv8<14>(a, stream); break;
            case 15: launch_gemv8<15>(a, stream); break;
            default: launch_gemv8<16>(a, stream); break;
        }
    } else if (n <= 8) {  // the pair form through LDS, 128 rows per workgroup
        dim3 grid((w.rows + 127) / 128, 1);
        hipLaunchKernelGGL((k4_gemm_w4a8_mfma<2, 1, 4, 1, true>), grid, dim3(256), 0, stream, a);
    } else {
        return launch_k4_gemm_w4a8_multi(&w, &y, 1, cols, qx, xs, n, ldy, epi, stream);
    }
    return hipGetLastError();
}

// The wide form for up to three matrices of the same width on one set of
// activations (Q / K / V, gate / up), one launch: 64-row tiles, or 32-row ones
// where 64-row tiles would leave the chip less than twice covered.
hipError_t launch_k4_gemm_w4a8_multi(const K4Mat* mats, float* const* ys, int nmat, int cols, const int8_t* qx,
                                     const float* xs, int n, int ldy, GemvEpi epi, hipStream_t stream) {
    const int bpr = (cols + 31) / 32;
    if (!mats || !ys || nmat < 1 || nmat > 3 || cols != bpr * 32 || bpr % kGemmKC || !qx || !xs || n <= 0 ||
        (epi != kEpiStore && epi != kEpiResAdd))
        return hipErrorInvalidValue;
    int total64 = 0;
    for (int m = 0; m < nmat; m++) {
        if (!mats[m].nib || !mats[m].sub || !mats[m].sup || mats[m].rows <= 0 || !ys[m] || ldy < mats[m].rows)
            return hipErrorInvalidValue;
        total64 += (mats[m].rows + 63) / 64;
    }
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int ncol = (n + 63) / 64;
    const int TR = total64 * ncol < 2 * cus ? 32 : 64;
    GemmArgs a{};
    a.w = mats[0];
    a.y = ys[0];
    a.bpr = bpr;
    a.qx = qx;
    a.xs = xs;
    a.n = n;
    a.ldy = ldy;
    a.epi = epi;
    a.nmat = nmat;
    int tiles = 0;
    for (int m = 0; m < nmat; m++) {
        a.ws[m] = mats[m];
        a.ys[m] = ys[m];
        tiles += (mats[m].rows + TR - 1) / TR;
        a.tile_end[m] = tiles;
    }
    for (int m = nmat; m < 3; m++) a.tile_end[m] = tiles;
    const dim3 grid(tiles, ncol);
    if (TR == 32)
        hipLaunchKernelGGL((k4_gemm_w4a8_mfma<1, 2, 2, 2, false>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((k4_gemm_w4a8_mfma<2, 2, 2, 2, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mantle
