// prefill_attention.hip -- causal GQA attention over a whole prompt (bf16
// inputs) on MFMA, gfx950 v_mfma_f32_32x32x16_f16: the one dense contraction
// of the path.
//
// Mantle prefills k4 models token by token: each position runs RunAttnHeads
// over the keys 0..t of the cache (internal/backend/simd/runtime_prefill.go:11-30,
// attnpool.go:77-153), after RoPE on q and k (ops_avx512.go:132-191).  This
// kernel produces the same outputs for every position at once: out[t] =
// softmax(q_t . K[0..t] * scale) V[0..t] per query head, K/V of its KV group.
// Inputs are bf16.  The MFMA operands are fp16 (same rate as bf16): q and k
// after RoPE, V and the probabilities.  With bf16 operands the rounding of the
// RoPE'd q / k alone put 0.2% of outputs past max-abs 1e-3 + rel 1e-2 of the
// CPU result (5e-3 worst), and bf16 probabilities put the worst output at
// 1.8x that tolerance (a float64 simulation at S = 512); fp16 keeps them under
// 6e-4.  fp16's range is narrower than bf16's: every operand is scaled by a
// power of two into [2^14, 2^15] before the conversion -- q per query (folded
// into that lane's softmax scale), K and V per 32-key tile of a KV head (K's
// factor into the tile's softmax scale; V's through the tile's probabilities,
// relative to the largest V factor the workgroup sees, which multiplies the
// output).  Power-of-two scaling commutes with rounding, so the scores are the
// same bits the unscaled fp16 operands give wherever those neither overflow
// nor underflow; values more than 2^28 below their block's largest one still
// fall into fp16's subnormals, and a tile's probabilities move down by its V
// factor (negligible ones first reach the subnormals).  Accumulation and the softmax are fp32: the result matches the CPU
// path within the tolerance above, not bit for bit.
//
// Layout (queries are MFMA columns throughout):
//  * S^T = K . Q^T per 32-key tile: A = K rows from LDS (RoPE'd by the
//    pre-pass), B = this wave's 32 queries, RoPE'd once into registers.  Lane l
//    then holds query l % 32 and 16 of the tile's keys, so each query's max and
//    sum are one lane's 16 values plus one exchange with lane l ^ 32.
//  * O^T += V^T . P^T: B = P straight from the S^T registers (fp16), A = V^T
//    from LDS, its keys taken in the order the P registers hold them (the sum
//    over keys does not depend on that order).  O^T keeps the query in the
//    column too, so the online-softmax rescale is one factor per lane.
//  * A workgroup is four waves: two query heads of one KV group x 64 queries
//    (or, without GQA, one head x 128 queries); K/V tiles are staged once for
//    all four by direct global-to-LDS copies, three stages deep.
//  * A pre-pass (prefill_prep_kv) writes each 32-key tile of K (RoPE'd) and V
//    in fp16 into the caller's workspace once, already in the LDS layout the
//    operand reads want, so the attention workgroups stage plain 1 KB copies.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <math.h>
#include <stdint.h>

#include "kernels.h"
#include "phase_trace.h"

namespace mantle {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

static constexpr int kPfHd = 128;             // head_dim
static constexpr int kPfKeys = 32;            // keys per tile

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t f16_bits(float x) {  // round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) { return f16_bits(lo) | (f16_bits(hi) << 16); }

// RoPE of the pairs (x0[j], x1[j]) = elements (i + j, i + 64 + j):
// y0 = x0*c - x1*s, y1 = fma(x0, s, x1*c) (ops_avx512.go:162-190).
__device__ __forceinline__ void rope8(float (&x0)[8], float (&x1)[8], const float* cs, const float* sn) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float y0 = x0[j] * cs[j] - x1[j] * sn[j];
        const float y1 = __builtin_fmaf(x0[j], sn[j], x1[j] * cs[j]);
        x0[j] = y0;
        x1[j] = y1;
    }
}

__device__ __forceinline__ void unpack8(const u32x4v w, float (&x)[8]) {
    x[0] = bf_lo(w.x); x[1] = bf_hi(w.x); x[2] = bf_lo(w.y); x[3] = bf_hi(w.y);
    x[4] = bf_lo(w.z); x[5] = bf_hi(w.z); x[6] = bf_lo(w.w); x[7] = bf_hi(w.w);
}

struct PrefillArgs {
    const uint16_t* q;  // bf16 [seq][n_head][128]
    const uint16_t* k;  // bf16 [seq][kv_heads][128]
    const uint16_t* v;
    const float* rope_cos;  // [seq][64] or null (no RoPE)
    const float* rope_sin;
    float* out;  // fp32 [seq][n_head][128]
    // workspace, per kv head and 32-key tile (8 KB blocks laid out as the
    // attention's LDS tiles, so a tile is staged by plain 1 KB copies):
    uint16_t* kt;   // fp16 RoPE'd K: [kv][tile][16-byte chunk c of hd][key][8]
    uint16_t* vt;   // fp16 V: [kv][tile][key quad][hd][4]
    uint32_t* kfv;  // [kv][tile][2]: the K tile's power-of-two factor (float bits; stored K = K * 2^-e), the V tile's exponent e
    int seq, seq_pad, n_head, kv_heads;
    int heads_per_wg;  // 2 (GQA groups of an even size) or 1
    int q_block;       // queries per workgroup and head
    int n_qblocks;
    float scale;
    // Load balance: a query block of more than t_max key tiles is split into
    // ceil(tiles / t_max) parts (at most kPfMaxParts) of even size, so no
    // workgroup's chain of tiles is much longer than the average one.  A split
    // block leaves each part's unnormalised O^T, running max (log2 units) and
    // sum in opart [seq][n_head][kPfMaxParts][128] / mlpart [seq][n_head][kPfMaxParts][2];
    // prefill_combine_parts joins them, with the block's output factor
    // exponent vmax (below) from vmx [query block][head group].
    int t_max;
    float *opart, *mlpart;
    int* vmx;
};

static constexpr int kPfMaxParts = 4;

__device__ __forceinline__ int pf_tiles(const PrefillArgs& a, int qb) {
    return (min((qb + 1) * a.q_block, a.seq) + kPfKeys - 1) / kPfKeys;
}
__device__ __forceinline__ int pf_parts(const PrefillArgs& a, int qb) {
    const int p = (pf_tiles(a, qb) + a.t_max - 1) / a.t_max;
    return p < kPfMaxParts ? p : kPfMaxParts;
}


// op(x of lane l, x of lane l ^ 32) in every lane, the two operands in the
// same order in both lanes (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The power of two 2^e that brings a block whose max |x| is m into
// [2^14, 2^15] (fp16-safe after rounding, clear of fp16's subnormals): e = E -
// 15 for m = f * 2^E, f in [0.5, 1), clamped to [-100, 113] (bf16's largest
// values fit); 0 for an all-zero or NaN block (NaN propagates as on the CPU).
__device__ __forceinline__ int range_exp(float m) {
    if (!(m > 0.0f)) return 0;
    if (isinf(m)) return 113;
    int E;
    (void)frexpf(m, &E);
    const int e = E - 15;
    return e < -100 ? -100 : (e > 113 ? 113 : e);
}

// Max over the workgroup (256 threads) of a non-negative value; red: 4 floats.
__device__ __forceinline__ float wg_max256(float v, float* red) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Pre-pass: workgroup (kv head g, keys t0..t0+31) writes the tile's K RoPE'd
// and its V (through LDS) in fp16 in the attention's tile layouts, zeros for
// keys past seq, each scaled by the tile's power of two into fp16 range
// (factors in kfv).
__global__ __launch_bounds__(256) void prefill_prep_kv(PrefillArgs a) {
    __shared__ __align__(16) uint16_t vs[kPfHd * 40];
    __shared__ float red[8];
    const int tid = threadIdx.x;
    const int nkb = a.seq_pad / kPfKeys;
    const int g = (int)blockIdx.x / nkb, tile = (int)blockIdx.x % nkb, t0 = tile * kPfKeys;
    const int kv_row = a.kv_heads * kPfHd;
    // K: key tid/8, pairs hd [8c, 8c+8) + 64
    const int kk = tid >> 3, kc = tid & 7;
    const int t = t0 + kk;
    float x0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, x1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (t < a.seq) {
        const uint16_t* krow = a.k + (size_t)t * kv_row + g * kPfHd;
        unpack8(*reinterpret_cast<const u32x4v*>(krow + 8 * kc), x0);
        unpack8(*reinterpret_cast<const u32x4v*>(krow + 64 + 8 * kc), x1);
        if (a.rope_cos) {
            float cs[8], sn[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                cs[j] = a.rope_cos[(size_t)t * 64 + 8 * kc + j];
                sn[j] = a.rope_sin[(size_t)t * 64 + 8 * kc + j];
            }
            rope8(x0, x1, cs, sn);
        }
    }
    // V: keys 2p, 2p+1, hd [8c, 8c+8)
    const int vp = tid & 15, vc = tid >> 4;
    float e0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, e1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int ta = t0 + 2 * vp, tb = ta + 1;
    if (ta < a.seq) unpack8(*reinterpret_cast<const u32x4v*>(a.v + (size_t)ta * kv_row + g * kPfHd + 8 * vc), e0);
    if (tb < a.seq) unpack8(*reinterpret_cast<const u32x4v*>(a.v + (size_t)tb * kv_row + g * kPfHd + 8 * vc), e1);
    float km = 0.0f, vm = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        km = fmaxf(km, fmaxf(fabsf(x0[j]), fabsf(x1[j])));
        vm = fmaxf(vm, fmaxf(fabsf(e0[j]), fabsf(e1[j])));
    }
    const int ek = range_exp(wg_max256(km, red));
    const int ev = range_exp(wg_max256(vm, red + 4));
    if (tid == 0) {
        a.kfv[2 * ((size_t)g * nkb + tile)] = __float_as_uint(ldexpf(1.0f, ek));
        a.kfv[2 * ((size_t)g * nkb + tile) + 1] = (uint32_t)ev;
    }
    {
        const float f = ldexpf(1.0f, -ek);
#pragma unroll
        for (int j = 0; j < 8; j++) { x0[j] *= f; x1[j] *= f; }
    }
    {
        const float f = ldexpf(1.0f, -ev);
#pragma unroll
        for (int j = 0; j < 8; j++) { e0[j] *= f; e1[j] *= f; }
    }
    {
        u32x4v w0, w1;
        w0.x = pack_f16(x0[0], x0[1]); w0.y = pack_f16(x0[2], x0[3]);
        w0.z = pack_f16(x0[4], x0[5]); w0.w = pack_f16(x0[6], x0[7]);
        w1.x = pack_f16(x1[0], x1[1]); w1.y = pack_f16(x1[2], x1[3]);
        w1.z = pack_f16(x1[4], x1[5]); w1.w = pack_f16(x1[6], x1[7]);
        // chunk c of key kk at c * 512 + kk * 16 bytes
        uint16_t* dst = a.kt + ((size_t)g * nkb + tile) * (kPfKeys * kPfHd) + kk * 8;
        *reinterpret_cast<u32x4v*>(dst + 256 * kc) = w0;
        *reinterpret_cast<u32x4v*>(dst + 256 * (8 + kc)) = w1;
    }
#pragma unroll
    for (int j = 0; j < 8; j++)
        *reinterpret_cast<uint32_t*>(&vs[(8 * vc + j) * 40 + 2 * vp]) = pack_f16(e0[j], e1[j]);
    __syncthreads();
    // keys 4q .. 4q+3 of hd at q * 1024 + hd * 8 bytes: 16 bytes = hd pair (2p, 2p+1) of quad q
    uint16_t* vdst = a.vt + ((size_t)g * nkb + tile) * (kPfKeys * kPfHd);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int u = tid + 256 * i, q = u >> 6, hp = u & 63;
        const u32x2v r0 = *reinterpret_cast<const u32x2v*>(&vs[(2 * hp) * 40 + 4 * q]);
        const u32x2v r1 = *reinterpret_cast<const u32x2v*>(&vs[(2 * hp + 1) * 40 + 4 * q]);
        *reinterpret_cast<u32x4v*>(vdst + q * 512 + hp * 8) = u32x4v{r0.x, r0.y, r1.x, r1.y};
    }
}

// Three waves per SIMD (three workgroups per CU, 108 KB of LDS): the
// register file then holds 165 VGPRs per lane, enough without spills, and one
// wave's softmax overlaps another's MFMAs.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void attention_prefill_bf16(PrefillArgs a) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h2 = lane >> 5, l32 = lane & 31;
    const int wph = 4 / a.heads_per_wg;  // waves per head
    const int groups = a.n_head / a.heads_per_wg;
    // the longest query blocks (most keys) are dispatched first; block qb has
    // pf_parts(qb) parts per head group
    int qb = a.n_qblocks - 1, rest = (int)blockIdx.x, nparts = pf_parts(a, qb);
    while (rest >= nparts * groups) {
        rest -= nparts * groups;
        qb--;
        nparts = pf_parts(a, qb);
    }
    const int hg = rest / nparts, part = rest - hg * nparts;
    const int head = hg * a.heads_per_wg + wave / wph;
    const int kvh = head * a.kv_heads / a.n_head;
    const int q0 = qb * a.q_block;
    const int qw = q0 + (wave % wph) * 32;  // this wave's first query
    const int myq = qw + l32;               // this lane's query
    const int qc = myq < a.seq ? myq : a.seq - 1;
    const bool rope = a.rope_cos != nullptr;

    // ---- this wave's queries, RoPE'd, as MFMA B operands: qb_op[s] holds
    // hd 16s + 8*h2 + j (j < 8) of query myq
    f16x8 qop[8];
    float qfac = 1.0f;  // this query's power-of-two range factor (stored q = q * 2^-e)
    {
        const uint16_t* qrow = a.q + ((size_t)qc * a.n_head + head) * kPfHd;
        float qx[4][2][8];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int d = 16 * s + 8 * h2;
            float x0[8], x1[8];
            unpack8(*reinterpret_cast<const u32x4v*>(qrow + d), x0);
            unpack8(*reinterpret_cast<const u32x4v*>(qrow + 64 + d), x1);
            if (rope) {
                float cs[8], sn[8];
                const float* cr = a.rope_cos + (size_t)qc * 64 + d;
                const float* sr = a.rope_sin + (size_t)qc * 64 + d;
#pragma unroll
                for (int j = 0; j < 8; j++) { cs[j] = cr[j]; sn[j] = sr[j]; }
                rope8(x0, x1, cs, sn);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                qx[s][0][j] = x0[j];
                qx[s][1][j] = x1[j];
            }
        }
        float qm = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int j = 0; j < 8; j++) qm = fmaxf(qm, fmaxf(fabsf(qx[s][0][j]), fabsf(qx[s][1][j])));
        qm = fmaxf(qm, __shfl_xor(qm, 32, 64));  // the other half of the query's 128 values
        const int eq = range_exp(qm);
        const float f = ldexpf(1.0f, -eq);
        qfac = ldexpf(1.0f, eq);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                qop[s][j] = (_Float16)(qx[s][0][j] * f);
                qop[s + 4][j] = (_Float16)(qx[s][1][j] * f);
            }
    }

    // ---- tile staging: direct global -> LDS loads (global_load_lds_dwordx4)
    // of the pre-pass tiles, three stages deep (two tiles in flight while one
    // is used), no registers held.  The pre-pass lays each tile out as the
    // LDS wants it -- K chunk c of key r at c * 512 + r * 16 bytes, V keys
    // 4q .. 4q+3 of hd at q * 1024 + hd * 8 -- so a tile is eight plain 1 KB
    // copies of each, the MFMA operand reads take consecutive 16 / 8 bytes
    // per lane (no bank conflicts) and differ only by immediate offsets.  The
    // stages are separate arrays and the loop is unrolled by three, so every
    // LDS read names its stage and the compiler's memory model needs no wait
    // on the loads still in flight into the others; the waits are explicit:
    // before stage i is read, this thread's loads of tile i (all but the last
    // five issued) have landed, and the barrier then covers the other threads'.
    __shared__ __align__(16) uint16_t ks0[kPfKeys * kPfHd], ks1[kPfKeys * kPfHd], ks2[kPfKeys * kPfHd];
    __shared__ __align__(16) uint16_t vs0[kPfHd * kPfKeys], vs1[kPfHd * kPfKeys], vs2[kPfHd * kPfKeys];
    // the tile's K factor and V exponent, copied the same way (a 256-byte slot
    // per wave and stage; lane l brings word l % 2)
    __shared__ __align__(16) uint32_t fs0[4 * 64], fs1[4 * 64], fs2[4 * 64];
    const int nkb = a.seq_pad / kPfKeys;
    const int kvh_u = __builtin_amdgcn_readfirstlane(kvh);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t* kfv = a.kfv + (size_t)kvh_u * nkb * 2;
    const char* kblk = reinterpret_cast<const char*>(a.kt + (size_t)kvh_u * nkb * (kPfKeys * kPfHd));
    const char* vblk = reinterpret_cast<const char*>(a.vt + (size_t)kvh_u * nkb * (kPfKeys * kPfHd));
    typedef __attribute__((address_space(3))) void* lds_ptr;
    // five loads per thread and tile: 1 KB pieces 2 wave, 2 wave + 1 of K and V, the factor pair
    auto issue_tile = [&](int it, uint16_t* ks, uint16_t* vs, uint32_t* fs) __attribute__((always_inline)) {
        const size_t tb = (size_t)it * (kPfKeys * kPfHd * 2);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int m = 2 * wv + j;
            __builtin_amdgcn_global_load_lds(kblk + tb + m * 1024 + lane * 16, (lds_ptr)(ks + m * 512), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vblk + tb + m * 1024 + lane * 16, (lds_ptr)(vs + m * 512), 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(kfv + 2 * (size_t)it + (lane & 1), (lds_ptr)(fs + wv * 64), 4, 0, 0);
    };
    // operand reads (bytes within a stage): K chunk 2s + h2 of key l32 at
    // kx + 1024 s; V keys 16 s2 + 4 h2 (+ 8) of hd 32 t + l32 at vx + 4096 s2 + 256 t (+ 2048)
    const int kx = h2 * 512 + l32 * 16;
    const int vx = h2 * 1024 + l32 * 8;
    const int fx = wv * 256;  // this wave's factor slot (bytes)

    // ---- online softmax state of this lane's query, O^T accumulators
    f32x16 o[4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[t][i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float sl2 = a.scale * 1.4426950408889634f * qfac;  // scale * log2(e), this query's range factor

    const int kend = min(q0 + a.q_block, a.seq);  // keys this workgroup needs
    const int ntiles = (kend + kPfKeys - 1) / kPfKeys;
    // the largest V tile exponent among those tiles: the output's factor 2^vmax;
    // tile j's probabilities carry 2^(e_j - vmax) <= 1
    __shared__ int vred[4];
    int vmax;
    {
        int e = -1000;
        for (int i = tid; i < ntiles; i += 256) e = max(e, (int)kfv[2 * i + 1]);
        for (int off = 32; off > 0; off >>= 1) e = max(e, __shfl_xor(e, off, 64));
        if (lane == 0) vred[wave] = e;
        __syncthreads();
        vmax = max(max(vred[0], vred[1]), max(vred[2], vred[3]));
    }
    const int per_part = (ntiles + nparts - 1) / nparts;
    const int it0 = part * per_part, it1 = min(ntiles, it0 + per_part);
    if (it0 < it1) issue_tile(it0, ks0, vs0, fs0);
    if (it0 + 1 < it1) issue_tile(it0 + 1, ks1, vs1, fs1);
    auto tile_step = [&](int it, const uint16_t* ks, const uint16_t* vs, const uint32_t* fs, uint16_t* ks_n,
                         uint16_t* vs_n, uint32_t* fs_n) __attribute__((always_inline)) {
        // this thread's loads of tile it have landed (those of it + 1 may not have)
        if (it + 1 < it1) __builtin_amdgcn_s_waitcnt(0x0070 | 5);  // vmcnt(5) lgkmcnt(0)
        else __builtin_amdgcn_s_waitcnt(0x0070);                   // vmcnt(0) lgkmcnt(0)
        __builtin_amdgcn_s_barrier();  // ... and every thread's; stage (it + 2) % 3 is free
        if (it + 2 < it1) issue_tile(it + 2, ks_n, vs_n, fs_n);
        const uint2 fw = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(fs) + fx);
        const float kf_cur = __uint_as_float(fw.x);
        const int ve_cur = (int)fw.y;
        const int t0 = it * kPfKeys;
        if (t0 <= qw + 31) {  // some key of the tile is visible to some query of this wave
            const float sl2t = sl2 * kf_cur;  // the tile's K factor
            const int vd = ve_cur - vmax;     // its V factor relative to the output's
            // S^T = K . Q^T
            f32x16 sacc;
#pragma unroll
            for (int i = 0; i < 16; i++) sacc[i] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const f16x8 ka = *reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(ks) + kx + 1024 * s);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qop[s], sacc, 0, 0, 0);
            }
            // element i: key t0 + (i/4)*8 + 4*h2 + i%4 of query myq; the causal
            // mask only on tiles that reach past the wave's first query
            // the raw scores' maximum (scale > 0), then p = 2^(s*scale*log2e - m)
            // as one FMA per score
            float mt = -INFINITY;
            if (t0 + kPfKeys - 1 <= qw && t0 + kPfKeys <= a.seq) {
#pragma unroll
                for (int i = 0; i < 16; i++) mt = fmaxf(mt, sacc[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = t0 + (i >> 2) * 8 + 4 * h2 + (i & 3);
                    sacc[i] = key <= myq && key < a.seq ? sacc[i] : -INFINITY;
                    mt = fmaxf(mt, sacc[i]);
                }
            }
            mt = halves_max(mt);
            const float m_new = fmaxf(m_run, mt * sl2t);
            // a query with no visible key yet (a later part of a split block):
            // exponentials against 0 keep its all -inf scores at 0 instead of NaN
            const float m_exp = m_new == -INFINITY ? 0.0f : m_new;
            float ls = 0.0f;
            f16x8 pb[2];
            // V stored at a smaller scale than the output's: the probabilities
            // enter the V sum times 2^vd, the row sum without it.  For vd >= -64
            // the factor joins the exponent (2^(x + vd)) and the tile's sum is
            // scaled back by 2^-vd (exact: probabilities small enough to lose
            // bits there are below 2^-60 of the running sum, which holds a 1);
            // beyond that the probabilities are multiplied by 2^vd one by one.
            if (vd >= -64) {
                const float c = (float)vd - m_exp;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i], sl2t, c));
                    ls += pv;
                    pb[i >> 3][i & 7] = (_Float16)pv;
                }
                ls = ldexpf(ls, -vd);
            } else {
                const float vf = ldexpf(1.0f, vd);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i], sl2t, -m_exp));
                    ls += pv;
                    pb[i >> 3][i & 7] = (_Float16)(pv * vf);
                }
            }
            ls = halves_sum(ls);
            // rescale only when some query's running maximum moved (alpha = 1
            // exactly otherwise: the 64 multiplies would change nothing)
            if (__any(m_new != m_run)) {
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_exp);  // 0 while m_run is -inf
                l_run = l_run * alpha;
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 16; i++) o[t][i] *= alpha;
            }
            l_run = l_run + ls;
            m_run = m_new;
            // O^T += V^T . P^T: k index 8*h2 + j of step s2 is key 16*s2 + (j/4)*8 + 4*h2 + j%4
#pragma unroll
            for (int t = 0; t < 4; t++) {
#pragma unroll
                for (int s2 = 0; s2 < 2; s2++) {
                    const char* vb = reinterpret_cast<const char*>(vs) + vx + 4096 * s2 + 256 * t;
                    const u32x2v lo = *reinterpret_cast<const u32x2v*>(vb);
                    const u32x2v hi = *reinterpret_cast<const u32x2v*>(vb + 2048);
                    u32x4v w;
                    w.x = lo.x; w.y = lo.y; w.z = hi.x; w.w = hi.y;
                    const f16x8 va = __builtin_bit_cast(f16x8, w);
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[s2], o[t], 0, 0, 0);
                }
            }
        }
    };
    for (int it = it0; it < it1; it += 3) {
        tile_step(it, ks0, vs0, fs0, ks2, vs2, fs2);
        if (it + 1 < it1) tile_step(it + 1, ks1, vs1, fs1, ks0, vs0, fs0);
        if (it + 2 < it1) tile_step(it + 2, ks2, vs2, fs2, ks1, vs1, fs1);
    }


    if (nparts > 1) {  // a part of a split block: its partial result
        if (part == 0 && tid == 0) a.vmx[qb * groups + hg] = vmax;
        if (myq < a.seq) {
            const size_t slot = ((size_t)myq * a.n_head + head) * kPfMaxParts + part;
            float* orow = a.opart + slot * kPfHd;
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    f32x4v r;
                    r.x = o[t][4 * g];
                    r.y = o[t][4 * g + 1];
                    r.z = o[t][4 * g + 2];
                    r.w = o[t][4 * g + 3];
                    *reinterpret_cast<f32x4v*>(orow + 32 * t + 8 * g + 4 * h2) = r;
                }
            if (h2 == 0) {
                a.mlpart[2 * slot] = m_run;
                a.mlpart[2 * slot + 1] = l_run;
            }
        }
        return;
    }
    // ---- out[myq][head][hd] = O^T[hd][myq] / l
    if (myq < a.seq) {
        const float inv = ldexpf(1.0f / l_run, vmax);
        float* orow = a.out + ((size_t)myq * a.n_head + head) * kPfHd;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                f32x4v r;
                r.x = o[t][4 * g] * inv;
                r.y = o[t][4 * g + 1] * inv;
                r.z = o[t][4 * g + 2] * inv;
                r.w = o[t][4 * g + 3] * inv;
                *reinterpret_cast<f32x4v*>(orow + 32 * t + 8 * g + 4 * h2) = r;
            }
    }
}

// The parts of a split query block joined: M = max_p m_p, l = sum_p l_p 2^(m_p - M),
// O = sum_p O_p 2^(m_p - M) (a part that saw no key: m = -inf, l = 0, O = 0),
// out = O / l * 2^vmax (vmax: the block's largest V tile exponent, as every part
// used).  One wave per (query, head) of a split block, lane = two columns.
__global__ __launch_bounds__(256) void prefill_combine_parts(PrefillArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int idx = (int)blockIdx.x * 4 + wave;
    if (idx >= a.seq * a.n_head) return;
    const int q = idx / a.n_head, head = idx - q * a.n_head;
    const int qb = q / a.q_block;
    const int nparts = pf_parts(a, qb);
    if (nparts <= 1) return;  // written whole by its workgroup
    const int vmax = a.vmx[qb * (a.n_head / a.heads_per_wg) + head / a.heads_per_wg];
    const size_t slot0 = ((size_t)q * a.n_head + head) * kPfMaxParts;
    float M = -INFINITY;
    for (int p = 0; p < nparts; p++) M = fmaxf(M, a.mlpart[2 * (slot0 + p)]);
    float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
    for (int p = 0; p < nparts; p++) {
        const float mp = a.mlpart[2 * (slot0 + p)];
        if (mp == -INFINITY) continue;
        const float al = __builtin_amdgcn_exp2f(mp - M);
        l += a.mlpart[2 * (slot0 + p) + 1] * al;
        const float* orow = a.opart + (slot0 + p) * kPfHd;
        o0 += orow[lane] * al;
        o1 += orow[lane + 64] * al;
    }
    const float inv = ldexpf(1.0f / l, vmax);
    float* out = a.out + ((size_t)q * a.n_head + head) * kPfHd;
    out[lane] = o0 * inv;
    out[lane + 64] = o1 * inv;
}

static size_t prefill_base_bytes(int seq, int kv_heads) {
    const size_t seq_pad = (size_t)(seq + kPfKeys - 1) / kPfKeys * kPfKeys;
    const size_t b = (size_t)kv_heads * seq_pad * kPfHd * 2 * sizeof(uint16_t) + (size_t)kv_heads * (seq_pad / kPfKeys) * 8;
    return (b + 255) / 256 * 256;
}

size_t attention_prefill_workspace(int seq, int n_head, int kv_heads) {
    // + vmx: one int per (query block of >= 32 queries, head group <= heads)
    return prefill_base_bytes(seq, kv_heads) + (size_t)seq * n_head * kPfMaxParts * (kPfHd + 2) * sizeof(float) +
           ((size_t)seq + 31) / 32 * n_head * sizeof(int);
}

hipError_t launch_attention_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                         const float* rope_cos, const float* rope_sin, float* out, int seq,
                                         int n_head, int kv_heads, int head_dim, float scale, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
    if (!q || !k || !v || !out || !workspace || seq <= 0 || n_head <= 0 || kv_heads <= 0 || head_dim != kPfHd ||
        n_head % kv_heads != 0 || (!rope_cos) != (!rope_sin))
        return hipErrorInvalidValue;
    if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)workspace) & 15) ||
        (rope_cos && (((uintptr_t)rope_cos | (uintptr_t)rope_sin) & 15)))
        return hipErrorInvalidValue;
    if (workspace_bytes < attention_prefill_workspace(seq, n_head, kv_heads)) return hipErrorInvalidValue;
    PrefillArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.out = out;
    a.seq = seq;
    a.seq_pad = (seq + kPfKeys - 1) / kPfKeys * kPfKeys;
    a.kt = static_cast<uint16_t*>(workspace);
    a.vt = a.kt + (size_t)kv_heads * a.seq_pad * kPfHd;
    a.kfv = reinterpret_cast<uint32_t*>(a.vt + (size_t)kv_heads * a.seq_pad * kPfHd);
    a.n_head = n_head;
    a.kv_heads = kv_heads;
    a.heads_per_wg = (n_head / kv_heads) % 2 == 0 ? 2 : 1;
    a.q_block = 32 * (4 / a.heads_per_wg);
    a.n_qblocks = (seq + a.q_block - 1) / a.q_block;
    a.scale = scale;
    // t_max: about the tiles one of the 3 x CUs resident workgroups gets on
    // average (never fewer than 16), so the longest chain is near the mean
    const int groups = n_head / a.heads_per_wg;
    long long work = 0;
    for (int qb = 0; qb < a.n_qblocks; qb++)
        work += (long long)((std::min((qb + 1) * a.q_block, seq) + kPfKeys - 1) / kPfKeys) * groups;
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const long long avg = (work + 3LL * cus - 1) / (3LL * cus);
    // only where the whole blocks leave CUs idle (S = 8192 measured 442 -> 450 us
    // with the split, S = 2048 93 -> 51 us + 18 us of combine)
    const bool fills = (long long)a.n_qblocks * groups >= 3LL * cus;
    a.t_max = fills ? 0x3FFFFFFF : (int)std::max<long long>(4, avg);
    a.opart = reinterpret_cast<float*>(static_cast<char*>(workspace) + prefill_base_bytes(seq, kv_heads));
    a.mlpart = a.opart + (size_t)seq * n_head * kPfMaxParts * kPfHd;
    a.vmx = reinterpret_cast<int*>(a.mlpart + (size_t)seq * n_head * kPfMaxParts * 2);
    long long grid = 0;
    bool split = false;
    for (int qb = 0; qb < a.n_qblocks; qb++) {
        const int tiles = (std::min((qb + 1) * a.q_block, seq) + kPfKeys - 1) / kPfKeys;
        const int parts = std::min(kPfMaxParts, (tiles + a.t_max - 1) / a.t_max);
        grid += (long long)parts * groups;
        split |= parts > 1;
    }
    const long long prep = (long long)kv_heads * (a.seq_pad / kPfKeys);
    if (grid > 0x7FFFFFFF || prep > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefill_prep_kv, dim3((unsigned)prep), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(attention_prefill_bf16, dim3((unsigned)grid), dim3(256), 0, stream, a);
    if (split)
        hipLaunchKernelGGL(prefill_combine_parts, dim3((unsigned)(((long long)seq * n_head + 3) / 4)), dim3(256), 0,
                           stream, a);
    return hipGetLastError();
}

}  // namespace mantle
