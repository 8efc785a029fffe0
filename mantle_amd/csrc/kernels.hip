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

#include "device_common.h"
#include "kernels.h"

namespace mantle {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

static constexpr int kThreads = 256;
static constexpr int kMaxPairs = 8;  // 32-weight blocks per lane per pass

// Byte position of element e (0..31) of a block in the even/odd permuted
// activation layout that k4_block_dot consumes.
__device__ __forceinline__ int qx_perm(int e) { return ((e & 1) << 4) | ((e >> 3) << 2) | ((e >> 1) & 3); }

// ---------------------------------------------------------------------------
// Parity reductions (Mantle's archsimd lane orders)

// Sum of squares exactly as rmsNormAVX512 / rmsNormSIMD / rmsNormScalar do it
// (internal/backend/simd/ops_avx512.go:92-112, ops_avx2.go:54-77, ops.go:70-76).
// Executed by a whole workgroup; red needs 17 floats of LDS.
__device__ float wg_sumsq_parity(const float* src, int n, int isa, float* red) {
    const int lanes = isa == kIsaAvx512 ? 16 : (isa == kIsaAvx2 ? 8 : 0);
    const int nfull = lanes ? (n / lanes) * lanes : 0;
    const int tid = threadIdx.x;
    if (lanes && tid < lanes) {
        float acc = 0.0f;
        for (int i = tid; i < nfull; i += lanes) acc = __builtin_fmaf(src[i], src[i], acc);
        red[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        if (lanes) {
            sum = red[0];
            for (int l = 1; l < lanes; l++) sum += red[l];
        }
        for (int i = nfull; i < n; i++) sum += src[i] * src[i];
        red[16] = sum;
    }
    __syncthreads();
    float r = red[16];
    __syncthreads();
    return r;
}

// Dot exactly as dotAVX512 / dotSIMD / dotScalar (internal/backend/simd/ops_avx512.go:27-90,
// ops_avx2.go:25-51, ops.go:49-55).  One thread computes the whole dot.
__device__ float dot_parity(const float* a, const float* b, int n, int isa) {
    if (isa == kIsaAvx512) {
        if (n == 0) return 0.0f;
        float acc[4][16];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int l = 0; l < 16; l++) acc[j][l] = 0.0f;
        int i = 0;
        for (; i + 64 <= n; i += 64) {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int l = 0; l < 16; l++) acc[j][l] = __builtin_fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        }
        for (; i + 32 <= n; i += 32) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int l = 0; l < 16; l++) acc[j][l] = __builtin_fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        }
        for (; i + 16 <= n; i += 16) {
#pragma unroll
            for (int l = 0; l < 16; l++) acc[0][l] = __builtin_fmaf(a[i + l], b[i + l], acc[0][l]);
        }
        float sum = acc[0][0];
#pragma unroll
        for (int k = 1; k < 64; k++) sum += acc[k / 16][k % 16];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    if (isa == kIsaAvx2) {
        if (n == 0) return 0.0f;
        float a0[8], a1[8];
#pragma unroll
        for (int l = 0; l < 8; l++) { a0[l] = 0.0f; a1[l] = 0.0f; }
        int i = 0;
        for (; i + 16 <= n; i += 16) {
#pragma unroll
            for (int l = 0; l < 8; l++) {
                a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
                a1[l] = __builtin_fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
            }
        }
        if (i + 8 <= n) {
#pragma unroll
            for (int l = 0; l < 8; l++) a0[l] = __builtin_fmaf(a[i + l], b[i + l], a0[l]);
            i += 8;
        }
#pragma unroll
        for (int l = 0; l < 8; l++) a0[l] = a0[l] + a1[l];
        float sum = a0[0];
#pragma unroll
        for (int l = 1; l < 8; l++) sum += a0[l];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

// ---------------------------------------------------------------------------
// Activation quantiser (+ optional RMSNorm), one workgroup per row.

__global__ __launch_bounds__(kThreads) void quantize_vec_kernel(const float* __restrict__ x, const float* __restrict__ weight,
                                                                  float eps, int n, int isa, int8_t* __restrict__ qx,
                                                                  float* __restrict__ xs, float* __restrict__ norm_out) {
    extern __shared__ __align__(16) float vals[];  // n + 17
    float* red = vals + n;
    const int row = blockIdx.x;
    const int blocks = (n + 31) / 32;
    x += (size_t)row * n;
    qx += (size_t)row * blocks * 32;
    xs += (size_t)row * blocks;
    if (weight) {
        float sumsq = wg_sumsq_parity(x, n, isa, red);
        float scale = rms_scale(sumsq, n, eps);
        for (int i = threadIdx.x; i < n; i += kThreads) vals[i] = (x[i] * scale) * weight[i];
    } else {
        for (int i = threadIdx.x; i < n; i += kThreads) vals[i] = x[i];
    }
    __syncthreads();
    if (norm_out)
        for (int i = threadIdx.x; i < n; i += kThreads) norm_out[(size_t)row * n + i] = vals[i];
    // quantizeVecBlocksInto (internal/backend/simd/matvec_quant.go:746-797): one lane per block.
    for (int b = threadIdx.x; b < blocks; b += kThreads) {
        const int base = b * 32;
        float maxabs = 0.0f;
        for (int i = 0; i < 32; i++) {
            if (base + i >= n) continue;
            float v = vals[base + i];
            if (v < 0) v = -v;
            if (v > maxabs) maxabs = v;
        }
        uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float scale = 0.0f;
        if (maxabs != 0.0f) {
            scale = maxabs / 127.0f;
            const float inv = 1.0f / scale;
            for (int i = 0; i < 32; i++) {
                if (base + i >= n) continue;
                int32_t q = go_round(vals[base + i] * inv);
                q = q > 127 ? 127 : (q < -127 ? -127 : q);
                const int p = qx_perm(i);
                words[p >> 2] |= ((uint32_t)(uint8_t)(int8_t)q) << ((p & 3) * 8);
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(qx + base);
        dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
        dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
        xs[b] = scale;
    }
}

hipError_t launch_quantize_vec(const float* x, const float* weight, float eps, int n, int batch, int isa,
                               int8_t* qx, float* xs, float* norm_out, hipStream_t stream) {
    if (!x || !qx || !xs || n <= 0 || batch <= 0) return hipErrorInvalidValue;
    size_t smem = sizeof(float) * ((size_t)n + 17);
    if (smem > 160 * 1024) return hipErrorInvalidValue;
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

hipError_t launch_rmsnorm(float* out, const float* x, const float* weight, float eps, int n, int rows, int isa,
                          hipStream_t stream) {
    if (!out || !x || !weight || n <= 0 || rows <= 0) return hipErrorInvalidValue;
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

struct GemvParams {
    K4Mat mats[3];
    float* outs[3];
    int wg_begin[4];
    int nmat;
    int cols, bpr, spr, rpw, batch;
    const int8_t* qx;
    const float* xs;
    const float* x;  // W4A32 input
    unsigned long long* key;
};

enum GemvMode : int { kModeW4A8 = 0, kModeW4A32 = 1 };

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    uint32_t u = __float_as_uint(v);
    uint32_t s = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)s << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

template <int MODE, int EPI>
__global__ __launch_bounds__(kThreads) void k4_gemv_kernel(GemvParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int bpr = p.bpr;
    const int B = p.batch;
    const int tid = threadIdx.x;
    const int qbytes = MODE == kModeW4A8 ? B * bpr * 32 : 0;
    int8_t* sq = reinterpret_cast<int8_t*>(smem);
    float* sxs = reinterpret_cast<float*>(smem + qbytes);
    float* terms = sxs + (MODE == kModeW4A8 ? B * bpr : 0);
    const int tstride = bpr + 1;  // odd stride: the row-sum lanes hit distinct banks

    int s = 0;
    if (EPI != kEpiSiluMul)
        while (s + 1 < p.nmat && (int)blockIdx.x >= p.wg_begin[s + 1]) s++;
    const int row0 = ((int)blockIdx.x - p.wg_begin[s]) * p.rpw;
    constexpr int nsub = EPI == kEpiSiluMul ? 2 : 1;

    if (MODE == kModeW4A8) {
        for (int i = tid * 16; i < qbytes; i += kThreads * 16)
            *reinterpret_cast<uint4*>(sq + i) = *reinterpret_cast<const uint4*>(p.qx + i);
        for (int i = tid; i < B * bpr; i += kThreads) sxs[i] = p.xs[i];
        __syncthreads();
    }

    const int per_sub = p.rpw * bpr;
    const int npairs = nsub * per_sub;
    for (int base = 0; base < npairs; base += kThreads * kMaxPairs) {
        uint4 w[kMaxPairs];
        float sw[kMaxPairs];
        int sk[kMaxPairs], rl[kMaxPairs], bb[kMaxPairs];
#pragma unroll
        for (int j = 0; j < kMaxPairs; j++) {
            const int pi = base + j * kThreads + tid;
            sw[j] = 0.0f;
            w[j] = make_uint4(0, 0, 0, 0);
            sk[j] = -1;
            if (pi < npairs) {
                const int k = nsub == 2 ? pi / per_sub : 0;
                const int rem = pi - k * per_sub;
                const int r = rem / bpr;
                const int b = rem - r * bpr;
                sk[j] = k;
                rl[j] = r;
                bb[j] = b;
                const K4Mat& M = p.mats[nsub == 2 ? k : s];
                const int grow = row0 + r;
                if (grow < M.rows) {
                    const size_t blk = (size_t)grow * bpr + b;
                    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(M.nib) + blk);
                    w[j] = make_uint4(v.x, v.y, v.z, v.w);
                    sw[j] = k4_scale(M.sup[(size_t)grow * p.spr + (b >> 3)], M.sub[blk]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kMaxPairs; j++) {
            if (sk[j] < 0) continue;
            const int b = bb[j];
            float* trow = terms + ((sk[j] * p.rpw + rl[j]) * B) * tstride + b;
            for (int bi = 0; bi < B; bi++) {
                float term = 0.0f;
                if (MODE == kModeW4A8) {
                    const float xsv = sxs[bi * bpr + b];
                    if (sw[j] != 0.0f && xsv != 0.0f) {
                        const int8_t* xb = sq + (bi * bpr + b) * 32;
                        const uint4 xe = *reinterpret_cast<const uint4*>(xb);
                        const uint4 xo = *reinterpret_cast<const uint4*>(xb + 16);
                        term = (float)k4_block_dot(w[j], xe, xo) * (sw[j] * xsv);
                    }
                } else {
                    if (sw[j] != 0.0f) {
                        const float* xb = p.x + (size_t)bi * p.cols + b * 32;
                        const int n = min(32, p.cols - b * 32);
                        const uint32_t wd[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
                        float d = 0.0f;
                        for (int e = 0; e < n; e++) d = __builtin_fmaf((float)k4_nib(wd[e >> 3], e & 7), xb[e], d);
                        term = sw[j] * d;
                    }
                }
                trow[bi * tstride] = term;
            }
        }
    }
    __syncthreads();

    if (EPI == kEpiSiluMul) {
        if (tid < p.rpw) {
            const int grow = row0 + tid;
            if (grow < p.mats[0].rows) {
                const float* tg = terms + tid * tstride;
                const float* tu = terms + (p.rpw + tid) * tstride;
                float g = 0.0f, u = 0.0f;
                for (int b = 0; b < bpr; b++) g += tg[b];
                for (int b = 0; b < bpr; b++) u += tu[b];
                p.outs[0][grow] = fast_silu_vec(g) * u;
            }
        }
        return;
    }

    const K4Mat& M = p.mats[s];
    float* out = p.outs[s];
    unsigned long long best = 0;
    for (int t = tid; t < p.rpw * B; t += kThreads) {
        const int r = t / B;
        const int bi = t - r * B;
        const int grow = row0 + r;
        if (grow >= M.rows) continue;
        const float* tr = terms + t * tstride;
        float sum = 0.0f;
        for (int b = 0; b < bpr; b++) sum += tr[b];
        if (EPI == kEpiResAdd) {
            out[grow] = out[grow] + sum;
        } else {
            out[(size_t)bi * M.rows + grow] = sum;
            if (EPI == kEpiArgmax) {
                unsigned long long k = argmax_key(sum, grow);
                best = k > best ? k : best;
            }
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
            atomicMax(p.key, m);
        }
    }
}

// Rows per workgroup: as many 32-weight blocks as 256 lanes x 8 passes hold,
// then fewer while the grid is under ~2 workgroups per CU (small matrices).
static int choose_rpw(int total_rows, int bpr, int nsub, int batch, size_t fixed_smem, size_t smem_cap) {
    int rpw = (kThreads * kMaxPairs) / (bpr * nsub);
    if (rpw < 1) rpw = 1;
    while (rpw > 1 && (total_rows + rpw - 1) / rpw < 512) rpw = (rpw + 1) / 2;
    while (rpw > 1 && fixed_smem + (size_t)nsub * rpw * batch * (bpr + 1) * 4 > smem_cap) rpw = (rpw + 1) / 2;
    return rpw;
}

template <int MODE>
static hipError_t launch_gemv(GemvParams& p, GemvEpi epi, hipStream_t stream) {
    const int nsub = epi == kEpiSiluMul ? 2 : 1;
    int total_rows = 0;
    for (int i = 0; i < p.nmat; i++) total_rows += p.mats[i].rows;
    if (epi == kEpiSiluMul) total_rows = p.mats[0].rows;
    const size_t fixed = MODE == kModeW4A8 ? (size_t)p.batch * p.bpr * 36 : 0;
    const size_t cap = 64 * 1024;
    p.rpw = choose_rpw(total_rows, p.bpr, nsub, p.batch, fixed, cap);
    const size_t smem = fixed + (size_t)nsub * p.rpw * p.batch * (p.bpr + 1) * 4;
    if (smem > cap) return hipErrorInvalidValue;
    int grid = 0;
    if (epi == kEpiSiluMul) {
        p.wg_begin[0] = 0;
        grid = (p.mats[0].rows + p.rpw - 1) / p.rpw;
    } else {
        for (int i = 0; i < p.nmat; i++) {
            p.wg_begin[i] = grid;
            grid += (p.mats[i].rows + p.rpw - 1) / p.rpw;
        }
    }
    p.wg_begin[p.nmat] = grid;
    switch (epi) {
        case kEpiStore:
            hipLaunchKernelGGL((k4_gemv_kernel<MODE, kEpiStore>), dim3(grid), dim3(kThreads), smem, stream, p);
            break;
        case kEpiResAdd:
            hipLaunchKernelGGL((k4_gemv_kernel<MODE, kEpiResAdd>), dim3(grid), dim3(kThreads), smem, stream, p);
            break;
        case kEpiSiluMul:
            hipLaunchKernelGGL((k4_gemv_kernel<MODE, kEpiSiluMul>), dim3(grid), dim3(kThreads), smem, stream, p);
            break;
        case kEpiArgmax:
            hipLaunchKernelGGL((k4_gemv_kernel<MODE, kEpiArgmax>), dim3(grid), dim3(kThreads), smem, stream, p);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
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
    return launch_gemv<kModeW4A8>(p, epi, stream);
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
    return launch_gemv<kModeW4A32>(p, kEpiStore, stream);
}

// ---------------------------------------------------------------------------
// Decode attention (internal/backend/simd/attn.go:255-419, attnpool.go:77-153)

__global__ __launch_bounds__(kThreads) void attention_decode_kernel(AttnArgs a) {
    __shared__ float sq[256], sk[256], sv[256], red[17];
    __shared__ float smax[kThreads / 64];
    __shared__ float ssum;
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int hd = a.head_dim;
    const int kvh = h * a.kv_heads / a.n_head;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos_host;
    float* scores = a.scores + (size_t)h * a.max_ctx;

    for (int i = tid; i < hd; i += kThreads) {
        sq[i] = a.q[h * hd + i];
        if (a.fused) {
            sk[i] = a.k[kvh * hd + i];
            sv[i] = a.v[kvh * hd + i];
        }
    }
    __syncthreads();
    if (a.fused) {
        if (a.q_norm) {  // attn.go:265-286 per-head RMSNorm (q, then k)
            float s = wg_sumsq_parity(sq, hd, a.isa, red);
            float sc = rms_scale(s, hd, a.eps);
            for (int i = tid; i < hd; i += kThreads) sq[i] = (sq[i] * sc) * a.q_norm[i];
        }
        if (a.k_norm) {
            float s = wg_sumsq_parity(sk, hd, a.isa, red);
            float sc = rms_scale(s, hd, a.eps);
            for (int i = tid; i < hd; i += kThreads) sk[i] = (sk[i] * sc) * a.k_norm[i];
        }
        __syncthreads();
        if (a.rope_cos) {  // ops_avx512.go:162-190: y0 = x0*c - x1*s, y1 = fma(x0, s, x1*c)
            const int half = hd / 2;
            const float* c = a.rope_cos + (size_t)pos * half;
            const float* sn = a.rope_sin + (size_t)pos * half;
            for (int i = tid; i < half; i += kThreads) {
                float x0 = sq[i], x1 = sq[i + half];
                sq[i] = x0 * c[i] - x1 * sn[i];
                sq[i + half] = __builtin_fmaf(x0, sn[i], x1 * c[i]);
                x0 = sk[i];
                x1 = sk[i + half];
                sk[i] = x0 * c[i] - x1 * sn[i];
                sk[i + half] = __builtin_fmaf(x0, sn[i], x1 * c[i]);
            }
        }
        __syncthreads();
        // ops_runtime.go:112-131 StoreKV: the first q-head of each kv group writes.
        const int first = (kvh * a.n_head + a.kv_heads - 1) / a.kv_heads;
        if (h == first) {
            for (int i = tid; i < hd; i += kThreads) {
                a.cache_k[(size_t)pos * a.kv_stride + kvh * hd + i] = sk[i];
                a.cache_v[(size_t)pos * a.kv_stride + kvh * hd + i] = sv[i];
            }
        }
    }

    // scores_t = Dot(q, k_t) * scale
    float lmax = -INFINITY;
    for (int t = tid; t <= pos; t += kThreads) {
        const float* kt = (a.fused && t == pos) ? sk : a.cache_k + (size_t)t * a.kv_stride + kvh * hd;
        float sc = dot_parity(sq, kt, hd, a.isa) * a.scale;
        scores[t] = sc;
        lmax = fmaxf(lmax, sc);
    }
    for (int off = 32; off > 0; off >>= 1) lmax = fmaxf(lmax, __shfl_down(lmax, off, 64));
    if ((tid & 63) == 0) smax[tid >> 6] = lmax;
    __syncthreads();
    float maxv = smax[0];
    for (int i = 1; i < kThreads / 64; i++) maxv = fmaxf(maxv, smax[i]);
    // Softmax (ops.go:83-106): exponentials, ordered sum, x *= 1/sum
    for (int t = tid; t <= pos; t += kThreads) scores[t] = fast_exp_scalar(scores[t] - maxv);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t = 0; t <= pos; t++) sum += scores[t];
        ssum = sum;
    }
    __syncthreads();
    const float sum = ssum;
    if (sum != 0.0f) {
        const float inv = 1.0f / sum;
        for (int t = tid; t <= pos; t += kThreads) scores[t] = scores[t] * inv;
    }
    __syncthreads();
    // out_d = sum_t p_t * v_t,d in t order
    for (int d = tid; d < hd; d += kThreads) {
        float acc = 0.0f;
        const float* vcol = a.cache_v + kvh * hd + d;
        for (int t = 0; t <= pos; t++) {
            float v = (a.fused && t == pos) ? sv[d] : vcol[(size_t)t * a.kv_stride];
            acc += scores[t] * v;
        }
        a.out[h * hd + d] = acc;
    }
}

hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t stream) {
    if (!a.q || !a.cache_k || !a.cache_v || !a.scores || !a.out || a.n_head <= 0 || a.kv_heads <= 0 ||
        a.head_dim <= 0 || a.head_dim > 256 || a.kv_stride < a.kv_heads * a.head_dim || a.max_ctx <= 0)
        return hipErrorInvalidValue;
    if (a.fused && (!a.k || !a.v)) return hipErrorInvalidValue;
    if (!a.pos_dev && (a.pos_host < 0 || a.pos_host >= a.max_ctx)) return hipErrorInvalidValue;
    if (a.rope_cos && (!a.rope_sin || (a.head_dim & 1))) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_decode_kernel, dim3(a.n_head), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
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
    if (threadIdx.x == 0) st->argmax_key = 0ull;
}

hipError_t launch_embed(const K4Mat& emb, int cols, const int* prompt, DecodeState* st, float* x,
                        hipStream_t stream) {
    if (!emb.nib || !prompt || !st || !x || cols <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(kThreads), 0, stream, emb, cols, prompt, st, x);
    return hipGetLastError();
}

__global__ void finish_step_kernel(DecodeState* st, int* out_tokens) {
    const unsigned long long key = st->argmax_key;
    const int idx = key == 0ull ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    st->next_tok = idx;
    out_tokens[st->pos] = idx;
    st->pos = st->pos + 1;
}

hipError_t launch_finish_step(DecodeState* st, int* out_tokens, hipStream_t stream) {
    if (!st || !out_tokens) return hipErrorInvalidValue;
    hipLaunchKernelGGL(finish_step_kernel, dim3(1), dim3(1), 0, stream, st, out_tokens);
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

// RoPE from float64 inverse frequencies (Mantle keeps invFreq as []float64,
// internal/backend/simd/loader.go:1604-1612); cos/sin evaluated in f64.
__global__ void rope_f64_kernel(float* x, const double* inv_freq, int pos, float attn_scale, int head_dim, int half) {
    float* lo = x + (size_t)blockIdx.x * head_dim;
    float* hi = lo + half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const double ang = (double)pos * inv_freq[i];
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

hipError_t launch_rope_f64(float* x, const double* inv_freq, int pos, float attn_scale, int head_dim, int half,
                           int n_heads, hipStream_t stream) {
    if (!x || !inv_freq || head_dim <= 0 || half <= 0 || half * 2 > head_dim || n_heads <= 0 || pos < 0)
        return hipErrorInvalidValue;
    if (attn_scale == 0.0f) attn_scale = 1.0f;
    hipLaunchKernelGGL(rope_f64_kernel, dim3(n_heads), dim3(128), 0, stream, x, inv_freq, pos, attn_scale, head_dim, half);
    return hipGetLastError();
}

__global__ void store_kv_row_kernel(float* cache, const float* src, int cache_pos, int kv_stride) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kv_stride; i += gridDim.x * blockDim.x)
        cache[(size_t)cache_pos * kv_stride + i] = src[i];
}

hipError_t launch_store_kv_row(float* cache, const float* src, int cache_pos, int kv_stride, hipStream_t stream) {
    if (!cache || !src || cache_pos < 0 || kv_stride <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(store_kv_row_kernel, dim3((kv_stride + kThreads - 1) / kThreads), dim3(kThreads), 0, stream,
                       cache, src, cache_pos, kv_stride);
    return hipGetLastError();
}

}  // namespace mantle
