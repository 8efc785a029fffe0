// gemm_w4a32.hip -- the k4 GEMV on fp32 activations (W4A32) at batch 2..8 on
// f16 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Arithmetic: y[v][r] = sum over blocks of s_w[r,b] * (sum_i q[r,b,i] * x[v][32b+i])
// -- the CUDA backend's quant_matvec_k4_f32 (internal/backend/cuda/native/
// softmax.cu:411-546) and the CPU's non-AVX2 branch (internal/backend/simd/
// matvec_quant.go:291-293) -- checked within max-abs 1e-3 / rel 1e-2 (the
// summation order is free).  The weights q in -8..7 are exact in f16.  Each
// activation is split into two f16 parts after a power-of-two range factor
// per vector (x * 2^-e = hi + lo, hi = f16(x * 2^-e), lo = f16(x * 2^-e - hi),
// the largest |x| of the vector brought into [2^14, 2^15)): the pair carries
// ~22 significant bits, the products and the block dot accumulate in fp32, and
// 2^e is applied to the output.
//
// MFMA columns: 16 = 8 vectors x {hi, lo}; rows: 16 weight rows; K = 32: one
// k4 block per instruction.  Lane l holds A[row l%16][k 8(l/16)..+7] (the 8
// nibbles of weight word l/16 of the block, as f16 in the order e0 e4 e1 e5 e2
// e6 e3 e7 that two nibbles per 32-bit word give) and B[k ...][column l%16]
// (the same 8 elements of that column's activation part, staged in LDS in the
// same order); the result D[row 4(l/16)+i][column l%16] is the block dot,
// scaled by s_w and accumulated per lane; lanes 2v and 2v+1 add their hi and lo
// sums at the end.
//
// Tiling (TR rows per workgroup): chunks of 8 blocks of weights (coalesced
// 16-byte loads) and of the activations (fp32, split while staging) go through
// LDS, the next chunk's loads in flight while the current one is multiplied.
// TR = 128: four waves of 2 x 16 rows, each over all 8 blocks of a chunk.
// TR = 32 (matrices of few rows, where 128-row workgroups would leave most of
// the chip idle): the four waves take the same 2 x 16 rows and blocks 2w, 2w+1
// of every chunk, and their sums are added through LDS at the end.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"
#include "kernels.h"

namespace mantle {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

static constexpr int kW32KC = 8;      // blocks per chunk
static constexpr int kW32WP = 36;     // weight row pitch in LDS (words): 8 blocks x 16 bytes + pad
static constexpr int kW32XP = 132;    // activation column pitch (words): 8 blocks x 32 f16 + pad

struct W32MfmaArgs {
    K4Mat w;
    int bpr, batch;
    const float* x;  // [batch][bpr*32]
    float* y;        // [batch][rows]
};

// 2^e bringing m = max |x| into [2^14, 2^15) (0 for 0 / non-finite: NaN and Inf propagate).
__device__ __forceinline__ int w32_range_exp(float m) {
    if (!(m > 0.0f) || !(m < INFINITY)) return 0;
    int E;
    (void)frexpf(m, &E);  // m = f * 2^E, f in [0.5, 1)
    return E - 15;
}

// Weight word w (8 nibbles, elements 0..7 of a k group) as 8 f16 in the order
// e0 e4 e1 e5 e2 e6 e3 e7: two nibbles per 32-bit word (bits 4k and 4k+16) put
// into the mantissas of 1024 + u (u = q + 8) and 1032 subtracted, exactly.
__device__ __forceinline__ half8_t w32_nibbles_f16(uint32_t w) {
    const uint32_t u = w ^ 0x88888888u;  // two's-complement nibble -> offset binary
    half8_t r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t t = ((u >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
        const __half2 h = __hsub2(*reinterpret_cast<const __half2*>(&t), __half2(__half(1032.0f), __half(1032.0f)));
        r[2 * k] = (_Float16)__low2float(h);
        r[2 * k + 1] = (_Float16)__high2float(h);
    }
    return r;
}

template <int TR>
__global__ __launch_bounds__(256) void k4_gemv_w4a32_mfma(W32MfmaArgs a) {
    constexpr int kW32TR = TR;
    constexpr bool KS = TR == 32;  // waves split the blocks of a chunk
    constexpr int NI = TR / 32;    // 16-byte weight loads per thread and chunk
    __shared__ __align__(16) uint32_t wn[kW32TR * kW32WP];
    __shared__ __align__(16) uint32_t xh[16 * kW32XP];
    __shared__ __align__(16) float swT[kW32KC * kW32TR];
    __shared__ int vexp[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = lane >> 4, l16 = lane & 15;
    const int rows = a.w.rows, bpr = a.bpr, spr = (bpr + 7) / 8, cols = bpr * 32;
    const int row0 = (int)blockIdx.x * kW32TR, wr0 = KS ? 0 : wave * 32;

    // this thread's activation group: vector tid/32, block (tid%32)/4 of the chunk, elements 8*(tid%4) .. +7
    const int sv = tid >> 5, sblk = (tid & 31) >> 2, sg = tid & 3;
    uint32_t rw[NI][4];
    float rx[8];
    uint32_t rsub[NI];
    uint16_t rsup[NI];
    auto load_chunk = [&](int b0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NI; i++) {  // TR rows x 8 blocks of 16 bytes
            const int it = tid + 256 * i, r = it >> 3, part = it & 7;
            const int gr = row0 + r < rows ? row0 + r : rows - 1;
            const uint4 u = reinterpret_cast<const uint4*>(a.w.nib)[(size_t)gr * bpr + b0 + part];
            rw[i][0] = u.x; rw[i][1] = u.y; rw[i][2] = u.z; rw[i][3] = u.w;
        }
        const int v = sv < a.batch ? sv : a.batch - 1;
        const float4* xs = reinterpret_cast<const float4*>(a.x + (size_t)v * cols + (size_t)(b0 + sblk) * 32 + 8 * sg);
        const float4 x0 = xs[0], x1 = xs[1];
        rx[0] = x0.x; rx[1] = x0.y; rx[2] = x0.z; rx[3] = x0.w;
        rx[4] = x1.x; rx[5] = x1.y; rx[6] = x1.z; rx[7] = x1.w;
#pragma unroll
        for (int i = 0; i < NI; i++) {  // TR rows x 8 block scales
            const int it = tid + 256 * i, r = it >> 3, blk = it & 7;
            const int gr = row0 + r < rows ? row0 + r : rows - 1;
            rsub[i] = a.w.sub[(size_t)gr * bpr + b0 + blk];
            rsup[i] = a.w.sup[(size_t)gr * spr + ((b0 + blk) >> 3)];
        }
    };
    load_chunk(0);  // the first chunk's loads in flight while the range factors are found
    // the vectors' range factors: wave w takes vectors 2w, 2w+1
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int v = 2 * wave + j;
        float m = 0.0f;
        if (v < a.batch)
            for (int i = lane * 4; i < cols; i += 256) {  // cols: a multiple of 256
                const float4 q = *reinterpret_cast<const float4*>(a.x + (size_t)v * cols + i);
                m = fmaxf(m, fmaxf(fmaxf(fabsf(q.x), fabsf(q.y)), fmaxf(fabsf(q.z), fabsf(q.w))));
            }
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (lane == 0) vexp[v] = w32_range_exp(m);
    }
    __syncthreads();
    const float sfac = ldexpf(1.0f, -vexp[sv]);
    auto store_chunk = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int it = tid + 256 * i;
            *reinterpret_cast<uint4*>(wn + (it >> 3) * kW32WP + (it & 7) * 4) =
                make_uint4(rw[i][0], rw[i][1], rw[i][2], rw[i][3]);
        }
        // hi / lo parts in the k order e0 e4 e1 e5 e2 e6 e3 e7 (zeros for vectors past the batch)
        half8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int e = (j >> 1) + 4 * (j & 1);
            const float xv = sv < a.batch ? rx[e] * sfac : 0.0f;
            const _Float16 h = (_Float16)xv;
            hi[j] = h;
            lo[j] = (_Float16)(xv - (float)h);
        }
        *reinterpret_cast<half8_t*>(xh + (2 * sv) * kW32XP + sblk * 16 + sg * 4) = hi;
        *reinterpret_cast<half8_t*>(xh + (2 * sv + 1) * kW32XP + sblk * 16 + sg * 4) = lo;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int it = tid + 256 * i;
            swT[(it & 7) * kW32TR + (it >> 3)] = k4_scale(rsup[i], (uint8_t)rsub[i]);
        }
    };

    float acc[2][4];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[rt][i] = 0.0f;
    const int nch = bpr / kW32KC;
    for (int c = 0; c < nch; c++) {
        __syncthreads();  // the previous chunk's readers are done
        store_chunk();
        __syncthreads();
        load_chunk((c + 1 < nch ? c + 1 : c) * kW32KC);  // in flight while this chunk is multiplied
#pragma unroll
        for (int bb = 0; bb < (KS ? 2 : kW32KC); bb++) {
            const int b = KS ? 2 * wave + bb : bb;
            const half8_t bx = *reinterpret_cast<const half8_t*>(xh + l16 * kW32XP + b * 16 + kq * 4);
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
                const half8_t aw = w32_nibbles_f16(wn[(wr0 + rt * 16 + l16) * kW32WP + b * 4 + kq]);
                const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
                const f32x4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw, bx, zero, 0, 0, 0);
                const float4 sw = *reinterpret_cast<const float4*>(&swT[b * kW32TR + wr0 + rt * 16 + 4 * kq]);
                acc[rt][0] = __builtin_fmaf(d[0], sw.x, acc[rt][0]);
                acc[rt][1] = __builtin_fmaf(d[1], sw.y, acc[rt][1]);
                acc[rt][2] = __builtin_fmaf(d[2], sw.z, acc[rt][2]);
                acc[rt][3] = __builtin_fmaf(d[3], sw.w, acc[rt][3]);
            }
        }
    }
    if constexpr (KS) {  // waves 1-3 hand their sums to wave 0 (added in wave order)
        float* red = reinterpret_cast<float*>(xh);  // the activation tile is no longer read (1536 of its 2112 words)
        __syncthreads();
        if (wave > 0)
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) red[((wave - 1) * 8 + rt * 4 + i) * 64 + lane] = acc[rt][i];
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 1; w < 4; w++)
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[rt][i] += red[((w - 1) * 8 + rt * 4 + i) * 64 + lane];
    }
    // column l16 = 2v + part: the lo lane's sums join the hi lane's
    const int v = l16 >> 1;
    const float ofac = v < a.batch ? ldexpf(1.0f, vexp[v]) : 0.0f;
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = acc[rt][i] + __shfl_xor(acc[rt][i], 1, 64);
            const int r = row0 + wr0 + rt * 16 + 4 * kq + i;
            if ((l16 & 1) == 0 && v < a.batch && r < rows) a.y[(size_t)v * rows + r] = s * ofac;
        }
}

// Whole 8-block chunks per row, batch 2..8, 16-byte aligned x; *used false otherwise.
hipError_t k4_gemv_w4a32_mfma_launch(const K4Mat& m, int cols, const float* x, float* y, int batch,
                                     hipStream_t stream, bool* used) {
    *used = false;
    const int bpr = (cols + 31) / 32;
    if (cols != bpr * 32 || bpr % kW32KC || batch < 2 || batch > 8 || ((uintptr_t)x & 15)) return hipSuccess;
    *used = true;
    W32MfmaArgs a;
    a.w = m;
    a.bpr = bpr;
    a.batch = batch;
    a.x = x;
    a.y = y;
    // 128-row workgroups where they give at least one per CU, else 32-row ones
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if ((m.rows + 127) / 128 >= cus)
        hipLaunchKernelGGL(k4_gemv_w4a32_mfma<128>, dim3((m.rows + 127) / 128), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(k4_gemv_w4a32_mfma<32>, dim3((m.rows + 31) / 32), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mantle
