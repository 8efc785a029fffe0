/*
 * mantle_oracle.c -- CPU restatement of Mantle's archsimd decode path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): see mantle_oracle.h.  Compiled with
 * -O2 -ffp-contract=off so that no a*b+c is fused unless fmaf() is written,
 * mirroring Go at GOAMD64=v1 (no implicit fusion) plus archsimd MulAdd (fused).
 *
 * Reference paths are relative to the samcharles93/mantle tree.
 */
#include "mantle_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void mo_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int mo_get_threads(void) { return g_threads; }

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* internal/backend/simd/float16.go:7-46 (Float32ToFloat16): truncating, FTZ,
 * underflow -> signed zero, overflow -> inf, NaN -> 0x200 payload. */
uint16_t mo_f32_to_f16(float f) {
    uint32_t bits = f2u(f);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int exp = (int)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    uint16_t out_exp = 0, out_mant = 0;
    if (exp == 0) {
        return (uint16_t)(sign << 15);
    } else if (exp == 0xFF) {
        out_exp = 0x1F;
        if (mant != 0) out_mant = 0x200;
    } else {
        int new_exp = exp - 127 + 15;
        if (new_exp >= 31) {
            out_exp = 0x1F;
        } else if (new_exp <= 0) {
            out_exp = 0;
        } else {
            out_exp = (uint16_t)new_exp;
            out_mant = (uint16_t)(mant >> 13);
        }
    }
    return (uint16_t)((sign << 15) | (out_exp << 10) | out_mant);
}

/* internal/backend/core/float16.go:42-64 (Float16ToFloat32): subnormals -> 0. */
float mo_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        out = sign << 31;
    } else if (exp == 0x1F) {
        out = (sign << 31) | 0x7F800000u;
        if (mant != 0) out |= mant << 13;
    } else {
        out = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return u2f(out);
}

static inline int64_t align64(int64_t n) { return (n + 63) & ~(int64_t)63; }

/* pkg/mcf/quant_payload.go:15-113 (QuantPayloadSize, family 'k', bits 4) and
 * internal/backend/core/quant_cache.go:103-214 (quantLayoutForMat offsets). */
int mo_k4_layout_for(int64_t rows, int64_t cols, mo_k4_layout* L) {
    if (rows <= 0 || cols <= 0 || !L) return -1;
    L->rows = rows;
    L->cols = cols;
    L->blocks_per_row = (cols + 31) / 32;
    L->super_per_row = (L->blocks_per_row + 7) / 8;
    int64_t total_blocks = rows * L->blocks_per_row;
    int64_t total_super = rows * L->super_per_row;
    L->super_off = 0;
    L->sub_off = align64(total_super * 2);
    L->data_off = align64(L->sub_off + total_blocks);
    L->size = L->data_off + total_blocks * 16;
    return 0;
}

/* cmd/mantle/quantize.go:752-759 (clamp) */
static inline float clampf_(float v, float lo, float hi) {
    if (v < lo) return lo;
    if (v > hi) return hi;
    return v;
}

/* Go math.Round: half away from zero.  C roundf has the same definition, and
 * float32->float64 is exact, so int32(math.Round(float64(v))) == (int)roundf(v). */
static inline int32_t go_round_f32(float v) { return (int32_t)roundf(v); }

/* cmd/mantle/quantize.go:352-398 (quantizeTensor: global +/-maxAbs clip) and
 * cmd/mantle/quantize.go:530-651 (quantizeK, bits=4: block scale maxAbs/7,
 * super = max block scale stored as truncated f16, u6 = round(32*s_b/super)
 * clamped to [1,63] using the UNROUNDED fp32 super, q = round(v/(super*u6/32))
 * clamped to +/-7), bitPacker LSB-first (:653-680). */
int mo_quantize_k4(const float* src, int64_t rows, int64_t cols, uint8_t* payload) {
    mo_k4_layout L;
    if (mo_k4_layout_for(rows, cols, &L) != 0) return -1;
    const int64_t n = rows * cols;
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) {
        float v = src[i];
        if (isnan(v) || isinf(v)) return -2;
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    /* quantize.go:734-741 maxAbs */
    float amn = fabsf(mn), amx = fabsf(mx);
    float maxabs = amn > amx ? amn : amx;
    const float lo = -maxabs, hi = maxabs;
    const int32_t qmax = 7;

    memset(payload, 0, (size_t)L.size);
    uint8_t* super_p = payload + L.super_off;
    uint8_t* sub_p = payload + L.sub_off;
    uint8_t* data_p = payload + L.data_off;
    const int64_t bpr = L.blocks_per_row, spr = L.super_per_row;

    for (int64_t r = 0; r < rows; r++) {
        const int64_t row_base = r * cols;
        const int64_t row_limit = row_base + cols;
        for (int64_t s = 0; s < spr; s++) {
            float block_scales[8];
            float max_scale = 0.0f;
            for (int b = 0; b < 8; b++) {
                int64_t block = s * 8 + b;
                if (block >= bpr) { block_scales[b] = 0; continue; }
                float ma = 0.0f;
                int64_t base = row_base + block * 32;
                for (int i = 0; i < 32; i++) {
                    int64_t idx = base + i;
                    float v = 0.0f;
                    if (idx < row_limit) v = clampf_(src[idx], lo, hi);
                    float av = fabsf(v);
                    if (av > ma) ma = av;
                }
                if (ma == 0.0f) { block_scales[b] = 0; continue; }
                block_scales[b] = ma / (float)qmax;
                if (block_scales[b] > max_scale) max_scale = block_scales[b];
            }
            const float super_scale = max_scale;
            uint16_t h = mo_f32_to_f16(super_scale);
            int64_t super_idx = r * spr + s;
            super_p[super_idx * 2] = (uint8_t)(h & 0xFF);
            super_p[super_idx * 2 + 1] = (uint8_t)(h >> 8);
            for (int b = 0; b < 8; b++) {
                int64_t block = s * 8 + b;
                if (block >= bpr) continue;
                int64_t block_idx = r * bpr + block;
                uint8_t u6 = 0;
                if (block_scales[b] > 0 && super_scale > 0) {
                    float ratio = block_scales[b] / super_scale;
                    int u = (int)go_round_f32(ratio * 32.0f);
                    if (u < 1) u = 1; else if (u > 63) u = 63;
                    u6 = (uint8_t)u;
                }
                sub_p[block_idx] = u6 & 0x3F;
                float scale = 0.0f;
                if (u6 > 0 && super_scale > 0) scale = super_scale * ((float)u6 / 32.0f);
                float inv = 0.0f;
                if (scale != 0.0f) inv = 1.0f / scale;
                int64_t base = row_base + block * 32;
                uint8_t* dst = data_p + block_idx * 16;
                for (int i = 0; i < 32; i++) {
                    int64_t idx = base + i;
                    float v = 0.0f;
                    if (idx < row_limit) v = clampf_(src[idx], lo, hi);
                    int32_t q = 0;
                    if (scale != 0.0f) {
                        q = go_round_f32(v * inv);
                        if (q > qmax) q = qmax; else if (q < -qmax) q = -qmax;
                    }
                    uint8_t nib = (uint8_t)((uint8_t)(int8_t)q & 0x0F);
                    dst[i >> 1] |= (uint8_t)(nib << ((i & 1) * 4));
                }
            }
        }
    }
    return 0;
}

/* internal/backend/core/quant_cache.go:26-29 (q4SignTable) via decodeBlock4 :238-255 */
static inline int8_t q4_sign(uint8_t nib) { return (int8_t)(nib < 8 ? nib : (int)nib - 16); }

/* internal/backend/core/quant_cache.go:216-223 (scaleAtRawLE) */
static inline float scale_at_le(const uint8_t* raw, int64_t idx) {
    uint16_t u = (uint16_t)(raw[idx * 2] | (raw[idx * 2 + 1] << 8));
    return mo_f16_to_f32(u);
}

/* internal/backend/core/quant_cache.go:77-100 (BuildQuantCache, k family):
 * scale = super * (float32(u6)/32), 0 when super==0 or u6==0. */
static inline float k4_block_scale(const uint8_t* payload, const mo_k4_layout* L, int64_t r, int64_t b) {
    float sup = scale_at_le(payload + L->super_off, r * L->super_per_row + b / 8);
    uint8_t u6 = payload[L->sub_off + r * L->blocks_per_row + b] & 0x3F;
    if (sup == 0.0f || u6 == 0) return 0.0f;
    return sup * ((float)u6 / 32.0f);
}

int mo_k4_block_scales(const uint8_t* payload, int64_t rows, int64_t cols, float* scales) {
    mo_k4_layout L;
    if (mo_k4_layout_for(rows, cols, &L) != 0) return -1;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t b = 0; b < L.blocks_per_row; b++)
            scales[r * L.blocks_per_row + b] = k4_block_scale(payload, &L, r, b);
    return 0;
}

static inline void k4_decode_block(const uint8_t* payload, const mo_k4_layout* L, int64_t r, int64_t b, int8_t q[32]) {
    const uint8_t* src = payload + L->data_off + (r * L->blocks_per_row + b) * 16;
    for (int i = 0; i < 16; i++) {
        q[2 * i] = q4_sign(src[i] & 0x0F);
        q[2 * i + 1] = q4_sign((src[i] >> 4) & 0x0F);
    }
}

/* internal/backend/core/quant_stub.go:51-85 (rowToQuant, k family) */
int mo_k4_row_to_f32(const uint8_t* payload, int64_t rows, int64_t cols, int64_t row, float* dst) {
    mo_k4_layout L;
    if (mo_k4_layout_for(rows, cols, &L) != 0) return -1;
    if (row < 0 || row >= rows) return -2;
    int8_t q[32];
    for (int64_t b = 0; b < L.blocks_per_row; b++) {
        int64_t col = b * 32;
        int64_t n = cols - col;
        if (n <= 0) break;
        if (n > 32) n = 32;
        float scale = k4_block_scale(payload, &L, row, b);
        if (scale == 0.0f) {
            for (int64_t i = 0; i < n; i++) dst[col + i] = 0.0f;
            continue;
        }
        k4_decode_block(payload, &L, row, b, q);
        for (int64_t i = 0; i < n; i++) dst[col + i] = (float)q[i] * scale;
    }
    return 0;
}

/* internal/backend/simd/matvec_quant.go:746-797 (quantizeVecBlocksInto):
 * per 32-block scale = maxAbs/127 (fp32 div), inv = 1/scale,
 * q = clamp(round_half_away(v*inv), +/-127); zero block -> scale 0, q 0. */
void mo_quantize_vec_blocks(const float* x, int64_t n, int64_t blocks, int8_t* q, float* scales) {
    memset(q, 0, (size_t)(blocks * 32));
    memset(scales, 0, sizeof(float) * (size_t)blocks);
    for (int64_t b = 0; b < blocks; b++) {
        int64_t base = b * 32;
        float maxabs = 0.0f;
        for (int i = 0; i < 32; i++) {
            int64_t idx = base + i;
            if (idx >= n) continue;
            float v = x[idx];
            if (v < 0) v = -v;
            if (v > maxabs) maxabs = v;
        }
        if (maxabs == 0.0f) continue;
        float scale = maxabs / 127.0f;
        scales[b] = scale;
        float inv = 1.0f / scale;
        for (int i = 0; i < 32; i++) {
            int64_t idx = base + i;
            if (idx >= n) continue;
            int32_t qq = go_round_f32(x[idx] * inv);
            if (qq > 127) qq = 127; else if (qq < -127) qq = -127;
            q[base + i] = (int8_t)qq;
        }
    }
}

/* internal/backend/simd/matvec_quant.go:256-296 (matVecRangeQuantCached, useInt8):
 * sum += float32(dot) * (scale * xScale), blocks in order, skipping zero scales;
 * dotInt8Int16 (:727-744) is an exact int32 dot. */
int mo_k4_matvec_w4a8_q(const uint8_t* payload, int64_t rows, int64_t cols,
                        const int8_t* qx, const float* xscales, float* y) {
    mo_k4_layout L;
    if (mo_k4_layout_for(rows, cols, &L) != 0) return -1;
    const int64_t bpr = L.blocks_per_row;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float sum = 0.0f;
        int8_t q[32];
        for (int64_t b = 0; b < bpr; b++) {
            int64_t col = b * 32;
            if (cols - col <= 0) break;
            float scale = k4_block_scale(payload, &L, r, b);
            if (scale == 0.0f) continue;
            float xs = xscales[b];
            if (xs == 0.0f) continue;
            k4_decode_block(payload, &L, r, b, q);
            int32_t dot = 0;
            for (int i = 0; i < 32; i++) dot += (int32_t)q[i] * (int32_t)qx[col + i];
            sum += (float)dot * (scale * xs);
        }
        y[r] = sum;
    }
    return 0;
}

/* internal/backend/simd/matvec.go:154-173 (matVecWithQuant: quantise x when AVX2) */
int mo_k4_matvec_w4a8(const uint8_t* payload, int64_t rows, int64_t cols, const float* x, float* y) {
    int64_t blocks = (cols + 31) / 32;
    int8_t* q = (int8_t*)malloc((size_t)(blocks * 32));
    float* s = (float*)malloc(sizeof(float) * (size_t)blocks);
    if (!q || !s) { free(q); free(s); return -3; }
    mo_quantize_vec_blocks(x, cols, blocks, q, s);
    int rc = mo_k4_matvec_w4a8_q(payload, rows, cols, q, s, y);
    free(q);
    free(s);
    return rc;
}

/* internal/backend/simd/matvec_quant.go:256-296 (useInt8 == false branch) with
 * dotInt8Float32Scalar (:681-687): sum += scale * sum_i(float32(q_i) * x_i). */
int mo_k4_matvec_w4a32(const uint8_t* payload, int64_t rows, int64_t cols, const float* x, float* y) {
    mo_k4_layout L;
    if (mo_k4_layout_for(rows, cols, &L) != 0) return -1;
    const int64_t bpr = L.blocks_per_row;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float sum = 0.0f;
        int8_t q[32];
        for (int64_t b = 0; b < bpr; b++) {
            int64_t col = b * 32;
            int64_t n = cols - col;
            if (n <= 0) break;
            if (n > 32) n = 32;
            float scale = k4_block_scale(payload, &L, r, b);
            if (scale == 0.0f) continue;
            k4_decode_block(payload, &L, r, b, q);
            float d = 0.0f;
            for (int64_t i = 0; i < n; i++) d += (float)q[i] * x[col + i];
            sum += scale * d;
        }
        y[r] = sum;
    }
    return 0;
}

/* Dot: internal/backend/simd/ops.go:26-33 dispatch;
 * AVX-512 internal/backend/simd/ops_avx512.go:27-90 (4 x 16-lane FMA accumulators
 * over 64-wide steps, then a 32-wide step on acc0/acc1, a 16-wide step on acc0,
 * then tmp0[0..15]+tmp1[..]+tmp2[..]+tmp3[..] left to right, then scalar tail);
 * AVX2 internal/backend/simd/ops_avx2.go:25-51 (2 x 8-lane over 16-wide steps,
 * one optional 8-wide step on acc0, acc0+=acc1 lane-wise, 8 lanes left to right);
 * scalar ops.go:49-55. */
float mo_dot(int isa, const float* a, const float* b, int64_t n) {
    if (isa == MO_ISA_AVX512) {
        if (n == 0) return 0.0f;
        float acc[4][16];
        memset(acc, 0, sizeof acc);
        int64_t i = 0;
        for (; i + 64 <= n; i += 64)
            for (int j = 0; j < 4; j++)
                for (int l = 0; l < 16; l++)
                    acc[j][l] = fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        for (; i + 32 <= n; i += 32)
            for (int j = 0; j < 2; j++)
                for (int l = 0; l < 16; l++)
                    acc[j][l] = fmaf(a[i + 16 * j + l], b[i + 16 * j + l], acc[j][l]);
        for (; i + 16 <= n; i += 16)
            for (int l = 0; l < 16; l++) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
        float sum = acc[0][0];
        for (int k = 1; k < 64; k++) sum += acc[k / 16][k % 16];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    if (isa == MO_ISA_AVX2) {
        if (n == 0) return 0.0f;
        float a0[8] = {0}, a1[8] = {0};
        int64_t i = 0;
        for (; i + 16 <= n; i += 16)
            for (int l = 0; l < 8; l++) {
                a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
                a1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], a1[l]);
            }
        if (i + 8 <= n) {
            for (int l = 0; l < 8; l++) a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
            i += 8;
        }
        for (int l = 0; l < 8; l++) a0[l] = a0[l] + a1[l];
        float sum = a0[0];
        for (int l = 1; l < 8; l++) sum += a0[l];
        for (; i < n; i++) sum += a[i] * b[i];
        return sum;
    }
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* RMSNorm: internal/backend/simd/ops_avx512.go:92-130 (16 lanes),
 * internal/backend/simd/ops_avx2.go:54-95 (8 lanes), internal/backend/simd/ops.go:70-81
 * (scalar).  Lane-striped FMA sum of squares, lanes added left to right, scalar
 * tail, mean = sum/float32(n), scale = 1/float32(sqrt(float64(mean+eps))),
 * dst = (src*scale)*w. */
void mo_rmsnorm(int isa, float* dst, const float* src, const float* w, int64_t n, float eps) {
    if (n == 0) return;
    float sum;
    int64_t i = 0;
    if (isa == MO_ISA_AVX512 || isa == MO_ISA_AVX2) {
        const int lanes = isa == MO_ISA_AVX512 ? 16 : 8;
        float acc[16] = {0};
        for (; i + lanes <= n; i += lanes)
            for (int l = 0; l < lanes; l++) acc[l] = fmaf(src[i + l], src[i + l], acc[l]);
        sum = acc[0];
        for (int l = 1; l < lanes; l++) sum += acc[l];
    } else {
        sum = 0.0f;
    }
    for (; i < n; i++) sum += src[i] * src[i];
    float mean = sum / (float)n;
    float scale = 1.0f / (float)sqrt((double)(mean + eps));
    for (int64_t k = 0; k < n; k++) dst[k] = (src[k] * scale) * w[k];
}

/* internal/backend/simd/ops.go:108-150 (fastExp, scalar; used by Softmax). */
float mo_fast_exp(float x) {
    if (x > 88.0f) return 3.4028235e38f;
    if (x < -88.0f) return 0.0f;
    const float ln2 = 0.693147180559945309417f;
    const float ln2inv = 1.44269504088896340736f;
    int32_t k = (int32_t)(x * ln2inv + 0.5f);
    if (x < 0) k = (int32_t)(x * ln2inv - 0.5f);
    float r = x - (float)k * ln2;
    float r2 = r * r;
    float r3 = r2 * r;
    float r4 = r2 * r2;
    float poly = 1.0f + r + r2 * 0.5f + r3 * 0.16666667f + r4 * 0.041666667f + (r4 * r) * 0.008333333f;
    uint32_t e = (uint32_t)(k + 127) << 23;
    return poly * u2f(e);
}

/* internal/backend/simd/ops.go:83-106 (Softmax): max, fastExp, ordered sum,
 * sum==0 guard, x *= 1/sum. */
void mo_softmax(float* x, int64_t n) {
    if (n == 0) return;
    float maxv = x[0];
    for (int64_t i = 1; i < n; i++) if (x[i] > maxv) maxv = x[i];
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = mo_fast_exp(x[i] - maxv);
        x[i] = v;
        sum += v;
    }
    if (sum == 0.0f) return;
    float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; i++) x[i] *= inv;
}

/* internal/backend/simd/ops_avx2.go:98-128 (fastExpVec), one lane: clamp to
 * [-88,88], k = RoundToEven(x*ln2inv), r = x - k*ln2 (no FMA),
 * poly = ((((1+r)+r2*c2)+r3*c3)+r4*c4)+r5*c5, times 2^k by exponent bits. */
float mo_fast_exp_vec_lane(float x) {
    const float ln2 = 0.693147180559945309417f;
    const float ln2inv = 1.44269504088896340736f;
    if (x < -88.0f) x = -88.0f;
    if (x > 88.0f) x = 88.0f;
    float kf = nearbyintf(x * ln2inv); /* default rounding mode: to nearest even */
    int32_t k = (int32_t)kf;
    kf = (float)k;
    float r = x - kf * ln2;
    float r2 = r * r;
    float r3 = r2 * r;
    float r4 = r2 * r2;
    float r5 = r4 * r;
    float poly = 1.0f + r;
    poly = poly + r2 * 0.5f;
    poly = poly + r3 * 0.16666667f;
    poly = poly + r4 * 0.041666667f;
    poly = poly + r5 * 0.008333333f;
    uint32_t e = (uint32_t)(k + 127) << 23;
    return poly * u2f(e);
}

/* internal/backend/simd/ops_avx2.go:131-141 (fastSigmoidVec, fastSiluVec):
 * silu(x) = x * (1 / (1 + fastExpVec(0 - x))). */
float mo_fast_silu_vec_lane(float x) {
    float e = mo_fast_exp_vec_lane(0.0f - x);
    float sig = 1.0f / (1.0f + e);
    return x * sig;
}

/* internal/backend/simd/ffn.go:72-90 (SiLU branch): act = fastSiluVec(gate)*up
 * for 8-wide chunks; scalar tail Silu(gate)*up (ops.go:154-185, fastExp). */
void mo_silu_mul(float* act, const float* gate, const float* up, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) act[i + l] = mo_fast_silu_vec_lane(gate[i + l]) * up[i + l];
    for (; i < n; i++) {
        float g = gate[i];
        float sig;
        if (g > 10.0f) sig = 1.0f;
        else if (g < -10.0f) sig = 0.0f;
        else sig = 1.0f / (1.0f + mo_fast_exp(-g));
        act[i] = (g * sig) * up[i];
    }
}

/* internal/backend/simd/loader.go:1604-1612 (invFreq[i] = 1/base^(2i/rot), f64)
 * and internal/backend/simd/ops_avx512.go:132-160 (cos/sin = float32(cos/sin(f64
 * pos*invFreq))), attention factor 1 (no multiply). */
void mo_rope_tables(double base, int rot_dim, int pos, float* cos_out, float* sin_out) {
    if (base <= 0) base = 10000;
    int half = rot_dim / 2;
    for (int i = 0; i < half; i++) {
        double power = (double)(2 * i) / (double)rot_dim;
        double inv = 1.0 / pow(base, power);
        double angle = (double)pos * inv;
        cos_out[i] = (float)cos(angle);
        sin_out[i] = (float)sin(angle);
    }
}

/* internal/backend/simd/ops_avx512.go:162-190 / ops_avx2.go:188-214 vector body:
 * y0 = x0*c - x1*s (no FMA), y1 = MulAdd(x0, s, x1*c) (FMA). */
void mo_apply_rope(float* x, int n_head, int head_dim, int half, const float* c, const float* s) {
    for (int h = 0; h < n_head; h++) {
        float* lo = x + (int64_t)h * head_dim;
        float* hi = lo + half;
        for (int i = 0; i < half; i++) {
            float x0 = lo[i], x1 = hi[i];
            lo[i] = x0 * c[i] - x1 * s[i];
            hi[i] = fmaf(x0, s[i], x1 * c[i]);
        }
    }
}

/* internal/backend/simd/attnpool.go:77-153 (RunAttnHeads, f32 cache, no ring,
 * no softcap): score_t = Dot(q_h, k_t)*scale, Softmax, out_d = sum_t p_t*v_t,d in
 * t order (no FMA).  kvHead = h*kvHeads/nHead. */
void mo_attn_heads(int isa, const float* q, const float* ck, const float* cv, float* out,
                   int pos, int start, int kv_stride, int head_dim, int n_head, int kv_heads, float scale) {
    int win = pos - start + 1;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int h = 0; h < n_head; h++) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)win);
        int kvh = h * kv_heads / n_head;
        const float* qh = q + (int64_t)h * head_dim;
        for (int t = start; t <= pos; t++) {
            const float* kt = ck + (int64_t)t * kv_stride + (int64_t)kvh * head_dim;
            scores[t - start] = mo_dot(isa, qh, kt, head_dim) * scale;
        }
        mo_softmax(scores, win);
        for (int d = 0; d < head_dim; d++) {
            float sum = 0.0f;
            for (int t = start; t <= pos; t++)
                sum += scores[t - start] * cv[(int64_t)t * kv_stride + (int64_t)kvh * head_dim + d];
            out[(int64_t)h * head_dim + d] = sum;
        }
        free(scores);
    }
}

/* RunAttnHeads over an f16 KV cache (internal/backend/simd/attnpool.go:103-106,
 * :127-135; the cache written by StoreKV's Float32ToFloat16Slice,
 * ops_runtime.go:112-131): scores = DotF16(q, k) * scale, where DotF16 is the
 * scalar sequential sum of q_i * f16(k_i) in every ISA (ops.go:35-46); the V
 * sum adds p_t * f16(v_t) in key order.  Caches hold Mantle's truncating f16. */
void mo_attn_heads_f16(const float* q, const uint16_t* ck, const uint16_t* cv, float* out, int pos, int start,
                       int kv_stride, int head_dim, int n_head, int kv_heads, float scale) {
    int win = pos - start + 1;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int h = 0; h < n_head; h++) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)win);
        int kvh = h * kv_heads / n_head;
        const float* qh = q + (int64_t)h * head_dim;
        for (int t = start; t <= pos; t++) {
            const uint16_t* kt = ck + (int64_t)t * kv_stride + (int64_t)kvh * head_dim;
            float sum = 0.0f;
            for (int i = 0; i < head_dim; i++) sum += qh[i] * mo_f16_to_f32(kt[i]);
            scores[t - start] = sum * scale;
        }
        mo_softmax(scores, win);
        for (int d = 0; d < head_dim; d++) {
            float sum = 0.0f;
            for (int t = start; t <= pos; t++)
                sum += scores[t - start] * mo_f16_to_f32(cv[(int64_t)t * kv_stride + (int64_t)kvh * head_dim + d]);
            out[(int64_t)h * head_dim + d] = sum;
        }
        free(scores);
    }
}

/* internal/backend/simd/ops_runtime.go:132-168 storeQ8: maxAbs over the whole
 * row by comparisons; zero row -> scale 0 and zeros; scale = maxAbs / 127,
 * inv = 127 / maxAbs (both float32 divisions); q = int32(v*inv + 0.5), or
 * int32(v*inv - 0.5) for v < 0 (Go does not fuse these: GOAMD64=v1), clamped
 * to +-127.  Go's float32 -> int32 on amd64 is CVTTSS2SL: truncation toward
 * zero, INT32_MIN for NaN or out-of-range values (then clamped to -127). */
static int32_t go_f32_to_i32_amd64(float r) {
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return INT32_MIN;
    return (int32_t)r;
}

void mo_store_q8(const float* src, int8_t* dst, float* scale_out, int64_t n) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = src[i];
        if (v < 0) {
            if (-v > max_abs) max_abs = -v;
        } else if (v > max_abs) {
            max_abs = v;
        }
    }
    if (max_abs == 0.0f) {
        *scale_out = 0.0f;
        for (int64_t i = 0; i < n; i++) dst[i] = 0;
        return;
    }
    *scale_out = max_abs / 127.0f;
    float inv = 127.0f / max_abs;
    for (int64_t i = 0; i < n; i++) {
        float v = src[i];
        float t = v * inv;
        float r = v < 0 ? t - 0.5f : t + 0.5f;
        int32_t q = go_f32_to_i32_amd64(r);
        if (q > 127) q = 127;
        else if (q < -127) q = -127;
        dst[i] = (int8_t)q;
    }
}

/* internal/backend/simd/attnpool.go:100-102 (DotQ8, ops.go:240-246: scalar
 * sum += a*float32(b), then sum*scale; times ctx.Scale) and :122-130 (sum +=
 * scores[t] * float32(q) * scale[t], evaluated left to right). */
void mo_attn_heads_q8(const float* q, const int8_t* ck, const int8_t* cv, const float* ks, const float* vs,
                      float* out, int pos, int start, int kv_stride, int head_dim, int n_head, int kv_heads,
                      float scale) {
    int win = pos - start + 1;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int h = 0; h < n_head; h++) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)win);
        int kvh = h * kv_heads / n_head;
        const float* qh = q + (int64_t)h * head_dim;
        for (int t = start; t <= pos; t++) {
            const int8_t* kt = ck + (int64_t)t * kv_stride + (int64_t)kvh * head_dim;
            float sum = 0.0f;
            for (int i = 0; i < head_dim; i++) sum += qh[i] * (float)kt[i];
            float dq = sum * ks[t];
            scores[t - start] = dq * scale;
        }
        mo_softmax(scores, win);
        for (int d = 0; d < head_dim; d++) {
            float sum = 0.0f;
            for (int t = start; t <= pos; t++) {
                float pq = scores[t - start] * (float)cv[(int64_t)t * kv_stride + (int64_t)kvh * head_dim + d];
                sum += pq * vs[t];
            }
            out[(int64_t)h * head_dim + d] = sum;
        }
        free(scores);
    }
}

/* internal/backend/simd/attnpool.go:77-153 (RunAttnHeads), every cache-type
 * pair and the ring / window placement: useRing = 0 < cacheLen < pos + 1,
 * cachePos = t % cacheLen; scores by Dot (f32, ISA order), DotF16 (f16,
 * scalar) or DotQ8 (q8_0: scalar sum * scale_t, ops.go:240-246) times
 * scale; Softmax; the V sum in key order with p * v, p * f16(v) or
 * (p * q) * s_t. */
void mo_attn_heads_mixed(int isa, const float* q, int k_type, const void* ck, const float* ks, int v_type,
                         const void* cv, const float* vs, float* out, int pos, int start, int cache_len,
                         int kv_stride, int head_dim, int n_head, int kv_heads, float scale) {
    int win = pos - start + 1;
    int ring = cache_len > 0 && cache_len < pos + 1;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int h = 0; h < n_head; h++) {
        float* scores = (float*)malloc(sizeof(float) * (size_t)win);
        int kvh = h * kv_heads / n_head;
        const float* qh = q + (int64_t)h * head_dim;
        for (int t = start; t <= pos; t++) {
            int cp = ring ? t % cache_len : t;
            int64_t off = (int64_t)cp * kv_stride + (int64_t)kvh * head_dim;
            float sc;
            if (k_type == MO_KV_Q8) {
                const int8_t* kt = (const int8_t*)ck + off;
                float sum = 0.0f;
                for (int i = 0; i < head_dim; i++) sum += qh[i] * (float)kt[i];
                sc = sum * ks[cp];
            } else if (k_type == MO_KV_F16) {
                const uint16_t* kt = (const uint16_t*)ck + off;
                float sum = 0.0f;
                for (int i = 0; i < head_dim; i++) sum += qh[i] * mo_f16_to_f32(kt[i]);
                sc = sum;
            } else {
                sc = mo_dot(isa, qh, (const float*)ck + off, head_dim);
            }
            scores[t - start] = sc * scale;
        }
        mo_softmax(scores, win);
        for (int d = 0; d < head_dim; d++) {
            float sum = 0.0f;
            for (int t = start; t <= pos; t++) {
                int cp = ring ? t % cache_len : t;
                int64_t off = (int64_t)cp * kv_stride + (int64_t)kvh * head_dim + d;
                float p = scores[t - start];
                if (v_type == MO_KV_Q8) sum += (p * (float)((const int8_t*)cv)[off]) * vs[cp];
                else if (v_type == MO_KV_F16) sum += p * mo_f16_to_f32(((const uint16_t*)cv)[off]);
                else sum += p * ((const float*)cv)[off];
            }
            out[(int64_t)h * head_dim + d] = sum;
        }
        free(scores);
    }
}

/* internal/backend/simd/runtime_greedy.go:70-82 (argmaxHost: strict '>'). */
int64_t mo_argmax(const float* x, int64_t n) {
    if (n <= 0) return -1;
    int64_t best = 0;
    float bv = x[0];
    for (int64_t i = 1; i < n; i++)
        if (x[i] > bv) { bv = x[i]; best = i; }
    return best;
}

/* ------------------------------------------------------------------------- */
/* bf16 dense GEMV: internal/backend/simd/matvec.go:406-416 (matVecRangeBF16
 * dispatch), :419-488 (Scalar), :490-713 (SIMD = AVX2), :715-979 (AVX512);
 * bf16 -> f32 is internal/backend/core/dtype.go:67-69 (bits << 16), the f32 ->
 * bf16 packer pkg/mcf/pack.go:789-793 (round to nearest even).
 *
 * Every row-grouping (4 / 2 / 1 rows at a time) of a path evaluates each row
 * in the same order, so rows are independent here.  Go does not fuse the
 * scalar a*b + c (GOAMD64=v1); archsimd MulAdd is an FMA. */

float mo_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t mo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float bf16_row_avx512(const uint16_t* row, const float* x, int64_t c) {
    /* matvec.go:738-834: acc (16 lanes) takes j = 32k + l, acc_2 j = 32k + 16 + l;
     * a remaining 16-chunk goes into acc; acc += acc_2; lanes summed in order;
     * the scalar tail follows. */
    float acc[16] = {0}, acc2[16] = {0};
    int64_t j = 0;
    for (; j + 32 <= c; j += 32)
        for (int l = 0; l < 16; l++) {
            acc[l] = fmaf(mo_bf16_to_f32(row[j + l]), x[j + l], acc[l]);
            acc2[l] = fmaf(mo_bf16_to_f32(row[j + 16 + l]), x[j + 16 + l], acc2[l]);
        }
    for (; j + 16 <= c; j += 16)
        for (int l = 0; l < 16; l++) acc[l] = fmaf(mo_bf16_to_f32(row[j + l]), x[j + l], acc[l]);
    float sum = 0.0f;
    for (int l = 0; l < 16; l++) sum += acc[l] + acc2[l];
    for (; j < c; j++) sum += mo_bf16_to_f32(row[j]) * x[j];
    return sum;
}

static float bf16_row_avx2(const uint16_t* row, const float* x, int64_t c) {
    /* matvec.go:513-610: one 8-lane accumulator, lane l takes j = 8m + l (the
     * 16-wide loop feeds it twice per step); sum += t0 + t1 + ... + t7 left to
     * right; the scalar tail follows. */
    float acc[8] = {0};
    int64_t j = 0;
    for (; j + 8 <= c; j += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(mo_bf16_to_f32(row[j + l]), x[j + l], acc[l]);
    float h = acc[0];
    for (int l = 1; l < 8; l++) h += acc[l];
    float sum = 0.0f;
    sum += h;
    for (; j < c; j++) sum += mo_bf16_to_f32(row[j]) * x[j];
    return sum;
}

static float bf16_row_scalar(const uint16_t* row, const float* x, int64_t c) {
    /* matvec.go:419-445: sum += p0 + p1 + ... + p7 per 8-chunk, then the tail. */
    float sum = 0.0f;
    int64_t j = 0;
    for (; j + 7 < c; j += 8) {
        float g = mo_bf16_to_f32(row[j]) * x[j];
        for (int e = 1; e < 8; e++) g += mo_bf16_to_f32(row[j + e]) * x[j + e];
        sum += g;
    }
    for (; j < c; j++) sum += mo_bf16_to_f32(row[j]) * x[j];
    return sum;
}

void mo_bf16_matvec(int isa, const uint16_t* w, int64_t rows, int64_t cols, const float* x, float* y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const uint16_t* row = w + r * cols;
        y[r] = isa == MO_ISA_AVX512 ? bf16_row_avx512(row, x, cols)
             : isa == MO_ISA_AVX2   ? bf16_row_avx2(row, x, cols)
                                    : bf16_row_scalar(row, x, cols);
    }
}

/* ------------------------------------------------------------------------- */
/* Qwen3 decoder: internal/backend/simd/runtime_greedy.go:12-67 (ForwardTokenGreedy),
 * internal/backend/simd/runtime_decode.go:29-203 (runDecoderLayers),
 * internal/backend/simd/attn.go:83-419 (CPU branch), internal/backend/simd/ffn.go:18-91. */

struct mo_model {
    mo_config c;
    mo_weights w;
    int max_ctx;
    int pos;
    int64_t q_dim, kv_dim;
    float *x, *tmp, *q, *k, *v, *attn, *proj, *up, *gate, *act, *down, *logits;
    float *cache_k, *cache_v; /* [L][max_ctx][kv_dim] */
    float *kscale, *vscale;   /* q8_0: [L][max_ctx] */
    float *cosv, *sinv;
    int8_t* qx;
    float* qs;
};

mo_model* mo_model_create(const mo_config* cfg, const mo_weights* w, int max_ctx) {
    mo_model* m = (mo_model*)calloc(1, sizeof(mo_model));
    if (!m) return NULL;
    m->c = *cfg;
    m->w = *w;
    m->max_ctx = max_ctx;
    m->q_dim = (int64_t)cfg->n_heads * cfg->head_dim;
    m->kv_dim = (int64_t)cfg->n_kv_heads * cfg->head_dim;
    int64_t d = cfg->d_model, f = cfg->ffn;
    int64_t big = d > m->q_dim ? d : m->q_dim;
    if (f > big) big = f;
    m->x = calloc((size_t)d, 4);
    m->tmp = calloc((size_t)d, 4);
    m->q = calloc((size_t)m->q_dim, 4);
    m->k = calloc((size_t)m->kv_dim, 4);
    m->v = calloc((size_t)m->kv_dim, 4);
    m->attn = calloc((size_t)m->q_dim, 4);
    m->proj = calloc((size_t)d, 4);
    m->up = calloc((size_t)f, 4);
    m->gate = calloc((size_t)f, 4);
    m->act = calloc((size_t)f, 4);
    m->down = calloc((size_t)d, 4);
    m->logits = calloc((size_t)cfg->vocab, 4);
    /* f32 cache, or uint16 f16 / int8 values in the same [L][max_ctx][kv_dim] slots */
    m->cache_k = calloc((size_t)(cfg->n_layers * (int64_t)max_ctx * m->kv_dim), 4);
    m->cache_v = calloc((size_t)(cfg->n_layers * (int64_t)max_ctx * m->kv_dim), 4);
    m->kscale = calloc((size_t)(cfg->n_layers * (int64_t)max_ctx), 4);
    m->vscale = calloc((size_t)(cfg->n_layers * (int64_t)max_ctx), 4);
    m->cosv = calloc((size_t)cfg->head_dim, 4);
    m->sinv = calloc((size_t)cfg->head_dim, 4);
    m->qx = calloc((size_t)((big + 31) / 32 * 32), 1);
    m->qs = calloc((size_t)((big + 31) / 32), 4);
    if (!m->x || !m->cache_k || !m->cache_v || !m->logits || !m->qx) { mo_model_free(m); return NULL; }
    return m;
}

void mo_model_free(mo_model* m) {
    if (!m) return;
    free(m->x); free(m->tmp); free(m->q); free(m->k); free(m->v); free(m->attn);
    free(m->proj); free(m->up); free(m->gate); free(m->act); free(m->down); free(m->logits);
    free(m->cache_k); free(m->cache_v); free(m->kscale); free(m->vscale); free(m->cosv); free(m->sinv); free(m->qx); free(m->qs);
    free(m);
}

void mo_model_reset(mo_model* m) { m->pos = 0; }
int mo_model_pos(const mo_model* m) { return m->pos; }
void mo_model_hidden(const mo_model* m, float* out) { memcpy(out, m->x, sizeof(float) * (size_t)m->c.d_model); }

static void quant_then_matvec(mo_model* m, const uint8_t* W, int64_t rows, int64_t cols, const float* x, float* y) {
    if (m->c.wdtype == MO_W_BF16) {  /* matvec.go:154-172: no activation quantisation for bf16 */
        mo_bf16_matvec(m->c.isa, (const uint16_t*)W, rows, cols, x, y);
        return;
    }
    int64_t blocks = (cols + 31) / 32;
    mo_quantize_vec_blocks(x, cols, blocks, m->qx, m->qs);
    mo_k4_matvec_w4a8_q(W, rows, cols, m->qx, m->qs, y);
}

/* The shared-activation GEMVs of Q/K/V and up/gate (attn.go:180-205,
 * ffn.go:41-57): the int8 activation is prepared once (k4); bf16 runs the
 * plain GEMV on x. */
static void shared_matvec(mo_model* m, const uint8_t* W, int64_t rows, int64_t cols, const float* x, float* y) {
    if (m->c.wdtype == MO_W_BF16) mo_bf16_matvec(m->c.isa, (const uint16_t*)W, rows, cols, x, y);
    else mo_k4_matvec_w4a8_q(W, rows, cols, m->qx, m->qs, y);
}

int64_t mo_model_forward_greedy(mo_model* m, int64_t tok, float* logits_out) {
    const mo_config* c = &m->c;
    const int64_t d = c->d_model, hd = c->head_dim, f = c->ffn;
    if (tok < 0 || tok >= c->vocab) return -1;
    if (m->pos >= m->max_ctx) return -2;
    const int pos = m->pos;
    /* runtime_decode.go:29-51: x = Embeddings.RowTo(tok) */
    if (c->wdtype == MO_W_BF16) {
        const uint16_t* er = (const uint16_t*)m->w.embed + tok * d;
        for (int64_t i = 0; i < d; i++) m->x[i] = mo_bf16_to_f32(er[i]);
    } else {
        mo_k4_row_to_f32(m->w.embed, c->vocab, d, tok, m->x);
    }
    const float scale = (float)(1.0 / sqrt((double)hd)); /* attn.go:311-314 */
    mo_rope_tables(c->rope_base, (int)hd, pos, m->cosv, m->sinv);
    for (int l = 0; l < c->n_layers; l++) {
        /* runtime_decode.go:107 RMSNorm(attn) */
        mo_rmsnorm(c->isa, m->tmp, m->x, m->w.attn_norm[l], d, c->eps);
        /* attn.go:180-205: one PrepareQuantVec shared by Q, K, V */
        int64_t blocks = (d + 31) / 32;
        if (c->wdtype != MO_W_BF16) mo_quantize_vec_blocks(m->tmp, d, blocks, m->qx, m->qs);
        shared_matvec(m, m->w.wq[l], m->q_dim, d, m->tmp, m->q);
        shared_matvec(m, m->w.wk[l], m->kv_dim, d, m->tmp, m->k);
        shared_matvec(m, m->w.wv[l], m->kv_dim, d, m->tmp, m->v);
        /* attn.go:265-286 per-head RMSNorm */
        for (int h = 0; h < c->n_heads; h++)
            mo_rmsnorm(c->isa, m->q + h * hd, m->q + h * hd, m->w.q_norm[l], hd, c->eps);
        for (int h = 0; h < c->n_kv_heads; h++)
            mo_rmsnorm(c->isa, m->k + h * hd, m->k + h * hd, m->w.k_norm[l], hd, c->eps);
        /* attn.go:293-309 RoPE */
        mo_apply_rope(m->q, c->n_heads, (int)hd, (int)hd / 2, m->cosv, m->sinv);
        mo_apply_rope(m->k, c->n_kv_heads, (int)hd, (int)hd / 2, m->cosv, m->sinv);
        /* ops_runtime.go:40-131 StoreKV + RunAttnHeads */
        float* ck = m->cache_k + (int64_t)l * m->max_ctx * m->kv_dim;
        float* cv = m->cache_v + (int64_t)l * m->max_ctx * m->kv_dim;
        float* ks = m->kscale + (int64_t)l * m->max_ctx;
        float* vs = m->vscale + (int64_t)l * m->max_ctx;
        /* ops_runtime.go:112-131 StoreKV: each row in its cache's type (loader.go:640-668) */
        int64_t row = (int64_t)pos * m->kv_dim;
        if (c->kv_k == MO_KV_Q8) mo_store_q8(m->k, (int8_t*)ck + row, ks + pos, m->kv_dim);
        else if (c->kv_k == MO_KV_F16)
            for (int64_t i = 0; i < m->kv_dim; i++) ((uint16_t*)ck)[row + i] = mo_f32_to_f16(m->k[i]);
        else memcpy(ck + row, m->k, sizeof(float) * (size_t)m->kv_dim);
        if (c->kv_v == MO_KV_Q8) mo_store_q8(m->v, (int8_t*)cv + row, vs + pos, m->kv_dim);
        else if (c->kv_v == MO_KV_F16)
            for (int64_t i = 0; i < m->kv_dim; i++) ((uint16_t*)cv)[row + i] = mo_f32_to_f16(m->v[i]);
        else memcpy(cv + row, m->v, sizeof(float) * (size_t)m->kv_dim);
        if (c->kv_k == c->kv_v && c->kv_k == MO_KV_Q8)
            mo_attn_heads_q8(m->q, (int8_t*)ck, (int8_t*)cv, ks, vs, m->attn, pos, 0, (int)m->kv_dim, (int)hd,
                             c->n_heads, c->n_kv_heads, scale);
        else if (c->kv_k == c->kv_v && c->kv_k == MO_KV_F16)
            mo_attn_heads_f16(m->q, (uint16_t*)ck, (uint16_t*)cv, m->attn, pos, 0, (int)m->kv_dim, (int)hd,
                              c->n_heads, c->n_kv_heads, scale);
        else if (c->kv_k == c->kv_v)
            mo_attn_heads(c->isa, m->q, ck, cv, m->attn, pos, 0, (int)m->kv_dim, (int)hd, c->n_heads, c->n_kv_heads,
                          scale);
        else
            mo_attn_heads_mixed(c->isa, m->q, c->kv_k, ck, ks, c->kv_v, cv, vs, m->attn, pos, 0, 0, (int)m->kv_dim,
                                (int)hd, c->n_heads, c->n_kv_heads, scale);
        /* attn.go:417 Wo (re-quantises attnOut) */
        quant_then_matvec(m, m->w.wo[l], d, m->q_dim, m->attn, m->proj);
        /* runtime.go:278-289 addResidual */
        for (int64_t i = 0; i < d; i++) m->x[i] += m->proj[i];
        /* runtime_decode.go:159 RMSNorm(ffn) ; ffn.go:41-57 shared qx for up, gate */
        mo_rmsnorm(c->isa, m->tmp, m->x, m->w.ffn_norm[l], d, c->eps);
        if (c->wdtype != MO_W_BF16) mo_quantize_vec_blocks(m->tmp, d, blocks, m->qx, m->qs);
        shared_matvec(m, m->w.w_up[l], f, d, m->tmp, m->up);
        shared_matvec(m, m->w.w_gate[l], f, d, m->tmp, m->gate);
        mo_silu_mul(m->act, m->gate, m->up, f);
        quant_then_matvec(m, m->w.w_down[l], d, f, m->act, m->down);
        for (int64_t i = 0; i < d; i++) m->x[i] += m->down[i];
    }
    /* runtime_greedy.go:53 FusedRMSNormMatVec fallback (ops_fusion.go:4-18) */
    mo_rmsnorm(c->isa, m->tmp, m->x, m->w.final_norm, d, c->eps);
    quant_then_matvec(m, m->w.lm_head, c->vocab, d, m->tmp, m->logits);
    if (logits_out) memcpy(logits_out, m->logits, sizeof(float) * (size_t)c->vocab);
    m->pos++;
    return mo_argmax(m->logits, c->vocab);
}
