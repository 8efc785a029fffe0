/*
 * mantle_oracle.h -- CPU restatement of Mantle's CPU (archsimd) decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP backend is
 * compared against; it is never linked into, loaded by, or called from the
 * product library (mantle_amd/).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may use it.
 *
 * Every function restates one function of samcharles93/mantle (Go 1.26,
 * GOEXPERIMENT=simd); the file:line it follows is cited at the definition in
 * mantle_oracle.c.  Floating point is evaluated exactly in the order Mantle's
 * Go code evaluates it: the file is compiled with -ffp-contract=off and
 * uses fmaf() exactly where Mantle calls archsimd MulAdd.
 */
#ifndef MANTLE_ORACLE_H
#define MANTLE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CPU ISA flavours of Mantle's archsimd kernels (internal/backend/simd/tensor_cpu.go:18-24).
 * They change the reduction order of Dot and RMSNorm, hence the bits. */
enum { MO_ISA_SCALAR = 0, MO_ISA_AVX2 = 1, MO_ISA_AVX512 = 2 };

/* ---- fp16 (Mantle's truncating / flush-to-zero conversions) ---- */
uint16_t mo_f32_to_f16(float f);
float mo_f16_to_f32(uint16_t h);

/* ---- k4 layout (pkg/mcf/quant_payload.go) ---- */
typedef struct {
    int64_t rows, cols;
    int64_t blocks_per_row, super_per_row;
    int64_t super_off, sub_off, data_off; /* byte offsets inside the payload */
    int64_t size;                         /* QuantPayloadSize */
} mo_k4_layout;
int mo_k4_layout_for(int64_t rows, int64_t cols, mo_k4_layout* out);

/* ---- k4 producer (cmd/mantle/quantize.go quantizeTensor + quantizeK, bits=4) ---- */
int mo_quantize_k4(const float* src, int64_t rows, int64_t cols, uint8_t* payload);

/* ---- dequant ---- */
int mo_k4_row_to_f32(const uint8_t* payload, int64_t rows, int64_t cols, int64_t row, float* dst);
int mo_k4_block_scales(const uint8_t* payload, int64_t rows, int64_t cols, float* scales);

/* ---- activation quantiser (quantizeVecBlocksInto) ---- */
void mo_quantize_vec_blocks(const float* x, int64_t n, int64_t blocks, int8_t* q, float* scales);

/* ---- k4 GEMV ---- */
/* W4A8: Mantle's AVX2+ path (int8 activations, exact int dot, ordered fp32 block sum). */
int mo_k4_matvec_w4a8(const uint8_t* payload, int64_t rows, int64_t cols, const float* x, float* y);
/* Same, with an already-quantised activation (PrepareQuantVec shared across Q/K/V, up/gate). */
int mo_k4_matvec_w4a8_q(const uint8_t* payload, int64_t rows, int64_t cols,
                        const int8_t* qx, const float* xscales, float* y);
/* W4A32: Mantle's non-AVX2 path (fp32 activations, scalar block dots). */
int mo_k4_matvec_w4a32(const uint8_t* payload, int64_t rows, int64_t cols, const float* x, float* y);

/* ---- bf16 dense GEMV (fp32 activations) ---- */
/* Mantle's matVecRangeBF16 in each ISA's order (AVX-512: 32 lane chains, AVX2:
 * 8, scalar: 8-term groups); bf16 -> fp32 is exact (bits << 16). */
float mo_bf16_to_f32(uint16_t b);
uint16_t mo_f32_to_bf16(float f);
void mo_bf16_matvec(int isa, const uint16_t* w, int64_t rows, int64_t cols, const float* x, float* y);

/* ---- elementwise / reductions ---- */
float mo_dot(int isa, const float* a, const float* b, int64_t n);
void mo_rmsnorm(int isa, float* dst, const float* src, const float* w, int64_t n, float eps);
float mo_fast_exp(float x);
void mo_softmax(float* x, int64_t n);
float mo_fast_exp_vec_lane(float x);
float mo_fast_silu_vec_lane(float x);
void mo_silu_mul(float* act, const float* gate, const float* up, int64_t n);
void mo_rope_tables(double base, int rot_dim, int pos, float* cos_out, float* sin_out);
void mo_apply_rope(float* x, int n_head, int head_dim, int half, const float* cosv, const float* sinv);
void mo_attn_heads(int isa, const float* q, const float* cache_k, const float* cache_v, float* out,
                   int pos, int start, int kv_stride, int head_dim, int n_head, int kv_heads, float scale);
/* The same over an f16 cache [pos][kv_stride] (DotF16 is scalar in every ISA). */
void mo_attn_heads_f16(const float* q, const uint16_t* cache_k, const uint16_t* cache_v, float* out, int pos, int start,
                       int kv_stride, int head_dim, int n_head, int kv_heads, float scale);
/* q8_0 cache (--cache-type-k/v q8_0): storeQ8 of one row of n values (one
 * scale per row), and the attention over int8 caches [pos][kv_stride] with
 * per-position scales (DotQ8 scalar order, V terms (p * q) * s). */
void mo_store_q8(const float* src, int8_t* dst, float* scale_out, int64_t n);
void mo_attn_heads_q8(const float* q, const int8_t* cache_k, const int8_t* cache_v, const float* k_scale,
                      const float* v_scale, float* out, int pos, int start, int kv_stride, int head_dim, int n_head,
                      int kv_heads, float scale);
int64_t mo_argmax(const float* x, int64_t n);
/* RunAttnHeads in general (internal/backend/simd/attnpool.go:77-153): K and V
 * caches of independent types (MO_KV_F32: float, MO_KV_F16: uint16 f16,
 * MO_KV_Q8: int8 with per-position scales ks / vs), keys t = start..pos, each
 * at cache slot t % cache_len when 0 < cache_len < pos + 1 (the ring), else t. */
enum { MO_KV_F32 = 0, MO_KV_F16 = 1, MO_KV_Q8 = 2 };
void mo_attn_heads_mixed(int isa, const float* q, int k_type, const void* cache_k, const float* ks, int v_type,
                         const void* cache_v, const float* vs, float* out, int pos, int start, int cache_len,
                         int kv_stride, int head_dim, int n_head, int kv_heads, float scale);

/* ---- Qwen3-shaped decoder (k4 weights, f32 KV cache) ---- */
typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn, vocab;
    double rope_base;
    float eps;
    int isa;
    int wdtype; /* MO_W_K4: the matrix pointers below are k4 payloads; MO_W_BF16: bf16 [rows][cols] */
    int kv_k;   /* K cache type (--cache-type-k): MO_KV_F32, MO_KV_F16 (Mantle's truncating f16), MO_KV_Q8 */
    int kv_v;   /* V cache type (--cache-type-v), independent of kv_k */
} mo_config;
enum { MO_W_K4 = 0, MO_W_BF16 = 1 };

typedef struct {
    const uint8_t* embed;       /* k4 [vocab, d] */
    const uint8_t* lm_head;     /* k4 [vocab, d]; == embed when tied */
    const float* final_norm;    /* [d] */
    const float* const* attn_norm;  /* [L][d] */
    const uint8_t* const* wq;       /* [L] k4 [nH*hd, d] */
    const uint8_t* const* wk;       /* [L] k4 [kvH*hd, d] */
    const uint8_t* const* wv;       /* [L] k4 [kvH*hd, d] */
    const float* const* q_norm;     /* [L][hd] */
    const float* const* k_norm;     /* [L][hd] */
    const uint8_t* const* wo;       /* [L] k4 [d, nH*hd] */
    const float* const* ffn_norm;   /* [L][d] */
    const uint8_t* const* w_gate;   /* [L] k4 [ffn, d] */
    const uint8_t* const* w_up;     /* [L] k4 [ffn, d] */
    const uint8_t* const* w_down;   /* [L] k4 [d, ffn] */
} mo_weights;

typedef struct mo_model mo_model;
mo_model* mo_model_create(const mo_config* cfg, const mo_weights* w, int max_ctx);
void mo_model_free(mo_model* m);
void mo_model_reset(mo_model* m);
int mo_model_pos(const mo_model* m);
/* One ForwardTokenGreedy step.  Returns the next token id (>=0) or <0 on error.
 * logits (nullable, length vocab) receives the logits of this step. */
int64_t mo_model_forward_greedy(mo_model* m, int64_t tok, float* logits);
/* Copy the residual stream x after the step (length d) -- divergence bisection aid. */
void mo_model_hidden(const mo_model* m, float* out);

void mo_set_threads(int n);
int mo_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
