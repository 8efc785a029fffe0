// kernels.h -- host-side launchers for the gfx950 kernels in kernels.hip.
// Every launcher validates its arguments on the host, enqueues on `stream`
// and returns a hipError_t; nothing here allocates or synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mantle {

// CPU ISA flavour whose reduction order the parity kernels reproduce
// (internal/backend/simd/tensor_cpu.go:18-24 selects it on the host).
enum Isa : int { kIsaScalar = 0, kIsaAvx2 = 1, kIsaAvx512 = 2 };

// One k4 matrix inside a (possibly multi-matrix) GEMV launch.  The three
// pointers are the SoA regions of the MCF k4 payload (pkg/mcf/quant_payload.go).
struct K4Mat {
    const uint8_t* nib;    // [rows][blocks_per_row][16]
    const uint8_t* sub;    // [rows][blocks_per_row] u6 in bits 0-5
    const uint16_t* sup;   // [rows][super_per_row] f16 (Mantle truncating encoding)
    int rows;
};

// Region pointers of a k4 payload that starts at `payload`.
K4Mat k4_mat_from_payload(const uint8_t* payload, int rows, int cols);
int64_t k4_payload_size(int64_t rows, int64_t cols);

enum GemvEpi : int {
    kEpiStore = 0,    // y[b][r] = sum
    kEpiResAdd = 1,   // y[r] = y[r] + sum  (residual folded into the epilogue)
    kEpiSiluMul = 2,  // two matrices (gate, up): y[r] = silu(gate_r) * up_r
    kEpiArgmax = 3,   // y[r] = sum and a 64-bit (value, -index) atomicMax key
};

// The argmax epilogue spreads its atomicMax over kArgmaxSlots keys, one per
// 128-byte line (workgroup w uses slot w % kArgmaxSlots): thousands of
// workgroups on one address serialise at the memory-side atomic unit.
constexpr int kArgmaxSlots = 64;
constexpr int kArgmaxStride = 16;  // u64 per slot

// Device-resident decode state (one per model).
struct DecodeState {
    int pos;            // next position to run
    int next_tok;       // argmax of the last step
    int n_prompt;       // positions < n_prompt take their token from prompt[]
    int pad;
    alignas(128) unsigned long long argmax_keys[kArgmaxSlots * kArgmaxStride];
};

// y = W * x with x quantised per 32-block to int8 (Mantle's W4A8 CPU path).
// kEpiArgmax: argmax_key points to kArgmaxSlots x kArgmaxStride keys, zeroed
// by the caller; the argmax is the max over the slots (finish_step does it).
// qx: [batch][blocks*32] in the even/odd permuted layout quantize_vec writes;
// xs: [batch][blocks].  outs[i] receives matrix i's rows.
hipError_t launch_k4_gemv_w4a8(const K4Mat* mats, float* const* outs, int nmat, int cols,
                               const int8_t* qx, const float* xs, int batch, GemvEpi epi,
                               unsigned long long* argmax_key, hipStream_t stream);
// The same product for n activation vectors at once on int8 MFMA (any n >= 1;
// blocks per row a multiple of 8): y[v * ldy + row] = (W x_v)[row] (kEpiStore)
// or += it (kEpiResAdd).  Bit-identical to launch_k4_gemv_w4a8 per vector.
hipError_t launch_k4_gemm_w4a8(const K4Mat& w, int cols, const int8_t* qx, const float* xs, int n, float* y, int ldy,
                               GemvEpi epi, hipStream_t stream);
// launch_k4_gemm_w4a8 for up to three matrices of one width on the same
// activations in one launch (matrix m into ys[m], all with leading dimension ldy).
hipError_t launch_k4_gemm_w4a8_multi(const K4Mat* mats, float* const* ys, int nmat, int cols, const int8_t* qx,
                                     const float* xs, int n, int ldy, GemvEpi epi, hipStream_t stream);
// Same arithmetic, but each workgroup quantises the fp32 activation x itself
// (after Mantle's RMSNorm with norm_w when non-null): no separate quantiser
// launch, and the weight loads are issued before the prologue runs.  With
// kEpiSiluMul, q_out / q_scale (nullable) also receive the output as int8
// blocks, the operand of the next W4A8 GEMV.
hipError_t launch_k4_gemv_w4a8_fused(const K4Mat* mats, float* const* outs, int nmat, int cols, const float* x,
                                     const float* norm_w, float eps, int isa, int batch, GemvEpi epi,
                                     unsigned long long* argmax_key, hipStream_t stream, int8_t* q_out = nullptr,
                                     float* q_scale = nullptr);
// launch_k4_gemv_w4a8 on an fp32 x quantised into a fixed per-device library
// array (no caller scratch, nothing allocated): cols <= kNoAllocMaxBlocks*32,
// batch <= kNoAllocMaxBatch.  Calls that overlap on one device share the array.
constexpr int kNoAllocMaxBlocks = 384;  // 12288 columns (the quantiser stages a row in 64 KiB of LDS)
constexpr int kNoAllocMaxBatch = 8;
constexpr size_t kNoAllocScratchBytes = (size_t)kNoAllocMaxBatch * kNoAllocMaxBlocks * 36;  // qx + scales
hipError_t launch_k4_gemv_w4a8_noalloc(const K4Mat& m, int cols, const float* x, float* y, int batch, int isa,
                                       hipStream_t stream);
// y = W * x with fp32 x (W4A32; tolerance-checked, not bit-exact).
hipError_t launch_k4_gemv_w4a32(const K4Mat& m, int cols, const float* x, float* y, int batch,
                                hipStream_t stream);

// Dense bf16 GEMV with fp32 x (raw-bf16 MCF weights, matvec.go:406-979), bit-exact
// to Mantle's `isa` order: y_i = W_i x for up to three matrices W_i [rows_i][cols]
// (bf16, 16-byte aligned) sharing x.  kEpiResAdd adds into y; kEpiArgmax
// (one matrix) also folds each row into argmax_key's kArgmaxSlots keys.
// cols: a multiple of 8, at most kBf16MaxCols (x is staged in LDS).
constexpr int kBf16MaxCols = 32768;
hipError_t launch_bf16_gemv(const uint16_t* const* w, float* const* y, const int* rows, int nmat, int cols,
                            const float* x, GemvEpi epi, unsigned long long* argmax_key, int isa,
                            hipStream_t stream);

// Activation quantiser (internal/backend/simd/matvec_quant.go:746-797), optionally
// preceded by Mantle's RMSNorm (weight != nullptr).  norm_out (nullable) receives
// the normalised fp32 vector.  batch rows of length n, one workgroup per row.
hipError_t launch_quantize_vec(const float* x, const float* weight, float eps, int n, int batch, int isa,
                               int8_t* qx, float* xs, float* norm_out, hipStream_t stream);

hipError_t launch_rmsnorm(float* out, const float* x, const float* weight, float eps, int n, int rows,
                          int isa, hipStream_t stream);

// Fused decode attention for one layer: per-head q/k RMSNorm, RoPE (host
// tables), KV append at *pos, scores, softmax, weighted V sum.
struct AttnArgs {
    const float* q;        // [n_head*head_dim] raw projection
    const float* k;        // [kv_heads*head_dim]
    const float* v;
    const float* q_norm;   // [head_dim] or null (no norm)
    const float* k_norm;
    float eps;
    const float* rope_cos; // [max_ctx][head_dim/2] or null (no RoPE)
    const float* rope_sin;
    const int* pos_dev;    // device position (fused) ...
    int pos_host;          // ... or a host position when pos_dev is null
    float* cache_k;        // row t of kv head g at cache + g*head_stride + t*kv_stride
    float* cache_v;
    int head_stride;       // head_dim for Mantle's [pos][kv_heads*head_dim] layout, max_ctx*head_dim head-major
    float* scores;         // [n_head][max_ctx] scratch
    float* out;            // [n_head*head_dim]
    int n_head, kv_heads, head_dim, kv_stride, max_ctx;
    float scale;
    int fused;             // 1: norm/rope/append inside, 0: q and cache are final
    int isa;
    int8_t* q_out;         // optional: out also as Mantle's int8 blocks (permuted layout) ...
    float* q_scale;        // ... and their scales, for the next W4A8 GEMV (head_dim % 32 == 0)
    int k_type, v_type;    // KvCacheType of cache_k / cache_v (--cache-type-k / --cache-type-v,
                           // cmd/mantle/run.go:183-195; independent).  f16: Mantle's truncating f16
                           // (uint16) values, split paths only.  q8_0: see k_scale below.
    int vt_stride;         // > 0: V is stored transposed, element (t, d) of kv head g at
                           // cache_v + (g*head_dim + d)*vt_stride + t (split paths only)
    unsigned* counters;    // [n_head] zeroed arrival counters of the one-launch split path (null: the
                           // library's own, for callers that serialise their launches on one stream)
    int key_base, key_ring;  // row-major caches only (fused 0, vt_stride 0), split path: the
                             // window's key t (0..pos) is cache row (key_base + t), taken
                             // mod key_ring when key_ring > 0 (RunAttnHeads' window start
                             // and ring, attnpool.go:88-99)
    const float* k_scale;  // a q8_0 cache holds int8 rows with one scale per position in k_scale /
    const float* v_scale;  // v_scale [max_ctx] (two-launch split path only).  Its step rows must
                           // already be in the cache (fused: launch_kv_append_q8 prepares and
                           // appends the q8_0 rows; this launch prepares q and the other rows)
    // Token rows (launch_attention_rows only; zero otherwise): query row r of the launch is the
    // position pos + r; its q, out, scores and q_out / q_scale start q_row, out_row,
    // scores_row and out_row elements (out_row / 32 scales) further on.
    int q_row, out_row;
    size_t scores_row;
};
hipError_t launch_attention_decode(const AttnArgs& a, hipStream_t stream);
// Attention of `rows` consecutive query positions pos .. pos+rows-1 (causal:
// row r sees keys 0 .. pos+r) on the two-launch split kernels, each row exactly
// the decode step's arithmetic at its position.  fused must be 0: q holds the
// prepared queries and the cache the rows' K / V (launch_attention_prep_rows,
// launch_kv_append_q8 with tokens).  Requires head_dim 64 / 128 and scores for
// rows * n_head * max_ctx floats (scores_row >= n_head * max_ctx).
hipError_t launch_attention_rows(const AttnArgs& a, int rows, hipStream_t stream);
// The prologue of those rows: per-head RMSNorm and RoPE of q (written to qo,
// row r at qo + r * a.out_row) and of k, and the K / V rows appended to the
// f32 / f16 caches (q8_0 sides: launch_kv_append_q8).  a.q / a.k / a.v: the
// raw projections of row 0, rows qkv_row floats apart.
hipError_t launch_attention_prep_rows(const AttnArgs& a, int rows, int qkv_row, float* qo, hipStream_t stream);
// Decode-attention kernel variant for head_dim 64 / 128 (other sizes always
// take the general kernel).  A model's captured step keeps the variant it was
// captured with.
// kAttnPathFused is the split-key path in one launch (kAttnPathSplit takes it
// past 8192 keys).
enum AttnPath : int { kAttnPathSplit = 0, kAttnPathSingle = 1, kAttnPathGeneral = 2, kAttnPathFused = 3 };
int attention_path();
bool set_attention_path(int path);

// Causal GQA attention over a whole prompt on bf16 MFMA (head_dim 128): q bf16
// [seq][n_head][128], k / v bf16 [seq][kv_heads][128], optional RoPE tables
// [seq][64] applied to q and k, out fp32 [seq][n_head][128].
// workspace: attention_prefill_workspace(seq, n_head, kv_heads) bytes, 16-byte aligned.
hipError_t launch_attention_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                         const float* rope_cos, const float* rope_sin, float* out, int seq,
                                         int n_head, int kv_heads, int head_dim, float scale, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream);
size_t attention_prefill_workspace(int seq, int n_head, int kv_heads);

hipError_t launch_embed(const K4Mat& emb, int cols, const int* prompt, DecodeState* st, float* x,
                        hipStream_t stream);
// Embedding rows of tokens[0 .. rows) into x[rows][cols] (a prompt at once).
hipError_t launch_embed_rows(const K4Mat& emb, int cols, const int* tokens, int rows, float* x, hipStream_t stream);
// st->pos = pos and cleared argmax slots (a step whose final GEMV runs outside the decode step).
hipError_t launch_set_step(DecodeState* st, int pos, hipStream_t stream);
hipError_t launch_embed_bf16(const uint16_t* emb, int vocab, int cols, const int* prompt, DecodeState* st, float* x,
                             hipStream_t stream);
hipError_t launch_finish_step(DecodeState* st, int* out_tokens, hipStream_t stream);

// Small standalone ops behind the mantleHip* C ABI.
hipError_t launch_dequant_k4(const K4Mat& m, int cols, float* out_f32, uint16_t* out_f16, hipStream_t stream);
hipError_t launch_silu_mul(const float* gate, const float* up, float* out, int n, hipStream_t stream);
hipError_t launch_add(float* dst, const float* src, int n, hipStream_t stream);
hipError_t launch_argmax(const float* x, int n, int* out_idx, hipStream_t stream);
hipError_t launch_softmax_rows(float* data, int rows, int cols, hipStream_t stream);
hipError_t launch_rope_table(float* x, const float* cosv, const float* sinv, int head_dim, int half, int n_heads,
                             hipStream_t stream);
hipError_t launch_rope_f64(float* x, const double* inv_freq, int pos, float attn_scale, int head_dim, int half,
                           int n_heads, hipStream_t stream);
hipError_t launch_rope_f32(float* x, const float* inv_freq, int pos, float attn_scale, int head_dim, int half,
                           int n_heads, hipStream_t stream);
hipError_t launch_store_kv_row(float* cache, const float* src, int cache_pos, int kv_stride, hipStream_t stream);
hipError_t launch_store_kv_row_f16(uint16_t* cache, const float* src, int cache_pos, int kv_stride,
                                   hipStream_t stream);
// KV cache element type of models loaded from now on (0 f32, 1 f16).
// The q8_0 KV append (ops_runtime.go:112-157 StoreKV / storeQ8): one int8
// row of kv_heads*head_dim values per position for K and for V, each with one
// scale (max |x| / 127 over the whole row).  prep: K is first given the
// per-head RMSNorm (k_norm, when not null) and RoPE (rope_cos / rope_sin at
// the position, when not null) of the fused attention step.
struct KvQ8Args {
    const float *k, *v;
    const float* k_norm;
    const float *rope_cos, *rope_sin;  // [max_ctx][head_dim/2]
    const int* pos_dev;                // device position, or pos_host when null
    int pos_host;
    float eps;
    int isa;
    int kv_heads, head_dim;
    int8_t *cache_k, *cache_v;  // element (t, d) of kv head g: g*head_stride + t*row_stride + d
    int head_stride, row_stride;
    int vt_stride;  // > 0: V transposed, (g*head_dim + d)*vt_stride + t
    float *k_scale, *v_scale;  // [max_ctx]
    int prep;
    int skip_k, skip_v;  // 1: that row is not a q8_0 cache (mixed cache types): left alone
    int tokens, tok_stride;  // > 1: rows pos .. pos+tokens-1, their k / v tok_stride floats apart
};
static constexpr int kKvQ8MaxRow = 4096;  // kv_heads*head_dim: both rows staged in LDS
hipError_t launch_kv_append_q8(const KvQ8Args& a, hipStream_t stream);
// KV cache element types (kv_cache_type): Mantle's CacheTypeF32 / F16 / Q8_0.
enum KvCacheType : int { kKvF32 = 0, kKvF16 = 1, kKvQ8 = 2 };
int kv_cache_type();
bool set_kv_cache_type(int t);

}  // namespace mantle
