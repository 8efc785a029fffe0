// runtime.cpp -- Qwen3-shaped k4 decoder resident in HBM, greedy decode.
//
// Replaces, for the k4 decode path, the Go plug-in seam backend.Backend.LoadModel
// + core.Runtime (internal/backend/backend.go:17-36, internal/backend/core/interfaces.go:4-18)
// with the CUDA backend's "whole token on device" design
// (internal/backend/cuda/attn_pipeline.go:391-805, internal/backend/cuda/ops.go:2180-2519):
//
//   * every k4 payload of the MCF is copied once, unchanged, into one HBM
//     arena (256-byte aligned per tensor); the GEMV reads the MCF layout;
//   * the decode state (position, next token, prompt, argmax key) lives in
//     device memory, so one decode step is a fixed sequence of kernel
//     launches that never reads the host: it is captured once as a HIP
//     graph and replayed per position;
//   * the f32 K cache is head-major, [layer][kv_head][max_ctx][head_dim]: the
//     keys a decode step reads for one kv head are one contiguous run; the V
//     cache is transposed for the split attention kernels (see vt_stride).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include <string>
#include <vector>

#include "../../include/mantle_hip.h"
#include "kernels.h"
#include "mcf.h"

using namespace mantle;

extern "C" int mantleHipGetParityISA(void);

struct mantleHipModel {
    mantleHipQwen3Config cfg{};
    int max_ctx = 0;
    int isa = kIsaAvx512;
    int q_dim = 0, kv_dim = 0;
    hipStream_t stream = nullptr;
    uint8_t* arena = nullptr;
    size_t arena_bytes = 0;
    K4Mat embed{}, lm_head{};
    const float* final_norm = nullptr;
    // raw-bf16 weights (cfg.weight_dtype == kDTypeBF16): the b* pointers below
    // instead of the K4Mat ones
    bool bf16 = false;
    const uint16_t *bembed = nullptr, *blm_head = nullptr;
    struct Layer {
        const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
        K4Mat wq, wk, wv, wo, gate, up, down;
        const uint16_t *bq, *bk, *bv, *bo, *bgate, *bup, *bdown;
    };
    std::vector<Layer> layers;
    // activations / scratch
    float *x = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr, *scores = nullptr;
    float *xn = nullptr, *up = nullptr;  // bf16 path: normalised x, the up projection
    unsigned* attn_counters = nullptr;  // [n_heads] arrival counters of the one-launch split attention
    int8_t* qx = nullptr;
    float* xs = nullptr;
    float *cache_k = nullptr, *cache_v = nullptr;
    // V cache: head-major like K, or (vt_stride > 0, the split attention
    // kernels) transposed, [layer][kv_head][head_dim][vt_stride]: a column's
    // keys contiguous, so the V sum loads four keys per 16 bytes.
    int vt_stride = 0;
    int v_rows = 0;  // per layer and kv column: max_ctx or vt_stride
    int k_type = kKvF32, v_type = kKvF32;  // KvCacheType of the K / V caches (--cache-type-k / -v):
                                           // f32, Mantle's truncating f16, or q8_0 int8 rows with
                                           // one scale per position
    float *k_scale = nullptr, *v_scale = nullptr;  // q8_0: [layer][max_ctx]
    float *rope_cos = nullptr, *rope_sin = nullptr;
    DecodeState* state = nullptr;
    int* prompt = nullptr;
    int* out_tokens = nullptr;
    int pos = 0;  // host mirror of state->pos
    bool use_graph = true;
    bool split = false;  // split attention kernels (transposed V cache)
    int load_ctx = 0;    // maxContext given at load (SetEffectiveContextLength(0) restores it)
    hipGraphExec_t graph = nullptr;
    // Batched prompt rows (prefill_rows): buffers for up to pf_cap rows, made on first use
    struct Prefill {
        int cap = 0;
        float *x = nullptr, *qkv = nullptr, *q = nullptr, *att = nullptr, *gate = nullptr, *up = nullptr;
        float *scores = nullptr, *xs = nullptr, *atts = nullptr;
        int8_t *qx = nullptr, *attq = nullptr;
    } pf;
};

// Layer l's base in a KV cache of `rows` keys per kv column (f32, f16 or int8 elements).
static size_t kv_elem_bytes(int type) { return type == kKvQ8 ? 1 : (type == kKvF16 ? 2 : 4); }
static float* layer_cache(const mantleHipModel* m, float* base, int l, int rows, int type) {
    const size_t elems = (size_t)l * rows * m->kv_dim;
    const size_t elem = kv_elem_bytes(type);
    return reinterpret_cast<float*>(reinterpret_cast<char*>(base) + elems * elem);
}

// The layer's KV cache in the attention arguments; a q8_0 cache first gets the
// step's prepared K / V rows from launch_kv_append_q8 (the attention launch
// then prepares q only and reads the step's rows from the cache).
static hipError_t attention_cache(const mantleHipModel* m, int l, AttnArgs& a, hipStream_t s) {
    const mantleHipQwen3Config& c = m->cfg;
    a.cache_k = layer_cache(m, m->cache_k, l, m->max_ctx, m->k_type);
    a.cache_v = layer_cache(m, m->cache_v, l, m->v_rows, m->v_type);
    a.k_type = m->k_type;
    a.v_type = m->v_type;
    a.vt_stride = m->vt_stride;
    a.kv_stride = c.head_dim;                 // head-major cache:
    a.head_stride = m->max_ctx * c.head_dim;  // [layer][kv_head][max_ctx][head_dim]
    if (m->k_type != kKvQ8 && m->v_type != kKvQ8) return hipSuccess;
    if (m->k_type == kKvQ8) a.k_scale = m->k_scale + (size_t)l * m->max_ctx;
    if (m->v_type == kKvQ8) a.v_scale = m->v_scale + (size_t)l * m->max_ctx;
    KvQ8Args q{};
    q.k = a.k;
    q.v = a.v;
    q.k_norm = a.k_norm;
    q.rope_cos = a.rope_cos;
    q.rope_sin = a.rope_sin;
    q.pos_dev = a.pos_dev;
    q.eps = a.eps;
    q.isa = a.isa;
    q.kv_heads = c.n_kv_heads;
    q.head_dim = c.head_dim;
    q.cache_k = reinterpret_cast<int8_t*>(a.cache_k);
    q.cache_v = reinterpret_cast<int8_t*>(a.cache_v);
    q.head_stride = a.head_stride;
    q.row_stride = a.kv_stride;
    q.vt_stride = a.vt_stride;
    q.k_scale = const_cast<float*>(a.k_scale);
    q.v_scale = const_cast<float*>(a.v_scale);
    q.prep = 1;
    q.skip_k = m->k_type != kKvQ8;
    q.skip_v = m->v_type != kKvQ8;
    return launch_kv_append_q8(q, s);
}

// One decode step with raw-bf16 weights: Mantle's same layer loop
// (runtime_decode.go:81-203) with every GEMV the plain bf16 one on fp32 x
// (matvec.go:154-172 quantises activations only for quantised weights).
static hipError_t enqueue_step_bf16(mantleHipModel* m, hipStream_t s) {
    const mantleHipQwen3Config& c = m->cfg;
    hipError_t e;
#define TRY(x)                         \
    do {                               \
        if ((e = (x)) != hipSuccess) { \
            return e;                  \
        }                              \
    } while (0)
    const int d = c.d_model;
    TRY(launch_embed_bf16(m->bembed, c.vocab, d, m->prompt, m->state, m->x, s));
    float* q = m->qkv;
    float* k = q + m->q_dim;
    float* v = k + m->kv_dim;
    for (int l = 0; l < c.n_layers; l++) {
        const auto& L = m->layers[l];
        TRY(launch_rmsnorm(m->xn, m->x, L.attn_norm, c.eps, d, 1, m->isa, s));
        const uint16_t* wqkv[3] = {L.bq, L.bk, L.bv};
        float* oqkv[3] = {q, k, v};
        const int rqkv[3] = {m->q_dim, m->kv_dim, m->kv_dim};
        TRY(launch_bf16_gemv(wqkv, oqkv, rqkv, 3, d, m->xn, kEpiStore, nullptr, m->isa, s));
        AttnArgs a{};
        a.q = q;
        a.k = k;
        a.v = v;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        a.eps = c.eps;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.pos_dev = &m->state->pos;
        a.scores = m->scores;
        a.out = m->attn;
        a.n_head = c.n_heads;
        a.kv_heads = c.n_kv_heads;
        a.head_dim = c.head_dim;
        a.max_ctx = m->max_ctx;
        a.scale = (float)(1.0 / sqrt((double)c.head_dim));
        a.fused = 1;
        a.isa = m->isa;
        a.counters = m->attn_counters;
        TRY(attention_cache(m, l, a, s));
        TRY(launch_attention_decode(a, s));
        const int rd[1] = {d};
        float* xo[1] = {m->x};
        TRY(launch_bf16_gemv(&L.bo, xo, rd, 1, m->q_dim, m->attn, kEpiResAdd, nullptr, m->isa, s));
        TRY(launch_rmsnorm(m->xn, m->x, L.ffn_norm, c.eps, d, 1, m->isa, s));
        const uint16_t* wgu[2] = {L.bgate, L.bup};
        float* ogu[2] = {m->act, m->up};
        const int rgu[2] = {c.ffn, c.ffn};
        TRY(launch_bf16_gemv(wgu, ogu, rgu, 2, d, m->xn, kEpiStore, nullptr, m->isa, s));
        TRY(launch_silu_mul(m->act, m->up, m->act, c.ffn, s));  // ffn.go:66-86 act = silu(gate) * up
        TRY(launch_bf16_gemv(&L.bdown, xo, rd, 1, c.ffn, m->act, kEpiResAdd, nullptr, m->isa, s));
    }
    TRY(launch_rmsnorm(m->xn, m->x, m->final_norm, c.eps, d, 1, m->isa, s));
    float* lo[1] = {m->logits};
    const int rv[1] = {c.vocab};
    TRY(launch_bf16_gemv(&m->blm_head, lo, rv, 1, d, m->xn, kEpiArgmax, m->state->argmax_keys, m->isa, s));
    TRY(launch_finish_step(m->state, m->out_tokens, s));
#undef TRY
    return hipSuccess;
}

static hipError_t enqueue_step(mantleHipModel* m, hipStream_t s) {
    if (m->bf16) return enqueue_step_bf16(m, s);
    const mantleHipQwen3Config& c = m->cfg;
    hipError_t e;
#define TRY(x)                         \
    do {                               \
        if ((e = (x)) != hipSuccess) { \
            return e;                  \
        }                              \
    } while (0)
    const int d = c.d_model;
    float* q = m->qkv;
    float* k = m->qkv + m->q_dim;
    float* v = k + m->kv_dim;
    const bool qattn = (c.head_dim & 31) == 0;  // whole int8 blocks per head
    float* xo[1] = {m->x};
    // The layer's four GEMVs.  runtime_decode.go:107 RMSNorm + attn.go:180-205
    // one int8 activation for Q, K, V.
    auto gemv_qkv = [&](int l) {
        const auto& L = m->layers[l];
        K4Mat qkv[3] = {L.wq, L.wk, L.wv};
        float* outs[3] = {q, k, v};
        return launch_k4_gemv_w4a8_fused(qkv, outs, 3, d, m->x, L.attn_norm, c.eps, m->isa, 1, kEpiStore, nullptr, s);
    };
    // attn.go:417 Wo on the re-quantised attention output (quantised by the
    // attention kernel), residual folded in
    auto gemv_wo = [&](int l) {
        const auto& L = m->layers[l];
        if (qattn) return launch_k4_gemv_w4a8(&L.wo, xo, 1, m->q_dim, m->qx, m->xs, 1, kEpiResAdd, nullptr, s);
        return launch_k4_gemv_w4a8_fused(&L.wo, xo, 1, m->q_dim, m->attn, nullptr, 0.0f, m->isa, 1, kEpiResAdd,
                                         nullptr, s);
    };
    // ffn.go:18-91: RMSNorm, up/gate on one int8 activation, SiLU*up (also
    // quantised for down), down + residual
    auto gemv_gu = [&](int l) {
        const auto& L = m->layers[l];
        K4Mat gu[2] = {L.gate, L.up};
        float* ao[2] = {m->act, m->act};
        return launch_k4_gemv_w4a8_fused(gu, ao, 2, d, m->x, L.ffn_norm, c.eps, m->isa, 1, kEpiSiluMul, nullptr, s,
                                         m->qx, m->xs);
    };
    auto gemv_down = [&](int l) {
        return launch_k4_gemv_w4a8(&m->layers[l].down, xo, 1, c.ffn, m->qx, m->xs, 1, kEpiResAdd, nullptr, s);
    };
    const int nl = c.n_layers;
    TRY(launch_embed(m->embed, d, m->prompt, m->state, m->x, s));
    for (int l = 0; l < nl; l++) {
        const auto& L = m->layers[l];
        TRY(gemv_qkv(l));
        AttnArgs a{};
        a.q = q;
        a.k = k;
        a.v = v;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        a.eps = c.eps;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.pos_dev = &m->state->pos;
        a.scores = m->scores;
        a.out = m->attn;
        a.n_head = c.n_heads;
        a.kv_heads = c.n_kv_heads;
        a.head_dim = c.head_dim;
        a.max_ctx = m->max_ctx;
        a.scale = (float)(1.0 / sqrt((double)c.head_dim));  // attn.go:311-314
        a.fused = 1;
        a.isa = m->isa;
        a.q_out = qattn ? m->qx : nullptr;
        a.q_scale = qattn ? m->xs : nullptr;
        a.counters = m->attn_counters;
        TRY(attention_cache(m, l, a, s));
        TRY(launch_attention_decode(a, s));
        TRY(gemv_wo(l));
        TRY(gemv_gu(l));
        TRY(gemv_down(l));
    }
    // runtime_greedy.go:53-67: final RMSNorm, lm_head, argmax (first max wins)
    float* lo[1] = {m->logits};
    TRY(launch_k4_gemv_w4a8_fused(&m->lm_head, lo, 1, d, m->x, m->final_norm, c.eps, m->isa, 1, kEpiArgmax,
                                  m->state->argmax_keys, s));
    TRY(launch_finish_step(m->state, m->out_tokens, s));
#undef TRY
    return hipSuccess;
}

static hipError_t run_steps(mantleHipModel* m, int steps) {
    if (steps <= 0) return hipSuccess;
    if (m->pos + steps > m->max_ctx) return hipErrorInvalidValue;  // context length exceeded
    hipError_t e = hipSuccess;
    if (m->use_graph && !m->graph) {
        hipGraph_t g = nullptr;
        e = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return e;
        hipError_t le = enqueue_step(m, m->stream);
        e = hipStreamEndCapture(m->stream, &g);
        if (le != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return le;
        }
        if (e != hipSuccess) return e;
        e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            m->graph = nullptr;
            return e;
        }
    }
    for (int i = 0; i < steps; i++) {
        e = m->use_graph ? hipGraphLaunch(m->graph, m->stream) : enqueue_step(m, m->stream);
        if (e != hipSuccess) return e;
        m->pos++;
    }
    return hipSuccess;
}

// Minimal reader for the numeric keys of an HF config.json.
static bool json_number(const std::string& js, const char* key, double* out) {
    std::string k = std::string("\"") + key + "\"";
    size_t p = js.find(k);
    if (p == std::string::npos) return false;
    p = js.find(':', p + k.size());
    if (p == std::string::npos) return false;
    p++;
    while (p < js.size() && (js[p] == ' ' || js[p] == '\t' || js[p] == '\n' || js[p] == '\r')) p++;
    if (js.compare(p, 4, "true") == 0) { *out = 1; return true; }
    if (js.compare(p, 5, "false") == 0) { *out = 0; return true; }
    char* end = nullptr;
    double v = strtod(js.c_str() + p, &end);
    if (end == js.c_str() + p) return false;
    *out = v;
    return true;
}

static void free_prefill(mantleHipModel* m) {
    auto& p = m->pf;
    void* bufs[] = {p.x, p.qkv, p.q, p.att, p.gate, p.up, p.scores, p.xs, p.atts, p.qx, p.attq};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    p = mantleHipModel::Prefill{};
}

static void free_model(mantleHipModel* m) {
    if (!m) return;
    free_prefill(m);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    void* bufs[] = {m->arena, m->x, m->qkv, m->attn, m->act, m->logits, m->scores, m->attn_counters, m->xn, m->up, m->qx, m->xs, m->cache_k,
                    m->cache_v, m->k_scale, m->v_scale, m->rope_cos, m->rope_sin, m->state, m->prompt, m->out_tokens};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

extern "C" void mantleHipModelClose(mantleHipModel* m) {
    if (m && m->stream) (void)hipStreamSynchronize(m->stream);
    free_model(m);
}

// Everything sized by the context length: scores, KV caches (+ q8_0
// scales), prompt / output tokens and the RoPE tables
// (internal/backend/simd/loader.go:1604-1612, ops_avx512.go:146-160: cos / sin
// of pos * invFreq in f64 on the host).  Frees what was there first.
static void free_context(mantleHipModel* m) {
    void* bufs[] = {m->scores, m->cache_k, m->cache_v, m->k_scale, m->v_scale, m->prompt, m->out_tokens, m->rope_cos, m->rope_sin};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    m->scores = nullptr;
    m->cache_k = m->cache_v = m->k_scale = m->v_scale = m->rope_cos = m->rope_sin = nullptr;
    m->prompt = m->out_tokens = nullptr;
}

static hipError_t rope_tables(mantleHipModel* m) {
    const mantleHipQwen3Config& c = m->cfg;
    const int half = c.head_dim / 2, ctx = m->max_ctx;
    std::vector<float> cs_tab((size_t)ctx * half), sn_tab((size_t)ctx * half);
    std::vector<double> inv(half);
    for (int i = 0; i < half; i++)
        inv[i] = 1.0 / pow(c.rope_base > 0 ? c.rope_base : 10000.0, (double)(2 * i) / (double)c.head_dim);
    for (int p = 0; p < ctx; p++)
        for (int i = 0; i < half; i++) {
            double ang = (double)p * inv[i];
            cs_tab[(size_t)p * half + i] = (float)cos(ang);
            sn_tab[(size_t)p * half + i] = (float)sin(ang);
        }
    hipError_t e = hipMemcpy(m->rope_cos, cs_tab.data(), sizeof(float) * cs_tab.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->rope_sin, sn_tab.data(), sizeof(float) * sn_tab.size(), hipMemcpyHostToDevice);
    return e;
}

static hipError_t alloc_context(mantleHipModel* m, int ctx) {
    const mantleHipQwen3Config& c = m->cfg;
    const bool any_q8 = m->k_type == kKvQ8 || m->v_type == kKvQ8;
    if ((any_q8 || m->k_type != m->v_type) && (ctx > 32768 || (any_q8 && m->kv_dim > kKvQ8MaxRow))) {
        fprintf(stderr, "mantle_hip: q8_0 and mixed KV caches support up to 32768 positions (q8_0: %d values per row)\n",
                kKvQ8MaxRow);
        return hipErrorInvalidValue;
    }
    free_context(m);
    m->max_ctx = ctx;
    hipError_t e;
#define TRYA(x)                        \
    do {                               \
        if ((e = (x)) != hipSuccess) { \
            free_context(m);           \
            return e;                  \
        }                              \
    } while (0)
    TRYA(hipMalloc((void**)&m->scores, sizeof(float) * (size_t)c.n_heads * ctx));
    const size_t kv_elems = (size_t)c.n_layers * ctx * m->kv_dim;
    // transposed V: a column's keys padded to 16 bytes (4 fp32, 8 f16, 16 int8 keys)
    const int vt_pad = m->v_type == kKvQ8 ? 16 : 4;
    m->vt_stride = m->split ? (ctx + vt_pad - 1) / vt_pad * vt_pad : 0;
    m->v_rows = m->split ? m->vt_stride : ctx;
    const size_t v_elems = (size_t)c.n_layers * m->v_rows * m->kv_dim;
    TRYA(hipMalloc((void**)&m->cache_k, kv_elem_bytes(m->k_type) * kv_elems));
    TRYA(hipMalloc((void**)&m->cache_v, kv_elem_bytes(m->v_type) * v_elems));
    TRYA(hipMemset(m->cache_k, 0, kv_elem_bytes(m->k_type) * kv_elems));
    TRYA(hipMemset(m->cache_v, 0, kv_elem_bytes(m->v_type) * v_elems));
    if (m->k_type == kKvQ8) {
        TRYA(hipMalloc((void**)&m->k_scale, sizeof(float) * (size_t)c.n_layers * ctx));
        TRYA(hipMemset(m->k_scale, 0, sizeof(float) * (size_t)c.n_layers * ctx));
    }
    if (m->v_type == kKvQ8) {
        TRYA(hipMalloc((void**)&m->v_scale, sizeof(float) * (size_t)c.n_layers * ctx));
        TRYA(hipMemset(m->v_scale, 0, sizeof(float) * (size_t)c.n_layers * ctx));
    }
    TRYA(hipMalloc((void**)&m->prompt, sizeof(int) * ctx));
    TRYA(hipMalloc((void**)&m->out_tokens, sizeof(int) * ctx));
    TRYA(hipMemset(m->prompt, 0, sizeof(int) * ctx));
    TRYA(hipMemset(m->out_tokens, 0, sizeof(int) * ctx));
    TRYA(hipMalloc((void**)&m->rope_cos, sizeof(float) * (size_t)ctx * (c.head_dim / 2)));
    TRYA(hipMalloc((void**)&m->rope_sin, sizeof(float) * (size_t)ctx * (c.head_dim / 2)));
    TRYA(rope_tables(m));
#undef TRYA
    // the captured step holds the old buffers
    if (m->graph) {
        (void)hipGraphExecDestroy(m->graph);
        m->graph = nullptr;
    }
    return hipSuccess;
}

// What a model is built from: the HF config.json text and the named tensor
// payloads (an MCF file's, or views the caller holds, e.g. Go's
// mcfstore.File.ReadTensorRaw results).
struct SrcTensor {
    std::string name;
    uint16_t dtype;
    std::vector<uint64_t> shape;
    const uint8_t* data;
    uint64_t size;
};
struct ModelSource {
    std::string config_json;
    std::vector<SrcTensor> tensors;
    int find(const std::string& n) const {
        for (size_t i = 0; i < tensors.size(); i++)
            if (tensors[i].name == n) return (int)i;
        return -1;
    }
};

static bool source_from_mcf(const McfFile& f, ModelSource* src, const char* path) {
    const McfSection* cs = f.section(kSecHFConfigJSON);
    if (!cs) {
        fprintf(stderr, "mantle_hip: %s: missing config.json section\n", path);
        return false;
    }
    src->config_json.assign((const char*)f.data() + cs->off, cs->size);
    for (const McfTensor& t : f.tensors()) src->tensors.push_back({t.name, t.dtype, t.shape, f.data() + t.off, t.size});
    return true;
}

// LoadModelMCF (internal/backend/simd/loader.go:51-80 + internal/backend/cuda/cuda.go:39-73,
// internal/backend/cuda/ops.go:5214-5313 weight residency).
static int load_model(const ModelSource& f, int max_ctx, const mantleHipLoadOptions& o, mantleHipModel** out,
                      const char* path);

// The process-wide settings (mantleHipSetParityISA / mantleHipSetKVCacheType)
// as load options, for the entry points that take none.
static mantleHipLoadOptions default_options() {
    mantleHipLoadOptions o{};
    o.parity_isa = mantleHipGetParityISA();
    o.cache_type_k = o.cache_type_v = kv_cache_type();
    o.use_graph = 1;
    return o;
}

static bool options_valid(const mantleHipLoadOptions* o) {
    return o && o->parity_isa >= kIsaScalar && o->parity_isa <= kIsaAvx512 && o->cache_type_k >= kKvF32 &&
           o->cache_type_k <= kKvQ8 && o->cache_type_v >= kKvF32 && o->cache_type_v <= kKvQ8;
}

extern "C" int mantleHipModelLoadMCF(const char* path, int max_ctx, mantleHipModel** out) {
    return mantleHipModelLoadMCFWithOptions(path, max_ctx, nullptr, out);
}

extern "C" int mantleHipModelLoadMCFImage(const uint8_t* data, uint64_t size, int max_ctx, mantleHipModel** out) {
    return mantleHipModelLoadMCFImageWithOptions(data, size, max_ctx, nullptr, out);
}

extern "C" int mantleHipModelLoadMCFWithOptions(const char* path, int max_ctx, const mantleHipLoadOptions* opts,
                                                mantleHipModel** out) {
    if (!path || !out || max_ctx <= 0) return hipErrorInvalidValue;
    const mantleHipLoadOptions o = opts ? *opts : default_options();
    if (!options_valid(&o)) return hipErrorInvalidValue;
    *out = nullptr;
    McfFile f;
    std::string err;
    if (!f.open(path, &err)) {
        fprintf(stderr, "mantle_hip: %s: %s\n", path, err.c_str());
        return hipErrorInvalidValue;
    }
    ModelSource src;
    if (!source_from_mcf(f, &src, path)) return hipErrorInvalidValue;
    return load_model(src, max_ctx, o, out, path);
}

extern "C" int mantleHipModelLoadMCFImageWithOptions(const uint8_t* data, uint64_t size, int max_ctx,
                                                     const mantleHipLoadOptions* opts, mantleHipModel** out) {
    if (!data || !out || max_ctx <= 0) return hipErrorInvalidValue;
    const mantleHipLoadOptions o = opts ? *opts : default_options();
    if (!options_valid(&o)) return hipErrorInvalidValue;
    *out = nullptr;
    McfFile f;
    std::string err;
    if (!f.open_image(data, size, &err)) {
        fprintf(stderr, "mantle_hip: MCF image: %s\n", err.c_str());
        return hipErrorInvalidValue;
    }
    ModelSource src;
    if (!source_from_mcf(f, &src, "MCF image")) return hipErrorInvalidValue;
    return load_model(src, max_ctx, o, out, "MCF image");
}

extern "C" int mantleHipModelLoadTensors(const char* configJSON, uint64_t configSize, const mantleHipTensorView* tensors,
                                         int nTensors, int max_ctx, const mantleHipLoadOptions* opts,
                                         mantleHipModel** out) {
    if (!configJSON || !tensors || nTensors <= 0 || !out || max_ctx <= 0) return hipErrorInvalidValue;
    *out = nullptr;
    const mantleHipLoadOptions o = opts ? *opts : default_options();
    if (!options_valid(&o)) return hipErrorInvalidValue;
    ModelSource src;
    src.config_json.assign(configJSON, configSize);
    for (int i = 0; i < nTensors; i++) {
        const mantleHipTensorView& t = tensors[i];
        if (!t.name || t.rank < 1 || t.rank > 4) return hipErrorInvalidValue;
        std::vector<uint64_t> shape;
        for (int d = 0; d < t.rank; d++) {
            if (t.shape[d] <= 0) return hipErrorInvalidValue;
            shape.push_back((uint64_t)t.shape[d]);
        }
        src.tensors.push_back({t.name, (uint16_t)t.dtype, shape, t.data, t.size});
    }
    return load_model(src, max_ctx, o, out, "tensor views");
}

static int load_model(const ModelSource& f, int max_ctx, const mantleHipLoadOptions& o, mantleHipModel** out,
                      const char* path) {
    (void)path;
    const std::string& js = f.config_json;
    mantleHipModel* m = new mantleHipModel();
    mantleHipQwen3Config& c = m->cfg;
    double v;
    auto need = [&](const char* key, double* dst) {
        if (!json_number(js, key, dst)) {
            fprintf(stderr, "mantle_hip: config.json lacks %s\n", key);
            return false;
        }
        return true;
    };
    double L, D, H, KV, F, V, HD;
    if (!need("num_hidden_layers", &L) || !need("hidden_size", &D) || !need("num_attention_heads", &H) ||
        !need("intermediate_size", &F) || !need("vocab_size", &V)) {
        free_model(m);
        return hipErrorInvalidValue;
    }
    KV = json_number(js, "num_key_value_heads", &v) ? v : H;
    HD = json_number(js, "head_dim", &v) ? v : D / H;
    c.n_layers = (int)L;
    c.d_model = (int)D;
    c.n_heads = (int)H;
    c.n_kv_heads = (int)KV;
    c.head_dim = (int)HD;
    c.ffn = (int)F;
    c.vocab = (int)V;
    c.rope_base = json_number(js, "rope_theta", &v) ? v : 10000.0;
    c.eps = json_number(js, "rms_norm_eps", &v) ? (float)v : 1e-6f;
    c.tie_embeddings = f.find("lm_head.weight") < 0;
    m->max_ctx = max_ctx;
    m->load_ctx = max_ctx;
    m->isa = o.parity_isa;
    m->use_graph = o.use_graph != 0;
    m->q_dim = c.n_heads * c.head_dim;
    m->kv_dim = c.n_kv_heads * c.head_dim;
    if (c.head_dim > 256 || (c.head_dim & 1) || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads) {
        fprintf(stderr, "mantle_hip: unsupported attention shape\n");
        free_model(m);
        return hipErrorInvalidValue;
    }

    // Rank-2 weights are all k4 or all raw bf16 (the embedding's dtype decides).
    {
        const int ei = f.find("model.embed_tokens.weight");
        m->bf16 = ei >= 0 && f.tensors[ei].dtype == kDTypeBF16;
    }
    c.weight_dtype = m->bf16 ? kDTypeBF16 : kDTypeK4;
    const uint16_t wdt = m->bf16 ? (uint16_t)kDTypeBF16 : (uint16_t)kDTypeK4;
    if (m->bf16 && (c.d_model % 8 || m->q_dim % 8 || c.ffn % 8)) {
        fprintf(stderr, "mantle_hip: bf16 weights need row lengths that are multiples of 8\n");
        free_model(m);
        return hipErrorInvalidValue;
    }
    // Tensor plan: (name, expected dtype, rows, cols); qwen3Spec names (internal/model/modelspec.go:173-240).
    struct Want {
        std::string name;
        uint16_t dtype;
        int64_t rows, cols;
        size_t arena_off;
    };
    std::vector<Want> wants;
    auto lname = [](int l, const char* s) { return "model.layers." + std::to_string(l) + "." + s; };
    wants.push_back({"model.embed_tokens.weight", wdt, c.vocab, c.d_model, 0});
    if (!c.tie_embeddings) wants.push_back({"lm_head.weight", wdt, c.vocab, c.d_model, 0});
    wants.push_back({"model.norm.weight", kDTypeF32, c.d_model, 1, 0});
    for (int l = 0; l < c.n_layers; l++) {
        wants.push_back({lname(l, "input_layernorm.weight"), kDTypeF32, c.d_model, 1, 0});
        wants.push_back({lname(l, "post_attention_layernorm.weight"), kDTypeF32, c.d_model, 1, 0});
        wants.push_back({lname(l, "self_attn.q_norm.weight"), kDTypeF32, c.head_dim, 1, 0});
        wants.push_back({lname(l, "self_attn.k_norm.weight"), kDTypeF32, c.head_dim, 1, 0});
        wants.push_back({lname(l, "self_attn.q_proj.weight"), wdt, m->q_dim, c.d_model, 0});
        wants.push_back({lname(l, "self_attn.k_proj.weight"), wdt, m->kv_dim, c.d_model, 0});
        wants.push_back({lname(l, "self_attn.v_proj.weight"), wdt, m->kv_dim, c.d_model, 0});
        wants.push_back({lname(l, "self_attn.o_proj.weight"), wdt, c.d_model, m->q_dim, 0});
        wants.push_back({lname(l, "mlp.gate_proj.weight"), wdt, c.ffn, c.d_model, 0});
        wants.push_back({lname(l, "mlp.up_proj.weight"), wdt, c.ffn, c.d_model, 0});
        wants.push_back({lname(l, "mlp.down_proj.weight"), wdt, c.d_model, c.ffn, 0});
    }
    size_t total = 0;
    std::vector<int> tidx;
    for (auto& w : wants) {
        int i = f.find(w.name);
        if (i < 0) {
            fprintf(stderr, "mantle_hip: missing tensor %s\n", w.name.c_str());
            free_model(m);
            return hipErrorInvalidValue;
        }
        const SrcTensor& t = f.tensors[i];
        bool shape_ok = w.dtype != kDTypeF32
                            ? (t.shape.size() == 2 && (int64_t)t.shape[0] == w.rows && (int64_t)t.shape[1] == w.cols)
                            : (t.shape.size() == 1 && (int64_t)t.shape[0] == w.rows);
        const int64_t elems = w.dtype == kDTypeF32 ? w.rows : w.rows * w.cols;
        const uint64_t want_size = w.dtype == kDTypeK4 ? (uint64_t)k4_payload_bytes(w.rows, w.cols)
                                                       : (uint64_t)elems * (w.dtype == kDTypeF32 ? 4 : 2);
        if (shape_ok && (t.size != want_size || !t.data)) shape_ok = false;
        if (t.dtype != w.dtype || !shape_ok) {
            fprintf(stderr, "mantle_hip: tensor %s has unexpected dtype/shape\n", w.name.c_str());
            free_model(m);
            return hipErrorInvalidValue;
        }
        w.arena_off = total;
        total += (t.size + 255) & ~(size_t)255;
        tidx.push_back(i);
    }
    hipError_t e;
#define CHECK(x)                  \
    do {                          \
        if ((e = (x)) != hipSuccess) { \
            free_model(m);        \
            return e;             \
        }                         \
    } while (0)
    CHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    CHECK(hipMalloc((void**)&m->arena, total));
    m->arena_bytes = total;
    for (size_t j = 0; j < wants.size(); j++) {
        const SrcTensor& t = f.tensors[tidx[j]];
        CHECK(hipMemcpy(m->arena + wants[j].arena_off, t.data, t.size, hipMemcpyHostToDevice));
    }
    size_t wi = 0;
    auto nextk = [&](int rows, int cols) { return k4_mat_from_payload(m->arena + wants[wi++].arena_off, rows, cols); };
    auto nextf = [&]() { return reinterpret_cast<const float*>(m->arena + wants[wi++].arena_off); };
    auto nextb = [&]() { return reinterpret_cast<const uint16_t*>(m->arena + wants[wi++].arena_off); };
    if (m->bf16) {
        m->bembed = nextb();
        m->blm_head = c.tie_embeddings ? m->bembed : nextb();
    } else {
        m->embed = nextk(c.vocab, c.d_model);
        m->lm_head = c.tie_embeddings ? m->embed : nextk(c.vocab, c.d_model);
    }
    m->final_norm = nextf();
    m->layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        auto& Ly = m->layers[l];
        Ly.attn_norm = nextf();
        Ly.ffn_norm = nextf();
        Ly.q_norm = nextf();
        Ly.k_norm = nextf();
        if (m->bf16) {
            Ly.bq = nextb();
            Ly.bk = nextb();
            Ly.bv = nextb();
            Ly.bo = nextb();
            Ly.bgate = nextb();
            Ly.bup = nextb();
            Ly.bdown = nextb();
            continue;
        }
        Ly.wq = nextk(m->q_dim, c.d_model);
        Ly.wk = nextk(m->kv_dim, c.d_model);
        Ly.wv = nextk(m->kv_dim, c.d_model);
        Ly.wo = nextk(c.d_model, m->q_dim);
        Ly.gate = nextk(c.ffn, c.d_model);
        Ly.up = nextk(c.ffn, c.d_model);
        Ly.down = nextk(c.d_model, c.ffn);
    }
    int big = c.d_model > m->q_dim ? c.d_model : m->q_dim;
    big = big > c.ffn ? big : c.ffn;
    const int big_blocks = (big + 31) / 32;
    CHECK(hipMalloc((void**)&m->x, sizeof(float) * c.d_model));
    CHECK(hipMalloc((void**)&m->qkv, sizeof(float) * (m->q_dim + 2 * m->kv_dim)));
    CHECK(hipMalloc((void**)&m->attn, sizeof(float) * m->q_dim));
    CHECK(hipMalloc((void**)&m->act, sizeof(float) * c.ffn));
    if (m->bf16) {
        CHECK(hipMalloc((void**)&m->xn, sizeof(float) * c.d_model));
        CHECK(hipMalloc((void**)&m->up, sizeof(float) * c.ffn));
    }
    CHECK(hipMalloc((void**)&m->logits, sizeof(float) * c.vocab));
    CHECK(hipMalloc((void**)&m->attn_counters, sizeof(unsigned) * c.n_heads));
    CHECK(hipMemset(m->attn_counters, 0, sizeof(unsigned) * c.n_heads));
    CHECK(hipMalloc((void**)&m->qx, (size_t)big_blocks * 32));
    CHECK(hipMalloc((void**)&m->xs, sizeof(float) * big_blocks));
    const int apath = attention_path();
    const bool split = (c.head_dim == 64 || c.head_dim == 128) && (apath == kAttnPathSplit || apath == kAttnPathFused);
    m->k_type = o.cache_type_k;
    m->v_type = o.cache_type_v;
    if ((m->k_type != kKvF32 || m->v_type != kKvF32) && !split) {
        fprintf(stderr, "mantle_hip: the f16 / q8_0 KV cache needs head_dim 64/128 and a split attention path\n");
        free_model(m);
        return hipErrorInvalidValue;
    }
    m->split = split;
    CHECK(hipMalloc((void**)&m->state, sizeof(DecodeState)));
    CHECK(hipMemset(m->state, 0, sizeof(DecodeState)));
    CHECK(alloc_context(m, max_ctx));
    CHECK(hipDeviceSynchronize());
#undef CHECK
    *out = m;
    return hipSuccess;
}

extern "C" int mantleHipModelConfig(const mantleHipModel* m, mantleHipQwen3Config* out) {
    if (!m || !out) return hipErrorInvalidValue;
    *out = m->cfg;
    return hipSuccess;
}

extern "C" int mantleHipModelReset(mantleHipModel* m) {
    if (!m) return hipErrorInvalidValue;
    DecodeState st{};
    m->pos = 0;
    hipError_t e = hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, m->stream);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(m->stream);
}

extern "C" int mantleHipModelPos(const mantleHipModel* m, int* pos) {
    if (!m || !pos) return hipErrorInvalidValue;
    *pos = m->pos;
    return hipSuccess;
}

// Writes prompt[pos..pos+n) and n_prompt = pos+n into device memory.
static hipError_t upload_tokens(mantleHipModel* m, const int* toks, int n) {
    for (int i = 0; i < n; i++)
        if (toks[i] < 0 || toks[i] >= m->cfg.vocab) return hipErrorInvalidValue;  // token id out of range
    if (m->pos + n > m->max_ctx) return hipErrorInvalidValue;
    hipError_t e = hipMemcpyAsync(m->prompt + m->pos, toks, sizeof(int) * n, hipMemcpyHostToDevice, m->stream);
    if (e != hipSuccess) return e;
    static thread_local int np;
    np = m->pos + n;
    e = hipMemcpyAsync(&m->state->n_prompt, &np, sizeof(int), hipMemcpyHostToDevice, m->stream);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(m->stream);  // np is a host stack-lifetime value
}

extern "C" int mantleHipModelForwardTokenGreedy(mantleHipModel* m, int tok, int* next) {
    if (!m || !next) return hipErrorInvalidValue;
    hipError_t e = upload_tokens(m, &tok, 1);
    if (e != hipSuccess) return e;
    if ((e = run_steps(m, 1)) != hipSuccess) return e;
    if ((e = hipMemcpyAsync(next, &m->state->next_tok, sizeof(int), hipMemcpyDeviceToHost, m->stream)) != hipSuccess)
        return e;
    return hipStreamSynchronize(m->stream);
}

extern "C" int mantleHipModelForwardToken(mantleHipModel* m, int tok, float* logits) {
    if (!m || !logits) return hipErrorInvalidValue;
    hipError_t e = upload_tokens(m, &tok, 1);
    if (e != hipSuccess) return e;
    if ((e = run_steps(m, 1)) != hipSuccess) return e;
    if ((e = hipMemcpyAsync(logits, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, m->stream)) !=
        hipSuccess)
        return e;
    return hipStreamSynchronize(m->stream);
}

// Prompt rows at once: the decode step's layer loop (runtime_decode.go:81-203)
// over R consecutive positions, each projection one int8-MFMA product over all
// R rows (launch_k4_gemm_w4a8, bit-identical per row to the step's GEMV), the
// attention row r at position pos + r with the step's kernels
// (launch_attention_rows), and the final RMSNorm / lm_head / argmax for the
// last row only -- the prompt's earlier rows need no logits.  Every value the
// cache and the last row receive equals the per-token steps' (the prefill
// tests compare the two).  Requires k4 weights, the split attention kernels,
// head_dim 64 / 128 and row widths of whole 8-block chunks; other models take
// the per-token steps.
static constexpr int kPrefillRows = 1024;                      // rows per pass at most ...
static constexpr size_t kPrefillScoreBytes = (size_t)512 << 20;  // ... and their scores within 512 MiB

static int prefill_pass_rows(const mantleHipModel* m, int n) {
    const size_t per_row = sizeof(float) * (size_t)m->cfg.n_heads * m->max_ctx;
    size_t r = kPrefillScoreBytes / per_row;
    r = r < 16 ? 16 : r;
    r = r > (size_t)kPrefillRows ? (size_t)kPrefillRows : r;
    return n < (int)r ? n : (int)r;
}

static bool prefill_rows_ok(const mantleHipModel* m) {
    const mantleHipQwen3Config& c = m->cfg;
    const char* e = getenv("MANTLE_HIP_PREFILL");
    if (e && !strcmp(e, "steps")) return false;
    return !m->bf16 && m->split && (c.head_dim == 64 || c.head_dim == 128) && c.d_model % 256 == 0 &&
           m->q_dim % 256 == 0 && c.ffn % 256 == 0 && m->max_ctx <= 32768 &&
           (attention_path() == kAttnPathSplit || attention_path() == kAttnPathFused);
}

static hipError_t prefill_alloc(mantleHipModel* m, int rows) {
    if (m->pf.cap >= rows) return hipSuccess;
    free_prefill(m);
    const mantleHipQwen3Config& c = m->cfg;
    auto& p = m->pf;
    const size_t R = (size_t)rows;
    const int wide = std::max(std::max(c.d_model, m->q_dim), c.ffn);
    hipError_t e;
#define TRYP(x)                        \
    do {                               \
        if ((e = (x)) != hipSuccess) { \
            free_prefill(m);           \
            return e;                  \
        }                              \
    } while (0)
    TRYP(hipMalloc((void**)&p.x, sizeof(float) * R * c.d_model));
    TRYP(hipMalloc((void**)&p.qkv, sizeof(float) * R * (m->q_dim + 2 * m->kv_dim)));
    TRYP(hipMalloc((void**)&p.q, sizeof(float) * R * m->q_dim));
    TRYP(hipMalloc((void**)&p.att, sizeof(float) * R * m->q_dim));
    TRYP(hipMalloc((void**)&p.gate, sizeof(float) * R * c.ffn));
    TRYP(hipMalloc((void**)&p.up, sizeof(float) * R * c.ffn));
    TRYP(hipMalloc((void**)&p.scores, sizeof(float) * R * c.n_heads * m->max_ctx));
    TRYP(hipMalloc((void**)&p.qx, R * wide));
    TRYP(hipMalloc((void**)&p.xs, sizeof(float) * R * (wide / 32)));
    TRYP(hipMalloc((void**)&p.attq, R * m->q_dim));
    TRYP(hipMalloc((void**)&p.atts, sizeof(float) * R * (m->q_dim / 32)));
#undef TRYP
    p.cap = rows;
    return hipSuccess;
}

// Rows pos .. pos+R-1 (tokens already in m->prompt); leaves the state as the
// per-token steps would: state->pos = pos + R, next_tok / out_tokens[pos+R-1]
// the argmax of the last row, logits of the last row.
static hipError_t prefill_rows(mantleHipModel* m, int R, hipStream_t s) {
    const mantleHipQwen3Config& c = m->cfg;
    auto& p = m->pf;
    const int d = c.d_model, pos = m->pos;
    const int qkvw = m->q_dim + 2 * m->kv_dim;
    hipError_t e;
#define TRY(x)                         \
    do {                               \
        if ((e = (x)) != hipSuccess) { \
            return e;                  \
        }                              \
    } while (0)
    TRY(launch_embed_rows(m->embed, d, m->prompt + pos, R, p.x, s));
    for (int l = 0; l < c.n_layers; l++) {
        const auto& L = m->layers[l];
        // attention: RMSNorm + one int8 activation per row, Q / K / V
        TRY(launch_quantize_vec(p.x, L.attn_norm, c.eps, d, R, m->isa, p.qx, p.xs, nullptr, s));
        {
            const K4Mat w3[3] = {L.wq, L.wk, L.wv};
            float* y3[3] = {p.qkv, p.qkv + m->q_dim, p.qkv + m->q_dim + m->kv_dim};
            TRY(launch_k4_gemm_w4a8_multi(w3, y3, 3, d, p.qx, p.xs, R, qkvw, kEpiStore, s));
        }
        AttnArgs a{};
        a.q = p.qkv;
        a.k = p.qkv + m->q_dim;
        a.v = p.qkv + m->q_dim + m->kv_dim;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        a.eps = c.eps;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.pos_host = pos;
        a.n_head = c.n_heads;
        a.kv_heads = c.n_kv_heads;
        a.head_dim = c.head_dim;
        a.max_ctx = m->max_ctx;
        a.scale = (float)(1.0 / sqrt((double)c.head_dim));
        a.isa = m->isa;
        a.out_row = m->q_dim;
        a.cache_k = layer_cache(m, m->cache_k, l, m->max_ctx, m->k_type);
        a.cache_v = layer_cache(m, m->cache_v, l, m->v_rows, m->v_type);
        a.k_type = m->k_type;
        a.v_type = m->v_type;
        a.vt_stride = m->vt_stride;
        a.kv_stride = c.head_dim;
        a.head_stride = m->max_ctx * c.head_dim;
        if (m->k_type == kKvQ8) a.k_scale = m->k_scale + (size_t)l * m->max_ctx;
        if (m->v_type == kKvQ8) a.v_scale = m->v_scale + (size_t)l * m->max_ctx;
        TRY(launch_attention_prep_rows(a, R, qkvw, p.q, s));
        if (m->k_type == kKvQ8 || m->v_type == kKvQ8) {
            KvQ8Args q{};
            q.k = a.k;
            q.v = a.v;
            q.k_norm = a.k_norm;
            q.rope_cos = a.rope_cos;
            q.rope_sin = a.rope_sin;
            q.pos_host = pos;
            q.eps = a.eps;
            q.isa = a.isa;
            q.kv_heads = c.n_kv_heads;
            q.head_dim = c.head_dim;
            q.cache_k = reinterpret_cast<int8_t*>(a.cache_k);
            q.cache_v = reinterpret_cast<int8_t*>(a.cache_v);
            q.head_stride = a.head_stride;
            q.row_stride = a.kv_stride;
            q.vt_stride = a.vt_stride;
            q.k_scale = const_cast<float*>(a.k_scale);
            q.v_scale = const_cast<float*>(a.v_scale);
            q.prep = 1;
            q.skip_k = m->k_type != kKvQ8;
            q.skip_v = m->v_type != kKvQ8;
            q.tokens = R;
            q.tok_stride = qkvw;
            TRY(launch_kv_append_q8(q, s));
        }
        a.q = p.q;
        a.q_row = m->q_dim;
        a.scores = p.scores;
        a.scores_row = (size_t)c.n_heads * m->max_ctx;
        a.out = p.att;
        a.q_out = p.attq;  // Wo's int8 activation (head_dim is a multiple of 32)
        a.q_scale = p.atts;
        TRY(launch_attention_rows(a, R, s));
        TRY(launch_k4_gemm_w4a8(L.wo, m->q_dim, p.attq, p.atts, R, p.x, d, kEpiResAdd, s));
        // FFN: RMSNorm + int8 activation, gate / up, SiLU(gate) * up re-quantised, down
        TRY(launch_quantize_vec(p.x, L.ffn_norm, c.eps, d, R, m->isa, p.qx, p.xs, nullptr, s));
        {
            const K4Mat w2[2] = {L.gate, L.up};
            float* y2[2] = {p.gate, p.up};
            TRY(launch_k4_gemm_w4a8_multi(w2, y2, 2, d, p.qx, p.xs, R, c.ffn, kEpiStore, s));
        }
        TRY(launch_silu_mul(p.gate, p.up, p.gate, R * c.ffn, s));
        TRY(launch_quantize_vec(p.gate, nullptr, 0.0f, c.ffn, R, m->isa, p.qx, p.xs, nullptr, s));
        TRY(launch_k4_gemm_w4a8(L.down, c.ffn, p.qx, p.xs, R, p.x, d, kEpiResAdd, s));
    }
    // the last row: final RMSNorm, lm_head, argmax, as the step's end
    TRY(launch_set_step(m->state, pos + R - 1, s));
    float* lo[1] = {m->logits};
    TRY(launch_k4_gemv_w4a8_fused(&m->lm_head, lo, 1, d, p.x + (size_t)(R - 1) * d, m->final_norm, c.eps, m->isa, 1,
                                  kEpiArgmax, m->state->argmax_keys, s));
    TRY(launch_finish_step(m->state, m->out_tokens, s));
    // x holds the last row's residual stream, as after its step (mantleHipModelHidden)
    TRY(hipMemcpyAsync(m->x, p.x + (size_t)(R - 1) * d, sizeof(float) * d, hipMemcpyDeviceToDevice, s));
#undef TRY
    m->pos += R;
    return hipSuccess;
}

// All n prompt tokens (already uploaded): passes of up to kPrefillRows rows,
// or the per-token steps where the batched form does not apply.
static hipError_t run_prompt(mantleHipModel* m, int n) {
    if (n <= 1 || !prefill_rows_ok(m)) return run_steps(m, n);
    if (m->pos + n > m->max_ctx) return hipErrorInvalidValue;
    hipError_t e = prefill_alloc(m, prefill_pass_rows(m, n));
    if (e != hipSuccess) return e;
    for (int done = 0; done < n;) {
        const int R = std::min(n - done, m->pf.cap);
        if ((e = prefill_rows(m, R, m->stream)) != hipSuccess) return e;
        done += R;
    }
    return hipSuccess;
}

extern "C" int mantleHipModelPrefillTokens(mantleHipModel* m, const int* toks, int n, int* next) {
    if (!m || !toks || n <= 0) return hipErrorInvalidValue;
    hipError_t e = upload_tokens(m, toks, n);
    if (e != hipSuccess) return e;
    if ((e = run_prompt(m, n)) != hipSuccess) return e;
    if (next) {
        if ((e = hipMemcpyAsync(next, &m->state->next_tok, sizeof(int), hipMemcpyDeviceToHost, m->stream)) !=
            hipSuccess)
            return e;
    }
    return hipStreamSynchronize(m->stream);
}

// prefillForwarder.PrefillTokens (internal/inference/engine.go:28-30): the
// prompt, then the logits of its last position (vocab floats, host).
extern "C" int mantleHipModelPrefillTokensLogits(mantleHipModel* m, const int* toks, int n, float* logits) {
    if (!m || !toks || n <= 0 || !logits) return hipErrorInvalidValue;
    hipError_t e = (hipError_t)mantleHipModelPrefillTokens(m, toks, n, nullptr);
    if (e != hipSuccess) return e;
    if ((e = hipMemcpyAsync(logits, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, m->stream)) !=
        hipSuccess)
        return e;
    return hipStreamSynchronize(m->stream);
}

// SetEffectiveContextLength (internal/backend/core/instance.go:325-339,
// internal/backend/cuda/cuda.go:237-250): size the KV cache and the other
// context-sized buffers for ctxLen positions (0: the maxContext given at
// load, which is also the upper bound).  Only before the first token (or
// after Reset): the caches are reallocated, not copied.
extern "C" int mantleHipModelSetEffectiveContextLength(mantleHipModel* m, int ctxLen) {
    if (!m || ctxLen < 0) return hipErrorInvalidValue;
    const int want = ctxLen == 0 || ctxLen > m->load_ctx ? m->load_ctx : ctxLen;
    if (m->pos != 0) return hipErrorInvalidValue;
    if (want == m->max_ctx) return hipSuccess;
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return e;
    return alloc_context(m, want);
}

// core.Runtime.UpdateRoPE (internal/backend/core/interfaces.go:14-18): the RoPE
// tables recomputed after the caller changed the RoPE base (ropeBase > 0;
// 0 keeps the current one).
extern "C" int mantleHipModelUpdateRoPE(mantleHipModel* m, double ropeBase) {
    if (!m || ropeBase < 0) return hipErrorInvalidValue;
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return e;
    if (ropeBase > 0) m->cfg.rope_base = ropeBase;
    return rope_tables(m);
}

extern "C" int mantleHipModelGenerateGreedy(mantleHipModel* m, const int* prompt, int n_prompt, int n_gen,
                                            int* out_tokens) {
    if (!m || !prompt || n_prompt <= 0 || n_gen <= 0 || !out_tokens) return hipErrorInvalidValue;
    const int p0 = m->pos;
    if (p0 + n_prompt + n_gen - 1 > m->max_ctx) return hipErrorInvalidValue;
    hipError_t e = upload_tokens(m, prompt, n_prompt);
    if (e != hipSuccess) return e;
    if ((e = run_prompt(m, n_prompt)) != hipSuccess) return e;
    if ((e = run_steps(m, n_gen - 1)) != hipSuccess) return e;
    e = hipMemcpyAsync(out_tokens, m->out_tokens + p0 + n_prompt - 1, sizeof(int) * n_gen, hipMemcpyDeviceToHost,
                       m->stream);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(m->stream);
}

extern "C" int mantleHipModelDecodeSteps(mantleHipModel* m, int steps) {
    if (!m || steps <= 0) return hipErrorInvalidValue;
    return run_steps(m, steps);
}

extern "C" int mantleHipModelSynchronize(mantleHipModel* m) {
    if (!m) return hipErrorInvalidValue;
    return hipStreamSynchronize(m->stream);
}

extern "C" int mantleHipModelHidden(mantleHipModel* m, float* out) {
    if (!m || !out) return hipErrorInvalidValue;
    hipError_t e = hipMemcpyAsync(out, m->x, sizeof(float) * m->cfg.d_model, hipMemcpyDeviceToHost, m->stream);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(m->stream);
}

extern "C" int mantleHipModelSetUseGraph(mantleHipModel* m, int on) {
    if (!m) return hipErrorInvalidValue;
    m->use_graph = on != 0;
    return hipSuccess;
}
