// capi.cpp -- the extern "C" entry points of libmantle_hip.so (declared in
// include/mantle_hip.h).  Each validates on the host and forwards to a launcher.
#include <hip/hip_runtime.h>
#include <string.h>

#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mantle_hip.h"
#include "kernels.h"
#include "mcf.h"

using namespace mantle;

static std::atomic<int> g_isa{kIsaAvx512};

static inline hipStream_t S(mantleHipStream_t s) { return reinterpret_cast<hipStream_t>(s); }

static K4Mat mat(const uint8_t* q, const uint16_t* sup, const uint8_t* sub, int rows) {
    K4Mat m;
    m.nib = q;
    m.sup = sup;
    m.sub = sub;
    m.rows = rows;
    return m;
}

static bool k4_dims_ok(const void* q, const void* sup, const void* sub, int rows, int bpr, int cols) {
    return q && sup && sub && rows > 0 && cols > 0 && bpr == (cols + 31) / 32;
}

extern "C" {

const char* mantleHipGetErrorString(int err) { return hipGetErrorString((hipError_t)err); }

int mantleHipGetDeviceCount(int* out) {
    if (!out) return hipErrorInvalidValue;
    return hipGetDeviceCount(out);
}

int mantleHipSetParityISA(int isa) {
    if (isa != kIsaScalar && isa != kIsaAvx2 && isa != kIsaAvx512) return hipErrorInvalidValue;
    g_isa.store(isa);
    return hipSuccess;
}

int mantleHipGetParityISA(void) { return g_isa.load(); }

int mantleHipSetAttentionPath(int path) { return set_attention_path(path) ? hipSuccess : hipErrorInvalidValue; }

int mantleHipGetAttentionPath(void) { return attention_path(); }

int mantleHipMatVecBF16F32(const uint16_t* w, const float* x, float* y, int rows, int cols, mantleHipStream_t stream) {
    if (!w || !x || !y || rows <= 0 || cols <= 0) return hipErrorInvalidValue;
    const int r[1] = {rows};
    float* o[1] = {y};
    return launch_bf16_gemv(&w, o, r, 1, cols, x, kEpiStore, nullptr, g_isa.load(), S(stream));
}

int mantleHipQuantMatVecK4F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                              const float* x, float* y, int rows, int blocksPerRow, int cols,
                              mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !x || !y)
        return hipErrorInvalidValue;
    return launch_k4_gemv_w4a32(mat(qData, superScalesF16, subScales, rows), cols, x, y, 1, S(stream));
}

int mantleHipQuantMatVecK4F32Batched(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                     const float* x, float* y, int rows, int blocksPerRow, int cols, int batch,
                                     mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !x || !y || batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    return launch_k4_gemv_w4a32(mat(qData, superScalesF16, subScales, rows), cols, x, y, batch, S(stream));
}

int mantleHipQuantMatVecK4W4A8F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                  const float* x, float* y, int rows, int blocksPerRow, int cols, int batch,
                                  int8_t* qxScratch, float* xScaleScratch, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !x || !y || !qxScratch ||
        !xScaleScratch || batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    hipError_t e = launch_quantize_vec(x, nullptr, 0.0f, cols, batch, g_isa.load(), qxScratch, xScaleScratch, nullptr,
                                       S(stream));
    if (e != hipSuccess) return e;
    K4Mat m = mat(qData, superScalesF16, subScales, rows);
    float* outs[1] = {y};
    return launch_k4_gemv_w4a8(&m, outs, 1, cols, qxScratch, xScaleScratch, batch, kEpiStore, nullptr, S(stream));
}

int mantleHipQuantMatMulK4W4A8F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                  const float* x, float* y, int rows, int blocksPerRow, int cols, int n,
                                  int8_t* qxScratch, float* xScaleScratch, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !x || !y || !qxScratch ||
        !xScaleScratch || n < 1 || blocksPerRow % 8)
        return hipErrorInvalidValue;
    hipError_t e = launch_quantize_vec(x, nullptr, 0.0f, cols, n, g_isa.load(), qxScratch, xScaleScratch, nullptr,
                                       S(stream));
    if (e != hipSuccess) return e;
    return launch_k4_gemm_w4a8(mat(qData, superScalesF16, subScales, rows), cols, qxScratch, xScaleScratch, n, y,
                               rows, kEpiStore, S(stream));
}

int mantleHipQuantMatVecK4W4A8F32NoAlloc(const uint8_t* qData, const uint16_t* superScalesF16,
                                         const uint8_t* subScales, const float* x, float* y, int rows,
                                         int blocksPerRow, int cols, int batch, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !x || !y) return hipErrorInvalidValue;
    return launch_k4_gemv_w4a8_noalloc(mat(qData, superScalesF16, subScales, rows), cols, x, y, batch, g_isa.load(),
                                       S(stream));
}

int mantleHipQuantMatVecK4W4A8QF32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                   const int8_t* qx, const float* xScales, float* y, int rows, int blocksPerRow,
                                   int cols, int batch, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !qx || !xScales || !y ||
        batch < 1 || batch > 8)
        return hipErrorInvalidValue;
    K4Mat m = mat(qData, superScalesF16, subScales, rows);
    float* outs[1] = {y};
    return launch_k4_gemv_w4a8(&m, outs, 1, cols, qx, xScales, batch, kEpiStore, nullptr, S(stream));
}

int mantleHipDequantizeK4ToF16(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                               uint16_t* outF16, int rows, int blocksPerRow, int cols, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !outF16) return hipErrorInvalidValue;
    return launch_dequant_k4(mat(qData, superScalesF16, subScales, rows), cols, nullptr, outF16, S(stream));
}

int mantleHipDequantizeK4ToF32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                               float* out, int rows, int blocksPerRow, int cols, mantleHipStream_t stream) {
    if (!k4_dims_ok(qData, superScalesF16, subScales, rows, blocksPerRow, cols) || !out) return hipErrorInvalidValue;
    return launch_dequant_k4(mat(qData, superScalesF16, subScales, rows), cols, out, nullptr, S(stream));
}

int mantleHipQuantizeVecBlocksF32(const float* x, int n, int8_t* qx, float* scales, mantleHipStream_t stream) {
    return launch_quantize_vec(x, nullptr, 0.0f, n, 1, g_isa.load(), qx, scales, nullptr, S(stream));
}

int mantleHipRMSNormF32(float* out, const float* x, const float* weight, float eps, int n, mantleHipStream_t stream) {
    return launch_rmsnorm(out, x, weight, eps, n, 1, g_isa.load(), S(stream));
}

int mantleHipRMSNormBatchedF32(float* out, const float* x, const float* weight, float eps, int headDim, int nHeads,
                               mantleHipStream_t stream) {
    return launch_rmsnorm(out, x, weight, eps, headDim, nHeads, g_isa.load(), S(stream));
}

int mantleHipApplyRoPEInplaceF32(float* x, const float* invFreq, int pos, float attnScale, int headDim, int half,
                                 int nHeads, mantleHipStream_t stream) {
    return launch_rope_f32(x, invFreq, pos, attnScale, headDim, half, nHeads, S(stream));
}

int mantleHipApplyRoPEInplaceF64FreqF32(float* x, const double* invFreq, int pos, float attnScale, int headDim,
                                        int half, int nHeads, mantleHipStream_t stream) {
    return launch_rope_f64(x, invFreq, pos, attnScale, headDim, half, nHeads, S(stream));
}

int mantleHipApplyRoPEInplaceTableF32(float* x, const float* cosv, const float* sinv, int headDim, int half,
                                      int nHeads, mantleHipStream_t stream) {
    return launch_rope_table(x, cosv, sinv, headDim, half, nHeads, S(stream));
}

int mantleHipStoreKVF32Row(float* cache, const float* src, int cachePos, int kvStride, mantleHipStream_t stream) {
    return launch_store_kv_row(cache, src, cachePos, kvStride, S(stream));
}

// RunAttnHeads over row-major caches ([cachePos][kvStride]) of any K / V
// types: keys start..pos, key t at row t % cacheLen when 0 < cacheLen < pos + 1
// (attnpool.go:77-153).  scores: nHead * (pos - start + 1) floats.
static int attention_rows(const float* q, const void* cacheK, const void* cacheV, int kt, int vt, const float* kScales,
                          const float* vScales, float* out, float* scores, int pos, int start, int kvStride,
                          int headDim, int nHead, int kvHeads, int cacheLen, float scale, hipStream_t stream) {
    if (pos < 0 || start < 0 || start > pos || kvHeads <= 0 || nHead % kvHeads || cacheLen < 0)
        return hipErrorInvalidValue;
    const bool ring = cacheLen > 0 && cacheLen < pos + 1;
    AttnArgs a{};
    a.q = q;
    a.cache_k = reinterpret_cast<float*>(const_cast<void*>(cacheK));  // element type k_type
    a.cache_v = reinterpret_cast<float*>(const_cast<void*>(cacheV));  // element type v_type
    a.k_type = kt;
    a.v_type = vt;
    a.k_scale = kScales;
    a.v_scale = vScales;
    a.scores = scores;
    a.out = out;
    a.pos_host = pos - start;  // the window's last key
    a.key_base = start;
    a.key_ring = ring ? cacheLen : 0;
    a.n_head = nHead;
    a.kv_heads = kvHeads;
    a.head_dim = headDim;
    a.kv_stride = kvStride;
    a.head_stride = headDim;  // Mantle's cache: row = cachePos * kvStride + kvHead * headDim
    a.max_ctx = pos - start + 1;
    a.scale = scale;
    a.fused = 0;
    a.isa = g_isa.load();
    return launch_attention_decode(a, stream);
}

// The library's per-device scores buffer for the entry points that take no
// scratch argument (the reference signatures): grown on demand, shared by
// every such call on the device, so such calls must be serialised on one
// stream per device.
static float* library_scores(size_t floats) {
    static std::mutex mu;
    static float* buf[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] < floats) {
        if (buf[dev]) {
            // earlier launches may still read it
            if (hipDeviceSynchronize() != hipSuccess) return nullptr;
            (void)hipFree(buf[dev]);
            buf[dev] = nullptr;
            cap[dev] = 0;
        }
        size_t n = floats < 65536 ? 65536 : floats;
        if (hipMalloc((void**)&buf[dev], sizeof(float) * n) != hipSuccess) return nullptr;
        cap[dev] = n;
    }
    return buf[dev];
}

int mantleHipAttentionInnerF32Cache(const float* q, const float* cacheK, const float* cacheV, float* out,
                                    float* scoresScratch, int pos, int start, int kvStride, int headDim, int nHead,
                                    int kvHeads, int cacheLen, float scale, mantleHipStream_t stream) {
    return attention_rows(q, cacheK, cacheV, kKvF32, kKvF32, nullptr, nullptr, out, scoresScratch, pos, start,
                          kvStride, headDim, nHead, kvHeads, cacheLen, scale, S(stream));
}

int mantleHipAttentionInnerF16CacheF32(const float* q, const uint16_t* cacheK, const uint16_t* cacheV, float* out,
                                       int pos, int start, int kvStride, int headDim, int nHead, int kvHeads,
                                       int cacheLen, float scale, mantleHipStream_t stream) {
    if (pos < 0 || start < 0 || start > pos || nHead <= 0) return hipErrorInvalidValue;
    float* scores = library_scores((size_t)nHead * (size_t)(pos - start + 1));
    if (!scores) return hipErrorOutOfMemory;
    return attention_rows(q, cacheK, cacheV, kKvF16, kKvF16, nullptr, nullptr, out, scores, pos, start, kvStride,
                          headDim, nHead, kvHeads, cacheLen, scale, S(stream));
}

int mantleHipAttentionInnerMixedCacheF32(const float* q, const uint16_t* cacheKF16, const uint16_t* cacheVF16,
                                         const int8_t* cacheKQ8, const int8_t* cacheVQ8, const float* cacheKScales,
                                         const float* cacheVScales, float* out, int useQ8K, int useQ8V, int pos,
                                         int start, int kvStride, int headDim, int nHead, int kvHeads, int cacheLen,
                                         float scale, mantleHipStream_t stream) {
    if (pos < 0 || start < 0 || start > pos || nHead <= 0) return hipErrorInvalidValue;
    const void* ck = useQ8K ? static_cast<const void*>(cacheKQ8) : static_cast<const void*>(cacheKF16);
    const void* cv = useQ8V ? static_cast<const void*>(cacheVQ8) : static_cast<const void*>(cacheVF16);
    if ((useQ8K && !cacheKScales) || (useQ8V && !cacheVScales)) return hipErrorInvalidValue;
    float* scores = library_scores((size_t)nHead * (size_t)(pos - start + 1));
    if (!scores) return hipErrorOutOfMemory;
    return attention_rows(q, ck, cv, useQ8K ? kKvQ8 : kKvF16, useQ8V ? kKvQ8 : kKvF16, cacheKScales, cacheVScales,
                          out, scores, pos, start, kvStride, headDim, nHead, kvHeads, cacheLen, scale, S(stream));
}

int mantleHipStoreKVF16Row(uint16_t* cache, const float* src, int cachePos, int kvStride, mantleHipStream_t stream) {
    return launch_store_kv_row_f16(cache, src, cachePos, kvStride, S(stream));
}

int mantleHipAttentionInnerQ8CacheF32(const float* q, const int8_t* cacheK, const int8_t* cacheV,
                                      const float* kScales, const float* vScales, float* out, float* scoresScratch,
                                      int pos, int start, int kvStride, int headDim, int nHead, int kvHeads,
                                      int cacheLen, float scale, mantleHipStream_t stream) {
    if (!kScales || !vScales) return hipErrorInvalidValue;
    return attention_rows(q, cacheK, cacheV, kKvQ8, kKvQ8, kScales, vScales, out, scoresScratch, pos, start, kvStride,
                          headDim, nHead, kvHeads, cacheLen, scale, S(stream));
}

int mantleHipStoreKVQ8Row(int8_t* cacheK, int8_t* cacheV, float* kScales, float* vScales, const float* k,
                          const float* v, int cachePos, int kvStride, mantleHipStream_t stream) {
    if (cachePos < 0 || kvStride <= 0) return hipErrorInvalidValue;
    KvQ8Args a{};
    a.k = k;
    a.v = v;
    a.pos_host = cachePos;
    a.kv_heads = 1;
    a.head_dim = kvStride;
    a.cache_k = cacheK;
    a.cache_v = cacheV;
    a.head_stride = 0;
    a.row_stride = kvStride;
    a.k_scale = kScales;
    a.v_scale = vScales;
    return launch_kv_append_q8(a, S(stream));
}

int mantleHipSetKVCacheType(int type) { return set_kv_cache_type(type) ? hipSuccess : hipErrorInvalidValue; }

int mantleHipGetKVCacheType(void) { return kv_cache_type(); }

int mantleHipAttentionPrefillBF16(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ropeCos,
                                  const float* ropeSin, float* out, int seqLen, int nHead, int kvHeads, int headDim,
                                  float scale, void* workspace, size_t workspaceBytes, mantleHipStream_t stream) {
    return launch_attention_prefill_bf16(q, k, v, ropeCos, ropeSin, out, seqLen, nHead, kvHeads, headDim, scale,
                                         workspace, workspaceBytes, S(stream));
}

int mantleHipAttentionPrefillWorkspaceSize(int seqLen, int nHead, int kvHeads, int headDim, size_t* bytes) {
    if (!bytes || seqLen <= 0 || nHead <= 0 || kvHeads <= 0 || nHead % kvHeads || headDim != 128)
        return hipErrorInvalidValue;
    *bytes = attention_prefill_workspace(seqLen, nHead, kvHeads);
    return hipSuccess;
}

int mantleHipSoftmaxRowsF32(float* data, int rows, int cols, mantleHipStream_t stream) {
    return launch_softmax_rows(data, rows, cols, S(stream));
}

int mantleHipSiluMulF32(const float* gate, const float* up, float* out, int n, mantleHipStream_t stream) {
    return launch_silu_mul(gate, up, out, n, S(stream));
}

int mantleHipAddVectorsF32(float* dst, const float* src, int n, mantleHipStream_t stream) {
    return launch_add(dst, src, n, S(stream));
}

int mantleHipArgMaxF32(const float* x, int n, int* outIdx, mantleHipStream_t stream) {
    return launch_argmax(x, n, outIdx, S(stream));
}

int64_t mantleHipK4PayloadSize(int64_t rows, int64_t cols) { return k4_payload_bytes(rows, cols); }

int mantleHipQuantizeK4Host(const float* src, int64_t rows, int64_t cols, uint8_t* payload) {
    if (!src || !payload || rows <= 0 || cols <= 0) return hipErrorInvalidValue;
    return quantize_k4(src, rows, cols, payload, nullptr, nullptr, 1) == 0 ? hipSuccess : hipErrorInvalidValue;
}

int mantleHipFillNormal(float* dst, int64_t n, uint64_t seed, float std_dev) {
    if (!dst || n < 0) return hipErrorInvalidValue;
    fill_normal(dst, n, seed, std_dev, 1);
    return hipSuccess;
}

// `mantle pack` + `mantle quantize --method k4` for a random-init Qwen3-shaped model.
int mantleHipPackSyntheticQwen3(const char* path, const mantleHipQwen3Config* c, uint64_t seed, int threads) {
    if (!path || !c || c->n_layers <= 0 || c->d_model <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
        c->head_dim <= 0 || c->ffn <= 0 || c->vocab <= 0)
        return hipErrorInvalidValue;
    if (threads < 1) threads = 1;
    if (c->weight_dtype != 0 && c->weight_dtype != kDTypeK4 && c->weight_dtype != kDTypeBF16) return hipErrorInvalidValue;
    McfWriter w;
    std::string err;
    if (!w.open(path, &err)) return hipErrorInvalidValue;
    char js[1024];
    snprintf(js, sizeof js,
             "{\"architectures\": [\"Qwen3ForCausalLM\"], \"model_type\": \"qwen3\", \"hidden_size\": %d, "
             "\"num_hidden_layers\": %d, \"num_attention_heads\": %d, \"num_key_value_heads\": %d, \"head_dim\": %d, "
             "\"intermediate_size\": %d, \"vocab_size\": %d, \"rope_theta\": %.17g, \"rms_norm_eps\": %.9g, "
             "\"tie_word_embeddings\": %s, \"hidden_act\": \"silu\", \"max_position_embeddings\": 40960}",
             c->d_model, c->n_layers, c->n_heads, c->n_kv_heads, c->head_dim, c->ffn, c->vocab, c->rope_base,
             (double)c->eps, c->tie_embeddings ? "true" : "false");
    if (!w.write_section(kSecHFConfigJSON, 1, js, strlen(js))) return hipErrorInvalidValue;
    struct T {
        std::string name;
        int64_t rows, cols;  // cols == 0: rank-1 norm gain (unit), stays f32
    };
    std::vector<T> ts;
    const int64_t qd = (int64_t)c->n_heads * c->head_dim, kvd = (int64_t)c->n_kv_heads * c->head_dim;
    ts.push_back({"model.embed_tokens.weight", c->vocab, c->d_model});
    if (!c->tie_embeddings) ts.push_back({"lm_head.weight", c->vocab, c->d_model});
    ts.push_back({"model.norm.weight", c->d_model, 0});
    for (int l = 0; l < c->n_layers; l++) {
        std::string p = "model.layers." + std::to_string(l) + ".";
        ts.push_back({p + "input_layernorm.weight", c->d_model, 0});
        ts.push_back({p + "post_attention_layernorm.weight", c->d_model, 0});
        ts.push_back({p + "self_attn.q_norm.weight", c->head_dim, 0});
        ts.push_back({p + "self_attn.k_norm.weight", c->head_dim, 0});
        ts.push_back({p + "self_attn.q_proj.weight", qd, c->d_model});
        ts.push_back({p + "self_attn.k_proj.weight", kvd, c->d_model});
        ts.push_back({p + "self_attn.v_proj.weight", kvd, c->d_model});
        ts.push_back({p + "self_attn.o_proj.weight", c->d_model, qd});
        ts.push_back({p + "mlp.gate_proj.weight", c->ffn, c->d_model});
        ts.push_back({p + "mlp.up_proj.weight", c->ffn, c->d_model});
        ts.push_back({p + "mlp.down_proj.weight", c->d_model, c->ffn});
    }
    // cmd/mantle/quantize.go:226 sorts names before writing payloads.
    std::sort(ts.begin(), ts.end(), [](const T& a, const T& b) { return a.name < b.name; });
    if (!w.begin_tensor_data()) return hipErrorInvalidValue;
    std::vector<float> buf;
    std::vector<uint8_t> payload;
    for (auto& t : ts) {
        if (t.cols == 0) {
            buf.assign((size_t)t.rows, 1.0f);
            if (!w.add_tensor(t.name, kDTypeF32, {(uint64_t)t.rows}, buf.data(), 4 * (uint64_t)t.rows, false, 0, 0))
                return hipErrorInvalidValue;
            continue;
        }
        buf.resize((size_t)(t.rows * t.cols));
        fill_normal(buf.data(), t.rows * t.cols, splitmix64(seed ^ fnv1a64(t.name)), 0.02f, threads);
        if (c->weight_dtype == kDTypeBF16) {  // pkg/mcf/pack.go:789-793 bf16FromF32Bits
            std::vector<uint16_t> b16(buf.size());
            for (size_t i = 0; i < buf.size(); i++) {
                uint32_t u;
                memcpy(&u, &buf[i], 4);
                b16[i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
            }
            if (!w.add_tensor(t.name, kDTypeBF16, {(uint64_t)t.rows, (uint64_t)t.cols}, b16.data(), 2 * b16.size(),
                              false, 0, 0))
                return hipErrorInvalidValue;
            continue;
        }
        payload.resize((size_t)k4_payload_bytes(t.rows, t.cols));
        float mn = 0, mx = 0;
        if (quantize_k4(buf.data(), t.rows, t.cols, payload.data(), &mn, &mx, threads) != 0) return hipErrorInvalidValue;
        if (!w.add_tensor(t.name, kDTypeK4, {(uint64_t)t.rows, (uint64_t)t.cols}, payload.data(), payload.size(), true,
                          mn, mx))
            return hipErrorInvalidValue;
    }
    if (!w.end_tensor_data()) return hipErrorInvalidValue;
    return w.finalise(1 /* FlagTensorDataAligned64 */) ? hipSuccess : hipErrorInvalidValue;
}

struct mantleHipMCF {
    McfFile f;
};

int mantleHipMCFOpen(const char* path, mantleHipMCF** out) {
    if (!path || !out) return hipErrorInvalidValue;
    auto* h = new mantleHipMCF();
    std::string err;
    if (!h->f.open(path, &err)) {
        delete h;
        *out = nullptr;
        return hipErrorInvalidValue;
    }
    *out = h;
    return hipSuccess;
}

void mantleHipMCFClose(mantleHipMCF* f) { delete f; }

int mantleHipMCFTensorCount(const mantleHipMCF* f) { return f ? (int)f->f.tensors().size() : -1; }

int mantleHipMCFTensorInfo(const mantleHipMCF* f, int i, char* nameBuf, int nameBufLen, int* dtype, int* rank,
                           int64_t* shape, const uint8_t** data, uint64_t* size) {
    if (!f || i < 0 || i >= (int)f->f.tensors().size()) return hipErrorInvalidValue;
    const McfTensor& t = f->f.tensors()[i];
    if (nameBuf && nameBufLen > 0) {
        size_t n = t.name.size() < (size_t)nameBufLen - 1 ? t.name.size() : (size_t)nameBufLen - 1;
        memcpy(nameBuf, t.name.data(), n);
        nameBuf[n] = 0;
    }
    if (dtype) *dtype = t.dtype;
    if (rank) *rank = (int)t.shape.size();
    if (shape)
        for (size_t d = 0; d < t.shape.size() && d < 4; d++) shape[d] = (int64_t)t.shape[d];
    if (data) *data = f->f.data() + t.off;
    if (size) *size = t.size;
    return hipSuccess;
}

int mantleHipMCFFind(const mantleHipMCF* f, const char* name) { return f && name ? f->f.find(name) : -1; }

int mantleHipMCFSection(const mantleHipMCF* f, uint32_t type, const uint8_t** data, uint64_t* size) {
    if (!f) return hipErrorInvalidValue;
    const McfSection* s = f->f.section(type);
    if (!s) return hipErrorInvalidValue;
    if (data) *data = f->f.data() + s->off;
    if (size) *size = s->size;
    return hipSuccess;
}

}  // extern "C"
