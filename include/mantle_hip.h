/*
 * mantle_hip.h -- C ABI of libmantle_hip.so, the MI355X (gfx950) backend for
 * Mantle's k4 decode path.
 *
 * Conventions (same as Mantle's CUDA C ABI, internal/backend/cuda/native/softmax.h:1-115):
 *  - every call returns a hipError_t as int (0 = success); null pointers and
 *    non-positive sizes return hipErrorInvalidValue (1) before any launch;
 *  - kernel-level calls take caller-owned device pointers, launch on the
 *    caller's stream and never allocate, free or synchronise;
 *  - the three k4 regions (f16 super-scales, u6 sub-scales, packed nibbles)
 *    are passed as separate pointers, exactly as the MCF payload stores them
 *    (pkg/mcf/quant_payload.go:86-112).
 * "Parity" kernels reproduce the arithmetic order of Mantle's CPU archsimd
 * path bit for bit; which ISA flavour (AVX-512 / AVX2 / scalar reduction
 * order) they follow is set with mantleHipSetParityISA.
 */
#ifndef MANTLE_HIP_H
#define MANTLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mantleHipStream_t; /* hipStream_t */

#define MANTLE_HIP_ISA_SCALAR 0
#define MANTLE_HIP_ISA_AVX2 1
#define MANTLE_HIP_ISA_AVX512 2

/* ---------------- library / device ---------------- */
/* Replaces mantleCudaGetErrorString / mantleCudaGetDeviceCount
 * (internal/backend/cuda/native/runtime.go:122-130). */
const char* mantleHipGetErrorString(int err);
int mantleHipGetDeviceCount(int* out);
/* Reduction order the parity kernels follow (internal/backend/simd/tensor_cpu.go:18-24). */
int mantleHipSetParityISA(int isa);
int mantleHipGetParityISA(void);
/* Decode-attention kernel variant for head_dim 64 / 128: no counterpart in
 * the reference (its CUDA backend has one attention kernel).  All variants are
 * bit-identical; the split ones spread a head over several CUs ("split", the
 * default: two launches up to 8192 keys, "fused" beyond; "fused": one launch
 * whose last workgroup per head does the softmax and V sum), "single" keeps
 * one workgroup per head, "general" is the any-head_dim kernel.
 * A loaded model's captured step keeps the variant it was captured with. */
#define MANTLE_HIP_ATTN_SPLIT 0
#define MANTLE_HIP_ATTN_SINGLE 1
#define MANTLE_HIP_ATTN_GENERAL 2
#define MANTLE_HIP_ATTN_FUSED 3
int mantleHipSetAttentionPath(int path);
int mantleHipGetAttentionPath(void);

/* ---------------- bf16 dense GEMV ---------------- */
/* y[rows] = W x with raw bf16 W [rows][cols] (16-byte aligned, cols a multiple
 * of 8, at most 32768) and fp32 x (16-byte aligned), bit-exact to Mantle's CPU
 * matVecRangeBF16 in the parity ISA's order (internal/backend/simd/matvec.go:406-979).
 * Replaces the BF16 weight branch of the CUDA backend's DeviceMatVec
 * (internal/backend/cuda/ops.go:1814-1824, cuBLAS on bf16-converted x), whose
 * arithmetic is not the CPU path's. */
int mantleHipMatVecBF16F32(const uint16_t* w, const float* x, float* y, int rows, int cols, mantleHipStream_t stream);

/* ---------------- k4 kernels ---------------- */
/* W4A32 k4 GEMV; replaces mantleCudaQuantMatVecK4F32
 * (internal/backend/cuda/native/softmax.h:32-41).  y[rows] = W x, fp32 x. */
int mantleHipQuantMatVecK4F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                              const float* x, float* y, int rows, int blocksPerRow, int cols,
                              mantleHipStream_t stream);
/* mantleHipQuantMatVecK4F32 over `batch` (1..8) fp32 vectors x[batch][cols] -> y[batch][rows],
 * the weights read once for all of them (config 2's batch-8 rows; Mantle's CPU path runs B
 * independent GEMVs).  Tolerance-checked like the single-vector form. */
int mantleHipQuantMatVecK4F32Batched(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                     const float* x, float* y, int rows, int blocksPerRow, int cols, int batch,
                                     mantleHipStream_t stream);
/* W4A8 CPU-parity k4 GEMV: the arithmetic of Mantle's AVX2+ CPU path
 * (internal/backend/simd/matvec.go:154-209, matvec_quant.go:256-296); batch
 * vectors x[batch][cols] -> y[batch][rows].  Bit-exact to the CPU path. */
int mantleHipQuantMatVecK4W4A8F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                  const float* x, float* y, int rows, int blocksPerRow, int cols, int batch,
                                  int8_t* qxScratch, float* xScaleScratch, mantleHipStream_t stream);
/* mantleHipQuantMatVecK4W4A8F32 over n activation rows at once (any n >= 1, blocksPerRow a
 * multiple of 8), on int8 matrix cores: y[v][r] bit-identical to the batch-1 call on row v.
 * No single counterpart in the reference: it replaces the per-token loop of
 * mantleCudaQuantMatVecK4F32 calls a prompt's projections make (internal/backend/cuda/native/
 * softmax.h:32-40) with one call.  Scratch: qx n*cols bytes, scales n*blocksPerRow floats. */
int mantleHipQuantMatMulK4W4A8F32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                  const float* x, float* y, int rows, int blocksPerRow, int cols, int n,
                                  int8_t* qxScratch, float* xScaleScratch, mantleHipStream_t stream);
/* mantleHipQuantMatVecK4W4A8F32 without the scratch arguments, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); no reference counterpart.  The quantised activation lives in a fixed library
 * array per device (110,592 bytes, held until the process ends): cols <= 12288 and
 * batch <= 8, larger sizes are rejected (hipErrorInvalidValue, with a message on stderr).
 * Nothing is allocated or freed.  Calls on one device share that array: calls that overlap
 * on one GPU (other streams) race. */
int mantleHipQuantMatVecK4W4A8F32NoAlloc(const uint8_t* qData, const uint16_t* superScalesF16,
                                         const uint8_t* subScales, const float* x, float* y, int rows,
                                         int blocksPerRow, int cols, int batch, mantleHipStream_t stream);
/* Same GEMV on an activation already quantised by mantleHipQuantizeVecBlocksF32
 * (MatVecWithQuant with a PrepareQuantVec result, internal/backend/simd/matvec.go:150-152,
 * internal/backend/simd/quant_vec.go:7-16): qx [batch][blocksPerRow*32] permuted, xScales [batch][blocksPerRow]. */
int mantleHipQuantMatVecK4W4A8QF32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                                   const int8_t* qx, const float* xScales, float* y, int rows, int blocksPerRow,
                                   int cols, int batch, mantleHipStream_t stream);
/* k4 -> f16 dense; replaces mantleCudaDequantizeK4ToF16 (internal/backend/cuda/native/softmax.h:50-57). */
int mantleHipDequantizeK4ToF16(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                               uint16_t* outF16, int rows, int blocksPerRow, int cols, mantleHipStream_t stream);
/* k4 -> f32 dense (exact: rowToQuant, internal/backend/core/quant_stub.go:51-85). */
int mantleHipDequantizeK4ToF32(const uint8_t* qData, const uint16_t* superScalesF16, const uint8_t* subScales,
                               float* out, int rows, int blocksPerRow, int cols, mantleHipStream_t stream);
/* Activation int8 quantiser (quantizeVecBlocksInto, internal/backend/simd/matvec_quant.go:746-797).
 * qx is written in the even/odd permuted block layout the W4A8 GEMV reads:
 * element e of block b lives at byte 32*b + 16*(e&1) + 4*(e>>3) + ((e>>1)&3). */
int mantleHipQuantizeVecBlocksF32(const float* x, int n, int8_t* qx, float* scales, mantleHipStream_t stream);

/* ---------------- fused / elementwise kernels ---------------- */
/* Replaces mantleCudaRMSNormF32 / mantleCudaRMSNormBatchedF32 (internal/backend/cuda/native/rmsnorm.cu:91-123). */
int mantleHipRMSNormF32(float* out, const float* x, const float* weight, float eps, int n, mantleHipStream_t stream);
int mantleHipRMSNormBatchedF32(float* out, const float* x, const float* weight, float eps, int headDim, int nHeads,
                               mantleHipStream_t stream);
/* Replaces mantleCudaApplyRoPEInplaceF32 with its argument list (internal/backend/cuda/native/
 * attn_fused.cu:51-75: float32 invFreq table, attnScale 0 taken as 1).  The angle
 * pos * invFreq[i] and its cos / sin are evaluated in float64 and the pairs updated as the CPU
 * path does (y0 = x0*c - x1*s, y1 = fma(x0, s, x1*c), internal/backend/simd/ops_avx512.go:146-190). */
int mantleHipApplyRoPEInplaceF32(float* x, const float* invFreq, int pos, float attnScale, int headDim, int half,
                                 int nHeads, mantleHipStream_t stream);
/* The same with Mantle's CPU float64 inverse frequencies (internal/backend/simd/loader.go:1604-1612),
 * which the CPU path's RoPE reads (no reference C counterpart). */
int mantleHipApplyRoPEInplaceF64FreqF32(float* x, const double* invFreq, int pos, float attnScale, int headDim,
                                        int half, int nHeads, mantleHipStream_t stream);
/* RoPE from precomputed float32 cos/sin rows (what the decode runtime uses). */
int mantleHipApplyRoPEInplaceTableF32(float* x, const float* cosv, const float* sinv, int headDim, int half,
                                      int nHeads, mantleHipStream_t stream);
/* f32 KV append; the f32 twin of mantleCudaStoreKVF16Row (internal/backend/cuda/native/attn_fused.cu:91-107). */
int mantleHipStoreKVF32Row(float* cache, const float* src, int cachePos, int kvStride, mantleHipStream_t stream);
/* Decode attention over row-major caches ([cachePos][kvStride], kvHead's vector at
 * + kvHead*headDim), CPU-parity with RunAttnHeads (internal/backend/simd/attnpool.go:77-153):
 * keys start..pos, key t read from row t % cacheLen when 0 < cacheLen < pos + 1 (the
 * ring; else row t).  headDim 64 / 128 on the split attention paths.
 * f32 cache: the f32 twin of mantleCudaAttentionInnerF16CacheF32 (no reference counterpart:
 * Mantle's CUDA backend keeps f16 caches); scoresScratch: nHead*(pos-start+1) floats.
 * Under the one-launch attention path (mantleHipSetAttentionPath(FUSED), or past 32768 keys)
 * the launch uses the library's per-device arrival counters: calls on one device must then
 * be serialised on one stream (overlapping launches would corrupt each other's counts). */
int mantleHipAttentionInnerF32Cache(const float* q, const float* cacheK, const float* cacheV, float* out,
                                    float* scoresScratch, int pos, int start, int kvStride, int headDim, int nHead,
                                    int kvHeads, int cacheLen, float scale, mantleHipStream_t stream);
/* Over Mantle's f16 KV cache (--cache-type-k/v f16, the CLI default: cmd/mantle/run.go:183-195).
 * Replaces mantleCudaAttentionInnerF16CacheF32 with its exact argument list
 * (internal/backend/cuda/native/softmax.h:70-83), with the CPU arithmetic of
 * internal/backend/simd/attnpool.go:103-106, :127-135 (DotF16 in the scalar order,
 * p_t * f16(v) summed in key order).  The scores live in a library-owned buffer per device
 * (grown on demand): calls on one device must be serialised on one stream. */
int mantleHipAttentionInnerF16CacheF32(const float* q, const uint16_t* cacheK, const uint16_t* cacheV, float* out,
                                       int pos, int start, int kvStride, int headDim, int nHead, int kvHeads,
                                       int cacheLen, float scale, mantleHipStream_t stream);
/* K and V caches each f16 or q8_0 (useQ8K / useQ8V; --cache-type-k / -v chosen independently).
 * Replaces mantleCudaAttentionInnerMixedCacheF32 with its exact argument list
 * (internal/backend/cuda/native/softmax.h:84-104); the CPU arithmetic of
 * attnpool.go:100-135 (DotQ8 / DotF16 scalar orders; q8_0 V terms (p_t * q) * s_t).  The
 * q8_0 side needs kvStride a multiple of 16 and 16-byte aligned rows, positions up to
 * 32768.  Scores as in mantleHipAttentionInnerF16CacheF32. */
int mantleHipAttentionInnerMixedCacheF32(const float* q, const uint16_t* cacheKF16, const uint16_t* cacheVF16,
                                         const int8_t* cacheKQ8, const int8_t* cacheVQ8, const float* cacheKScales,
                                         const float* cacheVScales, float* out, int useQ8K, int useQ8V, int pos,
                                         int start, int kvStride, int headDim, int nHead, int kvHeads, int cacheLen,
                                         float scale, mantleHipStream_t stream);
/* StoreKV into an f16 cache row; replaces mantleCudaStoreKVF16Row
 * (internal/backend/cuda/native/attn_fused.cu:91-107) but converts as the CPU
 * does (Float32ToFloat16: truncating, flush to zero, internal/backend/simd/float16.go:7-46). */
int mantleHipStoreKVF16Row(uint16_t* cache, const float* src, int cachePos, int kvStride, mantleHipStream_t stream);
/* Decode attention over Mantle's q8_0 KV cache (--cache-type-k/v q8_0, cmd/mantle/run.go:183-195;
 * a CPU-only cache type in Mantle, no CUDA counterpart), the arithmetic of
 * internal/backend/simd/attnpool.go:100-102, :122-130: score = DotQ8(q, k_t, kScales[t]) * scale
 * (ops.go:240-246, the scalar order), out_d = sum_t (p_t * v_t,d) * vScales[t] in key order.
 * Layout [pos][kvStride] int8 (kvStride a multiple of 16, 16-byte aligned rows), one scale
 * per position; scoresScratch, start and cacheLen as in mantleHipAttentionInnerF32Cache;
 * positions up to 32768.  Split attention paths only (both take the two-launch form, which
 * uses no shared counters; overlapping calls need scoresScratch of their own). */
int mantleHipAttentionInnerQ8CacheF32(const float* q, const int8_t* cacheK, const int8_t* cacheV,
                                      const float* kScales, const float* vScales, float* out, float* scoresScratch,
                                      int pos, int start, int kvStride, int headDim, int nHead, int kvHeads,
                                      int cacheLen, float scale, mantleHipStream_t stream);
/* StoreKV into a q8_0 cache (internal/backend/simd/ops_runtime.go:112-168, storeQ8): row cachePos
 * of cacheK / cacheV ([pos][kvStride] int8) and kScales / vScales[cachePos], each row quantised
 * with scale max|x|/127 over all kvStride values (kvStride <= 4096). */
int mantleHipStoreKVQ8Row(int8_t* cacheK, int8_t* cacheV, float* kScales, float* vScales, const float* k,
                          const float* v, int cachePos, int kvStride, mantleHipStream_t stream);
/* KV cache element type of models loaded afterwards by the entry points without options
 * (LoadModelOptions.CacheTypeK/V, internal/backend/core/load_options.go:7-8):
 * MANTLE_HIP_KV_F32, MANTLE_HIP_KV_F16 or MANTLE_HIP_KV_Q8_0, K and V of one type.
 * Process-wide: prefer mantleHipModelLoadMCFWithOptions, which also takes mixed types. */
#define MANTLE_HIP_KV_F32 0
#define MANTLE_HIP_KV_F16 1
#define MANTLE_HIP_KV_Q8_0 2
int mantleHipSetKVCacheType(int type);
int mantleHipGetKVCacheType(void);
/* Causal GQA attention over a whole prompt, bf16 inputs, on MFMA (head_dim 128).  Mantle
 * prefills k4 models position by position, RunAttnHeads over keys 0..t after RoPE
 * (internal/backend/simd/runtime_prefill.go:11-30, attnpool.go:77-153); its
 * FlashAttention fast path (internal/backend/simd/attn.go:33-35, flash_attn.go:17)
 * is the non-causal, one-KV-head-per-head form.  This computes every position at
 * once: q bf16 [seqLen][nHead][128], k / v bf16 [seqLen][kvHeads][128] (as the
 * cache rows), optional RoPE tables ropeCos / ropeSin [seqLen][64] (both or
 * neither) applied to q and k, out fp32 [seqLen][nHead][128].  fp16 MFMA operands
 * (the RoPE'd q / k, V, the probabilities), fp32 accumulation and softmax: within
 * max-abs 1e-3 + rel 1e-2 of the CPU path, not bit-exact.  workspace: caller-owned
 * device scratch of mantleHipAttentionPrefillWorkspaceSize bytes (the RoPE'd K
 * and transposed V in fp16, written once per call).  All pointers 16-byte aligned. */
int mantleHipAttentionPrefillBF16(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ropeCos,
                                  const float* ropeSin, float* out, int seqLen, int nHead, int kvHeads, int headDim,
                                  float scale, void* workspace, size_t workspaceBytes, mantleHipStream_t stream);
int mantleHipAttentionPrefillWorkspaceSize(int seqLen, int nHead, int kvHeads, int headDim, size_t* bytes);
/* Replaces mantleCudaSoftmaxRowsF32 (softmax.h:13), with Mantle's CPU fastExp / ordered sum. */
int mantleHipSoftmaxRowsF32(float* data, int rows, int cols, mantleHipStream_t stream);
/* Replaces mantleCudaSiluMulF32 (softmax.h:59-64), CPU fastSiluVec arithmetic. */
int mantleHipSiluMulF32(const float* gate, const float* up, float* out, int n, mantleHipStream_t stream);
/* Replaces mantleCudaAddVectorsF32 (internal/backend/cuda/native/add_vectors.cu:18-30). */
int mantleHipAddVectorsF32(float* dst, const float* src, int n, mantleHipStream_t stream);
/* Replaces mantleCudaArgMaxF32 (softmax.h:105-109): first maximum wins. */
int mantleHipArgMaxF32(const float* x, int n, int* outIdx, mantleHipStream_t stream);

/* ---------------- host-side k4 producer and MCF container ---------------- */
/* QuantPayloadSize for k4 (pkg/mcf/quant_payload.go:15-113). */
int64_t mantleHipK4PayloadSize(int64_t rows, int64_t cols);
/* quantizeTensor + quantizeK (cmd/mantle/quantize.go:352-398, 530-651), host code. */
int mantleHipQuantizeK4Host(const float* src, int64_t rows, int64_t cols, uint8_t* payload);

typedef struct {
    int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn, vocab;
    double rope_base;
    float eps;
    int tie_embeddings;
    int weight_dtype; /* rank-2 tensors: 0 or MANTLE_HIP_DTYPE_K4 (k4), MANTLE_HIP_DTYPE_BF16 (raw bf16) */
} mantleHipQwen3Config;
#define MANTLE_HIP_DTYPE_BF16 3
#define MANTLE_HIP_DTYPE_K4 0x31

/* Write a random-init (N(0,0.02), unit norm gains) Qwen3-shaped model as an MCF
 * file with k4 weights: the equivalent of `mantle pack` + `mantle quantize
 * --method k4` (pkg/mcf/pack.go:68, cmd/mantle/quantize.go:174-350); with
 * cfg->weight_dtype == MANTLE_HIP_DTYPE_BF16, `mantle pack --cast bf16`
 * (pkg/mcf/pack.go:291-294, round to nearest even, :789-793) instead. */
int mantleHipPackSyntheticQwen3(const char* path, const mantleHipQwen3Config* cfg, uint64_t seed, int threads);
/* Deterministic N(0, std) generator used by the packer (splitmix64 + Box-Muller). */
int mantleHipFillNormal(float* dst, int64_t n, uint64_t seed, float std);

/* Read-only MCF view (pkg/mcf/reader.go:21-69, pkg/mcf/tensor_index.go:132-220). */
typedef struct mantleHipMCF mantleHipMCF;
int mantleHipMCFOpen(const char* path, mantleHipMCF** out);
void mantleHipMCFClose(mantleHipMCF* f);
int mantleHipMCFTensorCount(const mantleHipMCF* f);
/* name (NUL-terminated copy into nameBuf), dtype, rank, shape[4], payload pointer into the mapping. */
int mantleHipMCFTensorInfo(const mantleHipMCF* f, int i, char* nameBuf, int nameBufLen, int* dtype, int* rank,
                           int64_t* shape, const uint8_t** data, uint64_t* size);
int mantleHipMCFFind(const mantleHipMCF* f, const char* name);
/* Section payload by type (e.g. 0x0100 = HF config.json). */
int mantleHipMCFSection(const mantleHipMCF* f, uint32_t type, const uint8_t** data, uint64_t* size);

/* ---------------- model runtime (Backend.LoadModel / core.Runtime) ---------------- */
/* One Qwen3-shaped k4 model resident in HBM, greedy decode on one stream.
 * Replaces backend.Backend.LoadModel + core.Runtime (internal/backend/backend.go:17-36,
 * internal/backend/core/interfaces.go:4-18) for the k4 decode path. */
typedef struct mantleHipModel mantleHipModel;
int mantleHipModelLoadMCF(const char* path, int maxContext, mantleHipModel** out);
/* Backend.LoadModel's core.LoadModelOptions (internal/backend/core/load_options.go:5-13),
 * per model instead of process-wide: cacheTypeK / cacheTypeV (--cache-type-k / --cache-type-v,
 * cmd/mantle/run.go:183-195, independent: MANTLE_HIP_KV_*), parityIsa (the host ISA whose
 * reduction order Mantle's CPU path would use, tensor_cpu.go:18-24: 0 scalar, 1 AVX2,
 * 2 AVX-512; HostCaps stands in for it) and useGraph (UseGraph: replay the captured decode
 * step).  The entry points without options take mantleHipSetParityISA /
 * mantleHipSetKVCacheType's current values and useGraph 1. */
typedef struct mantleHipLoadOptions {
    int cache_type_k;
    int cache_type_v;
    int parity_isa;
    int use_graph;
    int reserved[4];
} mantleHipLoadOptions;
int mantleHipModelLoadMCFWithOptions(const char* path, int maxContext, const mantleHipLoadOptions* opts,
                                     mantleHipModel** out);
int mantleHipModelLoadMCFImageWithOptions(const uint8_t* data, uint64_t size, int maxContext,
                                          const mantleHipLoadOptions* opts, mantleHipModel** out);
/* Same, from an MCF image the caller already holds in memory (Mantle keeps the file mmapped:
 * pkg/mcf/reader.go:21-69); the image is only read during the call. */
int mantleHipModelLoadMCFImage(const uint8_t* data, uint64_t size, int maxContext, mantleHipModel** out);
/* Build the model from tensors the caller already holds, for a Go LoadModel that walks
 * mcfstore.File (internal/mcfstore/file.go:28-194: Tensor / ReadTensorRaw for each payload,
 * SectionData for the HF config.json): configJSON is that section's text, each view one
 * tensor's MCF payload with its MCF dtype code (1 f32, 3 bf16, 0x31 k4) and shape.  The views
 * are only read during the call (copied into HBM). */
typedef struct mantleHipTensorView {
    const char* name;
    int dtype;
    int rank;
    int64_t shape[4];
    const uint8_t* data;
    uint64_t size;
} mantleHipTensorView;
int mantleHipModelLoadTensors(const char* configJSON, uint64_t configSize, const mantleHipTensorView* tensors,
                              int nTensors, int maxContext, const mantleHipLoadOptions* opts, mantleHipModel** out);
void mantleHipModelClose(mantleHipModel* m);
int mantleHipModelConfig(const mantleHipModel* m, mantleHipQwen3Config* out);
/* Reset(): Pos = 0 (internal/backend/simd/runtime.go:293-333). */
int mantleHipModelReset(mantleHipModel* m);
int mantleHipModelPos(const mantleHipModel* m, int* pos);
/* ForwardToken (runtime.go:224): logits of the step copied to host (vocab floats). */
int mantleHipModelForwardToken(mantleHipModel* m, int tok, float* logitsHost);
/* ForwardTokenGreedy (internal/backend/simd/runtime_greedy.go:12-67). */
int mantleHipModelForwardTokenGreedy(mantleHipModel* m, int tok, int* next);
/* PrefillTokens (internal/backend/simd/runtime_prefill.go:11-30): token-by-token,
 * as Mantle runs k4 prefill; *next receives the greedy token after the last one. */
int mantleHipModelPrefillTokens(mantleHipModel* m, const int* toks, int n, int* next);
/* prefillForwarder.PrefillTokens([]int) ([]float32, error) (internal/inference/engine.go:28-30):
 * the prompt, then the logits of its last position copied to logitsHost (vocab floats). */
int mantleHipModelPrefillTokensLogits(mantleHipModel* m, const int* toks, int n, float* logitsHost);
/* SetEffectiveContextLength (internal/backend/core/instance.go:325-339): reallocate the KV cache
 * and the other context-sized buffers for ctxLen positions (0 or more than the load-time
 * maxContext: that maxContext).  Only at position 0 (before the first token or after Reset). */
int mantleHipModelSetEffectiveContextLength(mantleHipModel* m, int ctxLen);
/* core.Runtime.UpdateRoPE (internal/backend/core/interfaces.go:14-18): recompute the RoPE tables,
 * with a new RoPE base when ropeBase > 0. */
int mantleHipModelUpdateRoPE(mantleHipModel* m, double ropeBase);
/* Greedy generation kept on the device: prompt then nGen tokens, one replay
 * of the captured decode-step graph per position, no host round trip between
 * steps.  outTokens receives the nGen generated ids. */
int mantleHipModelGenerateGreedy(mantleHipModel* m, const int* prompt, int nPrompt, int nGen, int* outTokens);
/* Launch `steps` decode steps continuing from the current position with the
 * device-side argmax feeding the next step (no host sync); for timing. */
int mantleHipModelDecodeSteps(mantleHipModel* m, int steps);
int mantleHipModelSynchronize(mantleHipModel* m);
/* Residual stream x after the last step (d_model floats) -- divergence bisection aid. */
int mantleHipModelHidden(mantleHipModel* m, float* out);
/* Use the captured HIP graph for a decode step (1, default) or plain launches (0). */
int mantleHipModelSetUseGraph(mantleHipModel* m, int on);

#ifdef __cplusplus
}
#endif
#endif
