"""ctypes binding of libmantle_hip.so (the C ABI in include/mantle_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback behind any entry point of this package.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# MANTLE_HIP_LIB selects another build of the same library (the phase-trace one).
LIB_PATH = os.environ.get("MANTLE_HIP_LIB") or os.path.join(_HERE, "libmantle_hip.so")

P = C.c_void_p
I = C.c_int
I64 = C.c_int64
U64 = C.c_uint64
F = C.c_float
D = C.c_double


class Qwen3Config(C.Structure):
    _fields_ = [
        ("n_layers", I), ("d_model", I), ("n_heads", I), ("n_kv_heads", I), ("head_dim", I),
        ("ffn", I), ("vocab", I), ("rope_base", D), ("eps", F), ("tie_embeddings", I), ("weight_dtype", I),
    ]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


# name -> (restype, argtypes)
class LoadOptions(C.Structure):
    """mantleHipLoadOptions: core.LoadModelOptions (internal/backend/core/load_options.go:5-13)."""
    _fields_ = [("cache_type_k", I), ("cache_type_v", I), ("parity_isa", I), ("use_graph", I), ("reserved", I * 4)]


class TensorView(C.Structure):
    """mantleHipTensorView: one MCF tensor payload held by the caller."""
    _fields_ = [("name", C.c_char_p), ("dtype", I), ("rank", I), ("shape", I64 * 4), ("data", P), ("size", U64)]


_SIGS = {
    "mantleHipGetErrorString": (C.c_char_p, [I]),
    "mantleHipGetDeviceCount": (I, [C.POINTER(I)]),
    "mantleHipSetParityISA": (I, [I]),
    "mantleHipSetAttentionPath": (I, [I]),
    "mantleHipGetAttentionPath": (I, []),
    "mantleHipGetParityISA": (I, []),
    "mantleHipMatVecBF16F32": (I, [P, P, P, I, I, P]),
    "mantleHipAttentionInnerF16CacheF32": (I, [P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "mantleHipAttentionInnerMixedCacheF32": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, F, P]),
    "mantleHipStoreKVF16Row": (I, [P, P, I, I, P]),
    "mantleHipAttentionInnerQ8CacheF32": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "mantleHipStoreKVQ8Row": (I, [P, P, P, P, P, P, I, I, P]),
    "mantleHipSetKVCacheType": (I, [I]),
    "mantleHipGetKVCacheType": (I, []),
    "mantleHipQuantMatVecK4F32": (I, [P, P, P, P, P, I, I, I, P]),
    "mantleHipQuantMatVecK4F32Batched": (I, [P, P, P, P, P, I, I, I, I, P]),
    "mantleHipQuantMatVecK4W4A8F32": (I, [P, P, P, P, P, I, I, I, I, P, P, P]),
    "mantleHipQuantMatMulK4W4A8F32": (I, [P, P, P, P, P, I, I, I, I, P, P, P]),
    "mantleHipQuantMatVecK4W4A8QF32": (I, [P, P, P, P, P, P, I, I, I, I, P]),
    "mantleHipQuantMatVecK4W4A8F32NoAlloc": (I, [P, P, P, P, P, I, I, I, I, P]),
    "mantleHipDequantizeK4ToF16": (I, [P, P, P, P, I, I, I, P]),
    "mantleHipDequantizeK4ToF32": (I, [P, P, P, P, I, I, I, P]),
    "mantleHipQuantizeVecBlocksF32": (I, [P, I, P, P, P]),
    "mantleHipRMSNormF32": (I, [P, P, P, F, I, P]),
    "mantleHipRMSNormBatchedF32": (I, [P, P, P, F, I, I, P]),
    "mantleHipApplyRoPEInplaceF32": (I, [P, P, I, F, I, I, I, P]),
    "mantleHipApplyRoPEInplaceF64FreqF32": (I, [P, P, I, F, I, I, I, P]),
    "mantleHipApplyRoPEInplaceTableF32": (I, [P, P, P, I, I, I, P]),
    "mantleHipStoreKVF32Row": (I, [P, P, I, I, P]),
    "mantleHipAttentionInnerF32Cache": (I, [P, P, P, P, P, I, I, I, I, I, I, I, F, P]),
    "mantleHipAttentionPrefillBF16": (I, [P, P, P, P, P, P, I, I, I, I, F, P, C.c_size_t, P]),
    "mantleHipAttentionPrefillWorkspaceSize": (I, [I, I, I, I, C.POINTER(C.c_size_t)]),
    "mantleHipSoftmaxRowsF32": (I, [P, I, I, P]),
    "mantleHipSiluMulF32": (I, [P, P, P, I, P]),
    "mantleHipAddVectorsF32": (I, [P, P, I, P]),
    "mantleHipArgMaxF32": (I, [P, I, P, P]),
    "mantleHipK4PayloadSize": (I64, [I64, I64]),
    "mantleHipQuantizeK4Host": (I, [P, I64, I64, P]),
    "mantleHipPackSyntheticQwen3": (I, [C.c_char_p, C.POINTER(Qwen3Config), U64, I]),
    "mantleHipFillNormal": (I, [P, I64, U64, F]),
    "mantleHipMCFOpen": (I, [C.c_char_p, C.POINTER(P)]),
    "mantleHipMCFClose": (None, [P]),
    "mantleHipMCFTensorCount": (I, [P]),
    "mantleHipMCFTensorInfo": (I, [P, I, C.c_char_p, I, C.POINTER(I), C.POINTER(I), C.POINTER(I64),
                                   C.POINTER(P), C.POINTER(U64)]),
    "mantleHipMCFFind": (I, [P, C.c_char_p]),
    "mantleHipMCFSection": (I, [P, C.c_uint32, C.POINTER(P), C.POINTER(U64)]),
    "mantleHipModelLoadMCF": (I, [C.c_char_p, I, C.POINTER(P)]),
    "mantleHipModelLoadMCFImage": (I, [P, U64, I, C.POINTER(P)]),
    "mantleHipModelLoadMCFWithOptions": (I, [C.c_char_p, I, C.POINTER(LoadOptions), C.POINTER(P)]),
    "mantleHipModelLoadMCFImageWithOptions": (I, [P, U64, I, C.POINTER(LoadOptions), C.POINTER(P)]),
    "mantleHipModelClose": (None, [P]),
    "mantleHipModelConfig": (I, [P, C.POINTER(Qwen3Config)]),
    "mantleHipModelReset": (I, [P]),
    "mantleHipModelPos": (I, [P, C.POINTER(I)]),
    "mantleHipModelForwardToken": (I, [P, I, P]),
    "mantleHipModelForwardTokenGreedy": (I, [P, I, C.POINTER(I)]),
    "mantleHipModelPrefillTokens": (I, [P, P, I, C.POINTER(I)]),
    "mantleHipModelPrefillTokensLogits": (I, [P, P, I, P]),
    "mantleHipModelSetEffectiveContextLength": (I, [P, I]),
    "mantleHipModelUpdateRoPE": (I, [P, C.c_double]),
    "mantleHipModelLoadTensors": (I, [C.c_char_p, U64, C.POINTER(TensorView), I, I, C.POINTER(LoadOptions),
                                      C.POINTER(P)]),
    "mantleHipModelGenerateGreedy": (I, [P, P, I, I, P]),
    "mantleHipModelDecodeSteps": (I, [P, I]),
    "mantleHipModelSynchronize": (I, [P]),
    "mantleHipModelHidden": (I, [P, P]),
    "mantleHipModelSetUseGraph": (I, [P, I]),
}

_lib = None


class HipError(RuntimeError):
    def __init__(self, fn: str, code: int):
        msg = lib().mantleHipGetErrorString(code)
        super().__init__(f"{fn} failed: hip error {code} ({msg.decode() if msg else '?'})")
        self.code = code


def lib() -> C.CDLL:
    """The loaded libmantle_hip.so; raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mantle_amd.build`")
        so = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(so, name)
            fn.restype = res
            fn.argtypes = args
        _lib = so
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(fn: str, code: int) -> None:
    if code != 0:
        raise HipError(fn, code)


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))
