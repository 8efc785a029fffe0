"""Host-side mirror of Mantle's backend seam for the HIP backend.

Mantle: backend.New(name) -> Backend{Name(), LoadModel(...)} -> core.Runtime
with ForwardToken / ForwardTokenGreedy / PrefillTokens / Reset / Close
(internal/backend/backend.go:17-36, internal/backend/core/interfaces.go:4-18,
internal/inference/engine.go:129-191).  Errors surface as exceptions, as the
Go side surfaces them as `error` values; nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import I, LoadOptions, P, Qwen3Config, TensorView, call, lib

ISA = {"scalar": 0, "avx2": 1, "avx512": 2}


def new_backend(name: str = "hip") -> "Backend":
    """backend.New (internal/backend/backend.go:22-36) with the `hip` case."""
    n = name.strip().lower()
    if n in ("hip", "rocm", "auto"):
        return Backend()
    raise ValueError(f"unknown backend {name!r} (this package provides only 'hip')")


class Backend:
    def name(self) -> str:
        return "hip"

    def load_model(self, path: str, max_context: int = 4096, parity_isa: str = "avx512",
                   kv_cache: str = "f32", kv_cache_k: str | None = None, kv_cache_v: str | None = None,
                   use_graph: bool = True) -> "Runtime":
        """LoadModel with core.LoadModelOptions (internal/backend/core/load_options.go:5-13),
        per model: kv_cache "f32" (Mantle's loader default), "f16" (`mantle run`'s
        --cache-type-k/v default, cmd/mantle/run.go:183-195) or "q8_0" for both
        caches, or kv_cache_k / kv_cache_v separately."""
        opts = _options(parity_isa, kv_cache_k or kv_cache, kv_cache_v or kv_cache, use_graph)
        h = P()
        call("mantleHipModelLoadMCFWithOptions", path.encode(), int(max_context), C.byref(opts), C.byref(h))
        return Runtime(h, max_context)

    def load_model_image(self, image, max_context: int = 4096, parity_isa: str = "avx512",
                         kv_cache: str = "f32", kv_cache_k: str | None = None, kv_cache_v: str | None = None,
                         use_graph: bool = True) -> "Runtime":
        """LoadModel from an MCF image already in memory (bytes / numpy uint8)."""
        opts = _options(parity_isa, kv_cache_k or kv_cache, kv_cache_v or kv_cache, use_graph)
        buf = np.frombuffer(image, dtype=np.uint8) if not isinstance(image, np.ndarray) else image
        h = P()
        call("mantleHipModelLoadMCFImageWithOptions", buf.ctypes.data, C.c_uint64(buf.nbytes), int(max_context),
             C.byref(opts), C.byref(h))
        return Runtime(h, max_context)


    def load_model_tensors(self, config_json: bytes, tensors, max_context: int = 4096, parity_isa: str = "avx512",
                           kv_cache: str = "f32", kv_cache_k: str | None = None, kv_cache_v: str | None = None,
                           use_graph: bool = True) -> "Runtime":
        """LoadModel from tensors the caller holds, as a Go backend walking
        mcfstore.File would (internal/mcfstore/file.go:28-194: SectionData for
        config.json, ReadTensorRaw per tensor): `tensors` yields (name, MCF dtype
        code, shape, uint8 payload)."""
        opts = _options(parity_isa, kv_cache_k or kv_cache, kv_cache_v or kv_cache, use_graph)
        items = list(tensors)
        views = (TensorView * len(items))()
        keep = []
        for v, (name, dtype, shape, payload) in zip(views, items):
            buf = np.ascontiguousarray(payload).view(np.uint8)
            nm = name.encode()
            keep += [buf, nm]
            v.name, v.dtype, v.rank = nm, int(dtype), len(shape)
            for i, d in enumerate(shape):
                v.shape[i] = int(d)
            v.data, v.size = buf.ctypes.data, buf.nbytes
        h = P()
        call("mantleHipModelLoadTensors", config_json, len(config_json), views, len(items), int(max_context),
             C.byref(opts), C.byref(h))
        return Runtime(h, max_context)


KV = {"f32": 0, "f16": 1, "q8_0": 2}


def _options(isa: str, k: str, v: str, use_graph: bool) -> LoadOptions:
    if isa not in ISA or k not in KV or v not in KV:
        raise ValueError(f"bad load options isa={isa!r} kv_cache_k={k!r} kv_cache_v={v!r}")
    o = LoadOptions()
    o.cache_type_k, o.cache_type_v, o.parity_isa, o.use_graph = KV[k], KV[v], ISA[isa], int(bool(use_graph))
    return o


class Runtime:
    def __init__(self, handle: P, max_context: int):
        self._h = handle
        self.max_context = max_context
        self._load_context = max_context
        cfg = Qwen3Config()
        call("mantleHipModelConfig", handle, C.byref(cfg))
        self.config = cfg.as_dict()

    def _handle(self):
        if not self._h:
            raise RuntimeError("runtime is closed")
        return self._h

    @property
    def pos(self) -> int:
        p = I()
        call("mantleHipModelPos", self._handle(), C.byref(p))
        return p.value

    def reset(self) -> None:
        call("mantleHipModelReset", self._handle())

    def forward_token(self, tok: int) -> np.ndarray:
        logits = np.empty(self.config["vocab"], dtype=np.float32)
        call("mantleHipModelForwardToken", self._handle(), int(tok), logits.ctypes.data)
        return logits

    def forward_token_greedy(self, tok: int) -> int:
        nxt = I()
        call("mantleHipModelForwardTokenGreedy", self._handle(), int(tok), C.byref(nxt))
        return nxt.value

    def prefill_tokens(self, toks) -> int:
        arr = np.ascontiguousarray(toks, dtype=np.int32)
        nxt = I()
        call("mantleHipModelPrefillTokens", self._handle(), arr.ctypes.data, len(arr), C.byref(nxt))
        return nxt.value

    def prefill_tokens_logits(self, toks) -> np.ndarray:
        """prefillForwarder.PrefillTokens: the logits after the last prompt token."""
        arr = np.ascontiguousarray(toks, dtype=np.int32)
        logits = np.empty(self.config["vocab"], dtype=np.float32)
        call("mantleHipModelPrefillTokensLogits", self._handle(), arr.ctypes.data, len(arr), logits.ctypes.data)
        return logits

    def set_effective_context_length(self, n: int) -> None:
        call("mantleHipModelSetEffectiveContextLength", self._handle(), int(n))
        self.max_context = int(n) if 0 < n < self._load_context else self._load_context

    def update_rope(self, rope_base: float = 0.0) -> None:
        call("mantleHipModelUpdateRoPE", self._handle(), float(rope_base))

    def model_config(self) -> dict:
        """core.Runtime.ModelConfig."""
        cfg = Qwen3Config()
        call("mantleHipModelConfig", self._handle(), C.byref(cfg))
        return cfg.as_dict()

    def generate_greedy(self, prompt, n_gen: int) -> list[int]:
        arr = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_gen, dtype=np.int32)
        call("mantleHipModelGenerateGreedy", self._handle(), arr.ctypes.data, len(arr), int(n_gen),
             out.ctypes.data)
        return out.tolist()

    def decode_steps(self, steps: int) -> None:
        """Enqueue `steps` device-fed greedy steps (asynchronous)."""
        call("mantleHipModelDecodeSteps", self._handle(), int(steps))

    def synchronize(self) -> None:
        call("mantleHipModelSynchronize", self._handle())

    def hidden(self) -> np.ndarray:
        out = np.empty(self.config["d_model"], dtype=np.float32)
        call("mantleHipModelHidden", self._handle(), out.ctypes.data)
        return out

    def set_use_graph(self, on: bool) -> None:
        call("mantleHipModelSetUseGraph", self._handle(), int(bool(on)))

    def close(self) -> None:
        if self._h:
            lib().mantleHipModelClose(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
