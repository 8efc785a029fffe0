"""MCF container access and the synthetic k4 model producer (host side).

`pack_synthetic_qwen3` is the equivalent of `mantle pack` followed by
`mantle quantize --method k4` (pkg/mcf/pack.go:68, cmd/mantle/quantize.go:174-350)
for a random-init Qwen3-shaped model: weights N(0, 0.02) from a seed, unit
RMSNorm gains, every rank-2 tensor k4-quantised with the global +/-maxAbs clip.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import I, I64, P, U64, Qwen3Config, call, lib

DTYPE_F32 = 1
DTYPE_K4 = 0x31

# Qwen3-0.6B shape.
QWEN3_0_6B = dict(n_layers=28, d_model=1024, n_heads=16, n_kv_heads=8, head_dim=128, ffn=3072,
                  vocab=151936, rope_base=1e6, eps=1e-6, tie_embeddings=1)
QWEN3_4B = dict(n_layers=36, d_model=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728,
                vocab=151936, rope_base=1e6, eps=1e-6, tie_embeddings=1)
QWEN3_8B = dict(n_layers=36, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288,
                vocab=151936, rope_base=1e6, eps=1e-6, tie_embeddings=0)


DTYPE_BF16 = 3


def make_config(**kw) -> Qwen3Config:
    """Config struct from a model dict; "weights": "bf16" selects raw bf16 tensors."""
    cfg = Qwen3Config()
    for k, v in kw.items():
        if k == "weights":
            cfg.weight_dtype = DTYPE_BF16 if v == "bf16" else 0
        else:
            setattr(cfg, k, v)
    return cfg


def pack_synthetic_qwen3(path: str, seed: int, threads: int | None = None, **cfg) -> str:
    c = make_config(**cfg)
    th = threads or min(16, os.cpu_count() or 1)
    call("mantleHipPackSyntheticQwen3", path.encode(), C.byref(c), U64(seed), th)
    return path


def pack_cached(path: str, seed: int, cfg: dict) -> str:
    """pack_synthetic_qwen3 unless `path` already exists (written atomically)."""
    if not os.path.exists(path):
        tmp = path + ".part"
        pack_synthetic_qwen3(tmp, seed, **cfg)
        os.replace(tmp, path)
    return path


def splitmix64(x: int) -> int:
    m = (1 << 64) - 1
    z = (x + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def uniform_tokens(n: int, vocab: int, seed: int) -> list[int]:
    """Uniform-random token ids: id_i = splitmix64(splitmix64(seed) + i) mod vocab
    (BASELINE config 1 prompt: 31 ids, seed 1)."""
    base = splitmix64(seed)
    return [splitmix64((base + i) & ((1 << 64) - 1)) % vocab for i in range(n)]


def payload_size(rows: int, cols: int) -> int:
    return int(lib().mantleHipK4PayloadSize(rows, cols))


def quantize_k4(w: np.ndarray) -> np.ndarray:
    """k4-quantise a float32 [rows, cols] matrix (host, bit-exact to Mantle's quantizer)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros(payload_size(rows, cols), dtype=np.uint8)
    call("mantleHipQuantizeK4Host", w.ctypes.data, I64(rows), I64(cols), out.ctypes.data)
    return out


def fill_normal(n: int, seed: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    call("mantleHipFillNormal", out.ctypes.data, I64(n), U64(seed), C.c_float(std))
    return out


def k4_regions(payload: np.ndarray, rows: int, cols: int):
    """(super f16 bits, sub u6, nibbles) views of a k4 payload (pkg/mcf/quant_payload.go:86-112)."""
    bpr = (cols + 31) // 32
    spr = (bpr + 7) // 8
    sub_off = (rows * spr * 2 + 63) & ~63
    data_off = (sub_off + rows * bpr + 63) & ~63
    sup = payload[: rows * spr * 2].view(np.uint16)
    sub = payload[sub_off: sub_off + rows * bpr]
    nib = payload[data_off: data_off + rows * bpr * 16]
    return sup, sub, nib


class MCFFile:
    """Read-only MCF view (mmap inside the library)."""

    def __init__(self, path: str):
        h = P()
        call("mantleHipMCFOpen", path.encode(), C.byref(h))
        self._h = h
        self.path = path
        self.tensors = {}
        name = C.create_string_buffer(512)
        for i in range(lib().mantleHipMCFTensorCount(h)):
            dt, rank = I(), I()
            shape = (I64 * 4)()
            data, size = P(), U64()
            call("mantleHipMCFTensorInfo", h, i, name, 512, C.byref(dt), C.byref(rank), shape, C.byref(data),
                 C.byref(size))
            self.tensors[name.value.decode()] = dict(dtype=dt.value, shape=tuple(shape[: rank.value]),
                                                     ptr=data.value, size=size.value)

    def raw(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        buf = (C.c_uint8 * t["size"]).from_address(t["ptr"])
        return np.frombuffer(buf, dtype=np.uint8)

    def section(self, typ: int) -> bytes:
        data, size = P(), U64()
        call("mantleHipMCFSection", self._h, C.c_uint32(typ), C.byref(data), C.byref(size))
        return C.string_at(data.value, size.value)

    def close(self):
        if self._h:
            lib().mantleHipMCFClose(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
