"""Model fixtures shared by the GPU model tests, smoke() and bench.py's CPU leg."""
from __future__ import annotations

import os

import numpy as np

TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=128, ffn=512, vocab=3000,
            rope_base=1e6, eps=1e-6, tie_embeddings=1)

# Two blocks at Qwen3-0.6B's row widths (1024 / 2048 / 3072 columns): every
# GEMV of the step takes the lane-chain kernel, with its fused RMSNorm.
LANE = dict(n_layers=2, d_model=1024, n_heads=16, n_kv_heads=8, head_dim=128, ffn=3072, vocab=2048,
            rope_base=1e6, eps=1e-6, tie_embeddings=1)

# Two blocks at Qwen3-4B's and Qwen3-8B's row widths (2560 / 4096 / 9728 and
# 4096 / 12288 columns): 80-, 128-, 304- and 384-block rows, the wide ones in
# pieces; 20000 logits rows take the large-matrix launch.
WIDE4B = dict(n_layers=2, d_model=2560, n_heads=32, n_kv_heads=8, head_dim=128, ffn=9728, vocab=20000,
              rope_base=1e6, eps=1e-6, tie_embeddings=1)
WIDE8B = dict(n_layers=2, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288, vocab=20000,
              rope_base=1e6, eps=1e-6, tie_embeddings=0)


def pack(path: str, seed: int, cfg: dict) -> str:
    from mantle_amd import mcf
    return mcf.pack_cached(path, seed, cfg)


def oracle_model(path: str, cfg: dict, max_ctx: int, isa: int = 2):
    """Oracle decoder over the same MCF payloads (views into the product's mmap)."""
    from mantle_amd.mcf import DTYPE_F32, MCFFile
    from oracle import oracle as o
    f = MCFFile(path)

    def tensors(name):
        raw = f.raw(name)
        return raw.view(np.float32) if f.tensors[name]["dtype"] == DTYPE_F32 else raw

    m = o.Model(cfg, tensors, max_ctx, isa)
    m._mcf = f  # keep the mapping alive
    return m


def splitmix64(x: int) -> int:
    from mantle_amd import mcf
    return mcf.splitmix64(x)


def prompt(n: int, vocab: int, seed: int) -> list[int]:
    from mantle_amd import mcf
    return mcf.uniform_tokens(n, vocab, seed)
