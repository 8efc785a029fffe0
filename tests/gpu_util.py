"""Device-memory helpers for the GPU parity tests (torch is only plumbing here:
it allocates HBM and provides the stream; every computation goes through the
C ABI of libmantle_hip.so)."""
from __future__ import annotations

import numpy as np
import torch

from mantle_amd import _lib


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


_KEEP: list = []


def keep(a: np.ndarray) -> torch.Tensor:
    """Upload and keep the tensor alive until the next host() sync (a bare
    temporary could be freed and its memory reused before the kernel runs)."""
    t = dev(a)
    _KEEP.append(t)
    return t


def empty(n: int, dtype=torch.float32) -> torch.Tensor:
    return torch.empty(n, dtype=dtype, device="cuda:0")


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def call(fn: str, *args) -> None:
    _lib.call(fn, *args)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    out = t.cpu().numpy()
    _KEEP.clear()
    return out


def k4_dev(payload: np.ndarray, rows: int, cols: int):
    """Upload a k4 payload; return (keepalive, nib_ptr, super_ptr, sub_ptr)."""
    t = dev(payload)
    bpr = (cols + 31) // 32
    spr = (bpr + 7) // 8
    sub_off = (rows * spr * 2 + 63) & ~63
    data_off = (sub_off + rows * bpr + 63) & ~63
    base = t.data_ptr()
    return t, base + data_off, base, base + sub_off


def unpermute_qx(qx: np.ndarray) -> np.ndarray:
    """Undo the even/odd block permutation the GPU quantiser writes."""
    q = qx.reshape(-1, 32)
    e = np.arange(32)
    pos = ((e & 1) << 4) | ((e >> 3) << 2) | ((e >> 1) & 3)
    return q[:, pos].reshape(-1)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitexact(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    g, w = bits(got), bits(want)
    if g.shape != w.shape or not np.array_equal(g, w):
        bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
        i = int(bad[0]) if len(bad) else -1
        raise AssertionError(f"{what}: {len(bad)} of {w.size} values differ; first at {i}: "
                             f"got {got.reshape(-1)[i]!r} want {want.reshape(-1)[i]!r}")
