"""mantle_amd -- MI355X (gfx950) backend for Mantle's k4 decode path.

The compute lives in libmantle_hip.so (hand-written HIP kernels behind the C
ABI in include/mantle_hip.h).  This package is the host-side mirror of
Mantle's backend seam: `Backend.load_model` -> `Runtime` with
`forward_token`, `forward_token_greedy`, `prefill_tokens`, `reset`
(internal/backend/backend.go:17-36, internal/backend/core/interfaces.go:4-18).
"""
from ._lib import HipError, Qwen3Config, lib  # noqa: F401
from .backend import Backend, Runtime, new_backend  # noqa: F401
from .mcf import MCFFile, pack_synthetic_qwen3, QWEN3_0_6B  # noqa: F401
