"""ctypes wrapper of liboracle.so -- the CPU restatement of Mantle's archsimd
decode path.  TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ISA_SCALAR, ISA_AVX2, ISA_AVX512 = 0, 1, 2

P = C.c_void_p
I = C.c_int
I64 = C.c_int64
F = C.c_float


class Config(C.Structure):
    _fields_ = [("n_layers", I), ("d_model", I), ("n_heads", I), ("n_kv_heads", I), ("head_dim", I), ("ffn", I),
                ("vocab", I), ("rope_base", C.c_double), ("eps", F), ("isa", I), ("wdtype", I), ("kv_k", I),
                ("kv_v", I)]


class Weights(C.Structure):
    _fields_ = [(n, P) for n in ("embed", "lm_head", "final_norm", "attn_norm", "wq", "wk", "wv", "q_norm",
                                 "k_norm", "wo", "ffn_norm", "w_gate", "w_up", "w_down")]


_SIGS = {
    "mo_f32_to_f16": (C.c_uint16, [F]),
    "mo_f16_to_f32": (F, [C.c_uint16]),
    "mo_quantize_k4": (I, [P, I64, I64, P]),
    "mo_k4_row_to_f32": (I, [P, I64, I64, I64, P]),
    "mo_k4_block_scales": (I, [P, I64, I64, P]),
    "mo_quantize_vec_blocks": (None, [P, I64, I64, P, P]),
    "mo_k4_matvec_w4a8": (I, [P, I64, I64, P, P]),
    "mo_k4_matvec_w4a8_q": (I, [P, I64, I64, P, P, P]),
    "mo_k4_matvec_w4a32": (I, [P, I64, I64, P, P]),
    "mo_bf16_to_f32": (F, [C.c_uint16]),
    "mo_f32_to_bf16": (C.c_uint16, [F]),
    "mo_bf16_matvec": (None, [I, P, I64, I64, P, P]),
    "mo_dot": (F, [I, P, P, I64]),
    "mo_rmsnorm": (None, [I, P, P, P, I64, F]),
    "mo_fast_exp": (F, [F]),
    "mo_softmax": (None, [P, I64]),
    "mo_fast_exp_vec_lane": (F, [F]),
    "mo_fast_silu_vec_lane": (F, [F]),
    "mo_silu_mul": (None, [P, P, P, I64]),
    "mo_rope_tables": (None, [C.c_double, I, I, P, P]),
    "mo_apply_rope": (None, [P, I, I, I, P, P]),
    "mo_attn_heads": (None, [I, P, P, P, P, I, I, I, I, I, I, F]),
    "mo_attn_heads_f16": (None, [P, P, P, P, I, I, I, I, I, I, F]),
    "mo_store_q8": (None, [P, P, P, C.c_int64]),
    "mo_attn_heads_q8": (None, [P, P, P, P, P, P, I, I, I, I, I, I, F]),
    "mo_argmax": (I64, [P, I64]),
    "mo_attn_heads_mixed": (None, [I, P, I, P, P, I, P, P, P, I, I, I, I, I, I, I, F]),
    "mo_model_create": (P, [C.POINTER(Config), C.POINTER(Weights), I]),
    "mo_model_free": (None, [P]),
    "mo_model_reset": (None, [P]),
    "mo_model_pos": (I, [P]),
    "mo_model_forward_greedy": (I64, [P, I64, P]),
    "mo_model_hidden": (None, [P, P]),
    "mo_set_threads": (None, [I]),
    "mo_get_threads": (I, []),
}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        so = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(so, name)
            fn.restype = res
            fn.argtypes = args
        _lib = so
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def set_threads(n: int) -> None:
    lib().mo_set_threads(int(n))


def f32_to_f16(v: float) -> int:
    return int(lib().mo_f32_to_f16(v))


def f16_to_f32(h: int) -> float:
    return float(lib().mo_f16_to_f32(h))


def payload_size(rows: int, cols: int) -> int:
    bpr = (cols + 31) // 32
    spr = (bpr + 7) // 8
    sub_off = (rows * spr * 2 + 63) & ~63
    data_off = (sub_off + rows * bpr + 63) & ~63
    return data_off + rows * bpr * 16


def quantize_k4(w: np.ndarray) -> np.ndarray:
    w = _f32(w)
    rows, cols = w.shape
    out = np.zeros(payload_size(rows, cols), dtype=np.uint8)
    rc = lib().mo_quantize_k4(_ptr(w), rows, cols, _ptr(out))
    if rc != 0:
        raise ValueError(f"mo_quantize_k4 rc={rc}")
    return out


def dequant_k4(payload: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        lib().mo_k4_row_to_f32(_ptr(payload), rows, cols, r, out[r].ctypes.data)
    return out


def block_scales(payload: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, (cols + 31) // 32), dtype=np.float32)
    lib().mo_k4_block_scales(_ptr(payload), rows, cols, _ptr(out))
    return out


def quantize_vec(x: np.ndarray):
    x = _f32(x)
    blocks = (len(x) + 31) // 32
    q = np.zeros(blocks * 32, dtype=np.int8)
    s = np.zeros(blocks, dtype=np.float32)
    lib().mo_quantize_vec_blocks(_ptr(x), len(x), blocks, _ptr(q), _ptr(s))
    return q, s


def matvec_w4a8(payload: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    y = np.empty(rows, dtype=np.float32)
    lib().mo_k4_matvec_w4a8(_ptr(payload), rows, cols, _ptr(x), _ptr(y))
    return y


def matvec_w4a32(payload: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    y = np.empty(rows, dtype=np.float32)
    lib().mo_k4_matvec_w4a32(_ptr(payload), rows, cols, _ptr(x), _ptr(y))
    return y


def f32_to_bf16(x) -> np.ndarray:
    """pkg/mcf/pack.go:789-793: round to nearest even on the dropped 16 bits."""
    x = _f32(x)
    return np.array([lib().mo_f32_to_bf16(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def bf16_matvec(isa: int, w_bits: np.ndarray, x) -> np.ndarray:
    """Mantle's matVecRangeBF16 (internal/backend/simd/matvec.go:406-979) in the ISA's order."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w_bits.shape
    x = _f32(x)
    y = np.empty(rows, dtype=np.float32)
    lib().mo_bf16_matvec(int(isa), _ptr(w_bits), rows, cols, _ptr(x), _ptr(y))
    return y


def dot(isa: int, a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().mo_dot(isa, _ptr(a), _ptr(b), len(a)))


def rmsnorm(isa: int, x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().mo_rmsnorm(isa, _ptr(out), _ptr(x), _ptr(w), len(x), eps)
    return out


def fast_exp(x: float) -> float:
    return float(lib().mo_fast_exp(x))


def fast_exp_vec(x: float) -> float:
    return float(lib().mo_fast_exp_vec_lane(x))


def fast_silu_vec(x: float) -> float:
    return float(lib().mo_fast_silu_vec_lane(x))


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().mo_softmax(_ptr(x), len(x))
    return x


def silu_mul(gate, up) -> np.ndarray:
    gate, up = _f32(gate), _f32(up)
    out = np.empty_like(gate)
    lib().mo_silu_mul(_ptr(out), _ptr(gate), _ptr(up), len(gate))
    return out


def rope_tables(base: float, rot_dim: int, pos: int):
    c = np.empty(rot_dim // 2, dtype=np.float32)
    s = np.empty(rot_dim // 2, dtype=np.float32)
    lib().mo_rope_tables(base, rot_dim, pos, _ptr(c), _ptr(s))
    return c, s


def apply_rope(x, n_head: int, head_dim: int, cos, sin) -> np.ndarray:
    x = _f32(x).copy()
    cos, sin = _f32(cos), _f32(sin)
    lib().mo_apply_rope(_ptr(x), n_head, head_dim, len(cos), _ptr(cos), _ptr(sin))
    return x


def attn_heads(isa: int, q, cache_k, cache_v, pos: int, kv_stride: int, head_dim: int, n_head: int,
               kv_heads: int, scale: float, start: int = 0) -> np.ndarray:
    q, ck, cv = _f32(q), _f32(cache_k), _f32(cache_v)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    lib().mo_attn_heads(isa, _ptr(q), _ptr(ck), _ptr(cv), _ptr(out), pos, start, kv_stride, head_dim, n_head,
                        kv_heads, scale)
    return out


def attn_heads_f16(q, cache_k16, cache_v16, pos: int, kv_stride: int, head_dim: int, n_head: int, kv_heads: int,
                   scale: float) -> np.ndarray:
    """RunAttnHeads over an f16 cache (attnpool.go:103-106, :127-135): uint16 f16 bits [pos+1][kv_stride]."""
    q = _f32(q)
    ck = np.ascontiguousarray(cache_k16, dtype=np.uint16)
    cv = np.ascontiguousarray(cache_v16, dtype=np.uint16)
    out = np.empty(n_head * head_dim, dtype=np.float32)
    lib().mo_attn_heads_f16(_ptr(q), _ptr(ck), _ptr(cv), _ptr(out), int(pos), 0, int(kv_stride), int(head_dim),
                            int(n_head), int(kv_heads), float(scale))
    return out


def store_q8(src):
    """storeQ8 (ops_runtime.go:132-168) of one row: (int8 row, its scale)."""
    src = _f32(src)
    dst = np.empty(len(src), dtype=np.int8)
    sc = np.zeros(1, dtype=np.float32)
    lib().mo_store_q8(_ptr(src), _ptr(dst), _ptr(sc), len(src))
    return dst, float(sc[0])


def attn_heads_q8(q, cache_k8, cache_v8, k_scale, v_scale, pos: int, kv_stride: int, head_dim: int, n_head: int,
                  kv_heads: int, scale: float) -> np.ndarray:
    """RunAttnHeads over a q8_0 cache (attnpool.go:100-102, :122-130): int8 [pos+1][kv_stride], scales [pos+1]."""
    q = _f32(q)
    ck = np.ascontiguousarray(cache_k8, dtype=np.int8)
    cv = np.ascontiguousarray(cache_v8, dtype=np.int8)
    ks, vs = _f32(k_scale), _f32(v_scale)
    out = np.empty(n_head * head_dim, dtype=np.float32)
    lib().mo_attn_heads_q8(_ptr(q), _ptr(ck), _ptr(cv), _ptr(ks), _ptr(vs), _ptr(out), int(pos), 0, int(kv_stride),
                           int(head_dim), int(n_head), int(kv_heads), float(scale))
    return out


KV_TYPES = {"f32": 0, "f16": 1, "q8_0": 2}


def attn_heads_mixed(isa, q, k_type, cache_k, k_scale, v_type, cache_v, v_scale, pos, start, cache_len, kv_stride,
                     head_dim, n_head, kv_heads, scale):
    """RunAttnHeads over K / V caches of independent types ("f32" / "f16" /
    "q8_0"; f16 caches as uint16, q8_0 as int8 with per-position scales) with
    the ring placement (cache_len) and window start."""
    q = _f32(q)
    dt = {"f32": np.float32, "f16": np.uint16, "q8_0": np.int8}
    ck = np.ascontiguousarray(cache_k, dtype=dt[k_type])
    cv = np.ascontiguousarray(cache_v, dtype=dt[v_type])
    ks = _f32(k_scale if k_scale is not None else np.zeros(1))
    vs = _f32(v_scale if v_scale is not None else np.zeros(1))
    out = np.empty(n_head * head_dim, dtype=np.float32)
    lib().mo_attn_heads_mixed(int(isa), _ptr(q), KV_TYPES[k_type], ck.ctypes.data, _ptr(ks), KV_TYPES[v_type],
                              cv.ctypes.data, _ptr(vs), _ptr(out), int(pos), int(start), int(cache_len),
                              int(kv_stride), int(head_dim), int(n_head), int(kv_heads), float(scale))
    return out


def argmax(x) -> int:
    x = _f32(x)
    return int(lib().mo_argmax(_ptr(x), len(x)))


class Model:
    """Qwen3-shaped decoder on the CPU (the greedy-token oracle), k4 weights or,
    with cfg["weights"] == "bf16", bf16 ones; cfg["kv_cache"] == "f16" stores the
    KV cache in Mantle's truncating f16, "q8_0" as int8 rows with one scale each
    (cfg["kv_cache_k"] / cfg["kv_cache_v"] set the two caches separately).

    `tensors(name) -> np.uint8 payload / np.float32 gains` supplies the weights
    (e.g. views into an MCF file); they must outlive the model.
    """

    def __init__(self, cfg: dict, tensors, max_ctx: int, isa: int = ISA_AVX512):
        self.cfg = cfg
        L = cfg["n_layers"]
        keep = []

        def raw(name):
            a = tensors(name)
            keep.append(a)
            return a.ctypes.data

        def arr(names):
            a = (P * L)(*[raw(n) for n in names])
            keep.append(a)
            return C.cast(a, P)

        lname = lambda l, s: f"model.layers.{l}.{s}"  # noqa: E731
        w = Weights()
        w.embed = raw("model.embed_tokens.weight")
        w.lm_head = w.embed if cfg.get("tie_embeddings", 1) else raw("lm_head.weight")
        w.final_norm = raw("model.norm.weight")
        for field, suffix in (("attn_norm", "input_layernorm.weight"), ("ffn_norm", "post_attention_layernorm.weight"),
                              ("q_norm", "self_attn.q_norm.weight"), ("k_norm", "self_attn.k_norm.weight"),
                              ("wq", "self_attn.q_proj.weight"), ("wk", "self_attn.k_proj.weight"),
                              ("wv", "self_attn.v_proj.weight"), ("wo", "self_attn.o_proj.weight"),
                              ("w_gate", "mlp.gate_proj.weight"), ("w_up", "mlp.up_proj.weight"),
                              ("w_down", "mlp.down_proj.weight")):
            setattr(w, field, arr([lname(l, suffix) for l in range(L)]))
        c = Config(cfg["n_layers"], cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"],
                   cfg["vocab"], cfg["rope_base"], cfg["eps"], isa, 1 if cfg.get("weights") == "bf16" else 0,
                   KV_TYPES[cfg.get("kv_cache_k", cfg.get("kv_cache", "f32"))],
                   KV_TYPES[cfg.get("kv_cache_v", cfg.get("kv_cache", "f32"))])
        self._keep = keep
        self._w = w
        self._c = c
        self._h = lib().mo_model_create(C.byref(c), C.byref(w), int(max_ctx))
        if not self._h:
            raise MemoryError("mo_model_create failed")

    def forward_greedy(self, tok: int, want_logits: bool = False):
        logits = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        nxt = lib().mo_model_forward_greedy(self._h, int(tok), logits.ctypes.data if want_logits else None)
        if nxt < 0:
            raise RuntimeError(f"oracle forward failed ({nxt})")
        return (int(nxt), logits) if want_logits else int(nxt)

    def generate_greedy(self, prompt, n_gen: int) -> list[int]:
        nxt = None
        for t in prompt:
            nxt = self.forward_greedy(t)
        out = []
        for _ in range(n_gen):
            out.append(nxt)
            if len(out) == n_gen:
                break
            nxt = self.forward_greedy(nxt)
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty(self.cfg["d_model"], dtype=np.float32)
        lib().mo_model_hidden(self._h, out.ctypes.data)
        return out

    def reset(self):
        lib().mo_model_reset(self._h)

    def close(self):
        if self._h:
            lib().mo_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
