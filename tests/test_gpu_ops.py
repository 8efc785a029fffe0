"""GPU parity of the norm / RoPE / softmax / SiLU / argmax / attention kernels
against the CPU oracle (bit-exact: they reproduce Mantle's CPU lane orders)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402

ISAS = [0, 1, 2]


@pytest.fixture(autouse=True)
def _reset_isa(hip):
    yield
    g.call("mantleHipSetParityISA", 2)


@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("n", [7, 128, 1000, 1024, 2048, 3072, 4096])
def test_rmsnorm_bitexact(hip, oracle, isa, n):
    rng = np.random.default_rng(n + isa)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    g.call("mantleHipSetParityISA", isa)
    out = g.empty(n)
    g.call("mantleHipRMSNormF32", g.ptr(out), g.ptr(g.keep(x)), g.ptr(g.keep(w)), ctypes.c_float(1e-6), n, g.stream())
    g.assert_bitexact(g.host(out), oracle.rmsnorm(isa, x, w, 1e-6), f"rmsnorm isa={isa} n={n}")


@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("n", [32, 64, 1024])
def test_rmsnorm_lane_order_kat(hip, oracle, isa, n):
    """x = [4096, 1, 1, ...]: 2^24 + 1 rounds back to 2^24, so each ISA order
    gives a different sum of squares (tests/test_oracle.py pins the oracle on
    it by hand-worked sums); the kernel must match the selected order."""
    x = np.ones(n, dtype=np.float32)
    x[0] = 4096.0
    w = np.ones(n, dtype=np.float32)
    g.call("mantleHipSetParityISA", isa)
    out = g.empty(n)
    g.call("mantleHipRMSNormF32", g.ptr(out), g.ptr(g.keep(x)), g.ptr(g.keep(w)), ctypes.c_float(0.0), n, g.stream())
    g.assert_bitexact(g.host(out), oracle.rmsnorm(isa, x, w, 0.0), f"rmsnorm KAT isa={isa} n={n}")


@pytest.mark.parametrize("isa", ISAS)
def test_rmsnorm_batched_bitexact(hip, oracle, isa):
    hd, nh = 128, 16
    rng = np.random.default_rng(isa)
    x = rng.standard_normal(hd * nh).astype(np.float32)
    w = rng.standard_normal(hd).astype(np.float32)
    g.call("mantleHipSetParityISA", isa)
    out = g.empty(hd * nh)
    g.call("mantleHipRMSNormBatchedF32", g.ptr(out), g.ptr(g.keep(x)), g.ptr(g.keep(w)), ctypes.c_float(1e-6), hd, nh,
           g.stream())
    want = np.concatenate([oracle.rmsnorm(isa, x[h * hd:(h + 1) * hd], w, 1e-6) for h in range(nh)])
    g.assert_bitexact(g.host(out), want, "rmsnorm batched")


@pytest.mark.parametrize("pos", [0, 1, 31, 4095, 16383])
def test_rope_table_bitexact(hip, oracle, pos):
    hd, nh = 128, 24
    x = np.random.default_rng(pos).standard_normal(hd * nh).astype(np.float32)
    c, s = oracle.rope_tables(1e6, hd, pos)
    xd = g.dev(x)
    g.call("mantleHipApplyRoPEInplaceTableF32", g.ptr(xd), g.ptr(g.keep(c)), g.ptr(g.keep(s)), hd, hd // 2, nh,
           g.stream())
    g.assert_bitexact(g.host(xd), oracle.apply_rope(x, nh, hd, c, s), "rope")


def test_rope_f64_close(hip, oracle):
    """Device f64 cos/sin path: within 1 ulp-level tolerance of the host tables."""
    hd, nh, pos = 128, 16, 777
    x = np.random.default_rng(1).standard_normal(hd * nh).astype(np.float32)
    inv = np.array([1.0 / (1e6 ** (2 * i / hd)) for i in range(hd // 2)], dtype=np.float64)
    xd = g.dev(x)
    g.call("mantleHipApplyRoPEInplaceF64FreqF32", g.ptr(xd), g.ptr(g.keep(inv)), pos, ctypes.c_float(1.0), hd, hd // 2,
           nh, g.stream())
    c, s = oracle.rope_tables(1e6, hd, pos)
    np.testing.assert_allclose(g.host(xd), oracle.apply_rope(x, nh, hd, c, s), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("cols", [1, 5, 160, 4097])
def test_softmax_bitexact(hip, oracle, cols):
    rows = 3
    x = (np.random.default_rng(cols).standard_normal(rows * cols) * 4).astype(np.float32)
    xd = g.dev(x)
    g.call("mantleHipSoftmaxRowsF32", g.ptr(xd), rows, cols, g.stream())
    want = np.concatenate([oracle.softmax(x[r * cols:(r + 1) * cols]) for r in range(rows)])
    g.assert_bitexact(g.host(xd), want, "softmax")


@pytest.mark.parametrize("n", [3072, 3075])
def test_silu_mul_bitexact(hip, oracle, n):
    rng = np.random.default_rng(n)
    gate = (rng.standard_normal(n) * 5).astype(np.float32)
    up = rng.standard_normal(n).astype(np.float32)
    out = g.empty(n)
    g.call("mantleHipSiluMulF32", g.ptr(g.keep(gate)), g.ptr(g.keep(up)), g.ptr(out), n, g.stream())
    g.assert_bitexact(g.host(out), oracle.silu_mul(gate, up), "silu*up")


def test_argmax_first_max_wins(hip):
    x = np.zeros(151936, dtype=np.float32)
    x[[5, 70000, 151935]] = 3.0
    x[4] = -1.0
    out = g.empty(1, torch.int32)
    g.call("mantleHipArgMaxF32", g.ptr(g.keep(x)), len(x), g.ptr(out), g.stream())
    assert int(g.host(out)[0]) == 5
    x = -np.abs(np.random.default_rng(0).standard_normal(1000)).astype(np.float32)
    g.call("mantleHipArgMaxF32", g.ptr(g.keep(x)), len(x), g.ptr(out), g.stream())
    assert int(g.host(out)[0]) == int(np.argmax(x))


@pytest.mark.parametrize("case", ["nan_later", "nan_first", "signed_zero", "neg_zero_first", "all_nan_tail"])
def test_argmax_nan_and_signed_zero(hip, oracle, case):
    """argmaxHost's strict '>' (runtime_greedy.go:70-82): a NaN never wins
    unless it is x[0] (then nothing beats it), and -0 equals +0 (first wins)."""
    n = 70000
    x = np.full(n, -5.0, dtype=np.float32)
    if case == "nan_later":
        x[[10, 500]] = np.nan
        x[700] = 1.0
    elif case == "nan_first":
        x[0] = np.nan
        x[900] = 100.0
    elif case == "signed_zero":
        x[30] = np.float32(-0.0)
        x[40] = np.float32(0.0)
    elif case == "neg_zero_first":
        x[3] = np.float32(0.0)
        x[2] = np.float32(-0.0)
    else:
        x[1:] = np.nan
    want = oracle.argmax(x) if hasattr(oracle, "argmax") else None
    ref = 0
    for i in range(1, n):  # argmaxHost, literally
        if x[i] > x[ref]:
            ref = i
    if want is not None:
        assert want == ref
    out = g.empty(1, torch.int32)
    g.call("mantleHipArgMaxF32", g.ptr(g.keep(x)), n, g.ptr(out), g.stream())
    assert int(g.host(out)[0]) == ref, case


def test_add_vectors(hip):
    a = np.arange(1000, dtype=np.float32)
    b = np.full(1000, 0.5, dtype=np.float32)
    ad = g.dev(a)
    g.call("mantleHipAddVectorsF32", g.ptr(ad), g.ptr(g.keep(b)), 1000, g.stream())
    np.testing.assert_array_equal(g.host(ad), a + b)


def _fill(n, scale):  # fillTestData (internal/backend/simd/attn_test.go:240-244)
    return np.array([scale * np.float32((i % 29) - 14) for i in range(n)], dtype=np.float32)


ATTN_PATHS = {"fused": 3, "split": 0, "single": 1, "general": 2}


@pytest.mark.parametrize("path", list(ATTN_PATHS))
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("n_head,kv_heads,head_dim,pos", [(4, 2, 8, 5), (16, 8, 128, 0), (16, 8, 128, 130),
                                                         (32, 8, 128, 1000), (16, 8, 128, 1100), (8, 2, 64, 300)])
def test_attention_bitexact(hip, oracle, path, isa, n_head, kv_heads, head_dim, pos):
    """Every kernel variant bit-identical to the CPU order; 1100 keys give the
    split variant more 64-key chunks than workgroups per head."""
    kv = kv_heads * head_dim
    if head_dim == 8:
        q, ck, cv = _fill(n_head * head_dim, 0.1), _fill((pos + 1) * kv, 0.2), _fill((pos + 1) * kv, 0.3)
    else:
        rng = np.random.default_rng(pos)
        q = rng.standard_normal(n_head * head_dim).astype(np.float32)
        ck = rng.standard_normal((pos + 1) * kv).astype(np.float32)
        cv = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(head_dim))
    g.call("mantleHipSetParityISA", isa)
    g.call("mantleHipSetAttentionPath", ATTN_PATHS[path])
    out = g.empty(n_head * head_dim)
    scratch = g.empty(n_head * (pos + 1))
    g.call("mantleHipAttentionInnerF32Cache", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)), g.ptr(out),
           g.ptr(scratch), pos, 0, kv, head_dim, n_head, kv_heads, pos + 1, ctypes.c_float(scale), g.stream())
    want = oracle.attn_heads(isa, q, ck, cv, pos, kv, head_dim, n_head, kv_heads, float(scale))
    got = g.host(out)
    g.call("mantleHipSetAttentionPath", 0)
    g.assert_bitexact(got, want, "attention")


@pytest.mark.parametrize("path", ["split", "fused", "single"])
def test_attention_long_context_bitexact(hip, oracle, path):
    """16500 keys (Qwen3-8B's 16k-token prompt): the split path's V-sum launch
    holds 66 KB of probabilities in LDS, the one-launch path keeps them in the
    scores buffer (past its 64 KiB), the single-head kernel streams scores
    through global memory."""
    n_head, kv_heads, head_dim, pos = 32, 8, 128, 16499
    kv = kv_heads * head_dim
    rng = np.random.default_rng(11)
    q = rng.standard_normal(n_head * head_dim).astype(np.float32)
    ck = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    cv = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(head_dim))
    g.call("mantleHipSetParityISA", 2)
    g.call("mantleHipSetAttentionPath", ATTN_PATHS[path])
    try:
        out = g.empty(n_head * head_dim)
        scratch = g.empty(n_head * (pos + 1))
        g.call("mantleHipAttentionInnerF32Cache", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)), g.ptr(out),
               g.ptr(scratch), pos, 0, kv, head_dim, n_head, kv_heads, pos + 1, ctypes.c_float(scale), g.stream())
        want = oracle.attn_heads(2, q, ck, cv, pos, kv, head_dim, n_head, kv_heads, float(scale))
        g.assert_bitexact(g.host(out), want, "attention")
    finally:
        g.call("mantleHipSetAttentionPath", 0)


def _f16(oracle, x):
    return np.array([oracle.f32_to_f16(float(v)) for v in np.ravel(x)], dtype=np.uint16)


@pytest.mark.parametrize("path", ["split", "fused"])
@pytest.mark.parametrize("isa", [2, 0])
@pytest.mark.parametrize("n_head,kv_heads,head_dim,pos", [(16, 8, 128, 0), (16, 8, 128, 130), (32, 8, 128, 1100),
                                                         (8, 2, 64, 300)])
def test_attention_f16_cache_bitexact(hip, oracle, path, isa, n_head, kv_heads, head_dim, pos):
    """RunAttnHeads over Mantle's f16 cache (attnpool.go:103-106, :127-135): DotF16
    is the scalar order in every ISA, so the parity ISA must not change the bits."""
    kv = kv_heads * head_dim
    rng = np.random.default_rng(pos + 7)
    q = rng.standard_normal(n_head * head_dim).astype(np.float32)
    ck = _f16(oracle, rng.standard_normal((pos + 1) * kv))
    cv = _f16(oracle, rng.standard_normal((pos + 1) * kv))
    # subnormal and signed-zero bit patterns: Mantle's Float16ToFloat32 flushes them to zero
    for arr in (ck, cv):
        idx = rng.choice(arr.size, size=min(arr.size, 64), replace=False)
        arr[idx] = np.array([0x0001, 0x83FF, 0x8000, 0x0200] * 16, np.uint16)[: idx.size]
    scale = np.float32(1.0 / np.sqrt(head_dim))
    g.call("mantleHipSetParityISA", isa)
    g.call("mantleHipSetAttentionPath", ATTN_PATHS[path])
    try:
        out = g.empty(n_head * head_dim)
        # mantleCudaAttentionInnerF16CacheF32's argument list (softmax.h:70-83): no scratch
        g.call("mantleHipAttentionInnerF16CacheF32", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)),
               g.ptr(out), pos, 0, kv, head_dim, n_head, kv_heads, pos + 1, ctypes.c_float(scale), g.stream())
        got = g.host(out)
    finally:
        g.call("mantleHipSetAttentionPath", 0)
        g.call("mantleHipSetParityISA", 2)
    g.assert_bitexact(got, oracle.attn_heads_f16(q, ck, cv, pos, kv, head_dim, n_head, kv_heads, float(scale)),
                      "f16 attention")


def _mixed_cache(oracle, kind, x, rows, kv):
    """A row-major cache of `kind` from fp32 rows x: (cache, per-row scales or None)."""
    if kind == "f32":
        return x.astype(np.float32), None
    if kind == "f16":
        return _f16(oracle, x), None
    q = np.empty(rows * kv, np.int8)
    sc = np.empty(rows, np.float32)
    for t in range(rows):
        q[t * kv:(t + 1) * kv], sc[t] = oracle.store_q8(x[t * kv:(t + 1) * kv])
    return q, sc


@pytest.mark.parametrize("kt,vt", [("f16", "q8_0"), ("q8_0", "f16"), ("q8_0", "q8_0"), ("f16", "f16")])
@pytest.mark.parametrize("pos", [0, 200, 1100])
def test_attention_mixed_cache_entry_bitexact(hip, oracle, kt, vt, pos):
    """mantleCudaAttentionInnerMixedCacheF32's argument list (softmax.h:84-104):
    each of K and V f16 or q8_0, RunAttnHeads' arithmetic per type
    (attnpool.go:100-135), bit-identical to the oracle."""
    n_head, kv_heads, head_dim = 16, 8, 128
    kv = kv_heads * head_dim
    rng = np.random.default_rng(pos + 3)
    q = rng.standard_normal(n_head * head_dim).astype(np.float32)
    kx = (rng.standard_normal((pos + 1) * kv) * 2).astype(np.float32)
    vx = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    ck, ks = _mixed_cache(oracle, kt, kx, pos + 1, kv)
    cv, vs = _mixed_cache(oracle, vt, vx, pos + 1, kv)
    scale = np.float32(1.0 / np.sqrt(head_dim))
    out = g.empty(n_head * head_dim)
    dk, dv = g.keep(ck), g.keep(cv)
    dks = g.keep(ks) if ks is not None else None
    dvs = g.keep(vs) if vs is not None else None
    g.call("mantleHipAttentionInnerMixedCacheF32", g.ptr(g.keep(q)),
           g.ptr(dk) if kt == "f16" else None, g.ptr(dv) if vt == "f16" else None,
           g.ptr(dk) if kt == "q8_0" else None, g.ptr(dv) if vt == "q8_0" else None,
           g.ptr(dks) if dks is not None else None, g.ptr(dvs) if dvs is not None else None, g.ptr(out),
           int(kt == "q8_0"), int(vt == "q8_0"), pos, 0, kv, head_dim, n_head, kv_heads, 0, ctypes.c_float(scale),
           g.stream())
    want = oracle.attn_heads_mixed(2, q, kt, ck, ks, vt, cv, vs, pos, 0, 0, kv, head_dim, n_head, kv_heads,
                                   float(scale))
    g.assert_bitexact(g.host(out), want, f"mixed attention {kt}/{vt}")


@pytest.mark.parametrize("kind", ["f32", "f16", "q8_0"])
@pytest.mark.parametrize("pos,start,cache_len", [(300, 0, 0), (300, 45, 0), (300, 45, 256), (999, 744, 256),
                                                 (130, 0, 100)])
def test_attention_window_and_ring_bitexact(hip, oracle, kind, pos, start, cache_len):
    """RunAttnHeads' window start and ring placement (attnpool.go:88-99: key t at
    row t % cacheLen when 0 < cacheLen < pos + 1) through the C ABI, each cache
    type; (130, 0, 100) is the ring read past its length (keys wrap onto
    overwritten rows, as the CPU reads them)."""
    n_head, kv_heads, head_dim = 16, 8, 128
    kv = kv_heads * head_dim
    rows = cache_len if 0 < cache_len < pos + 1 else pos + 1
    rng = np.random.default_rng(pos + start + cache_len)
    q = rng.standard_normal(n_head * head_dim).astype(np.float32)
    ck, ks = _mixed_cache(oracle, kind, (rng.standard_normal(rows * kv) * 2).astype(np.float32), rows, kv)
    cv, vs = _mixed_cache(oracle, kind, rng.standard_normal(rows * kv).astype(np.float32), rows, kv)
    scale = np.float32(1.0 / np.sqrt(head_dim))
    win = pos - start + 1
    out = g.empty(n_head * head_dim)
    scratch = g.empty(n_head * win)
    if kind == "f32":
        g.call("mantleHipAttentionInnerF32Cache", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)), g.ptr(out),
               g.ptr(scratch), pos, start, kv, head_dim, n_head, kv_heads, cache_len, ctypes.c_float(scale), g.stream())
    elif kind == "f16":
        g.call("mantleHipAttentionInnerF16CacheF32", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)),
               g.ptr(out), pos, start, kv, head_dim, n_head, kv_heads, cache_len, ctypes.c_float(scale), g.stream())
    else:
        g.call("mantleHipAttentionInnerQ8CacheF32", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)),
               g.ptr(g.keep(ks)), g.ptr(g.keep(vs)), g.ptr(out), g.ptr(scratch), pos, start, kv, head_dim, n_head,
               kv_heads, cache_len, ctypes.c_float(scale), g.stream())
    want = oracle.attn_heads_mixed(2, q, kind, ck, ks, kind, cv, vs, pos, start, cache_len, kv, head_dim, n_head,
                                   kv_heads, float(scale))
    g.assert_bitexact(g.host(out), want, f"window/ring {kind} pos={pos} start={start} cacheLen={cache_len}")


def test_rope_f32_invfreq_reference_kat(hip):
    """TestApplyRoPEInplaceF32 (internal/backend/cuda/native/attn_fused_test.go:32-105):
    4 heads x 16, pos 7, attnScale 1.25, x = 0.1 i - 1.5, float32 invFreq =
    1/10000^(2i/16), against applyRoPEScalarRef (float64 angle, cos/sin to float32,
    scaled) within 1e-4; attnScale 0 is taken as 1."""
    import math
    nh, hd, half, pos = 4, 16, 8, 7
    x = np.array([np.float32(i) * np.float32(0.1) - np.float32(1.5) for i in range(nh * hd)], np.float32)
    inv = np.array([1.0 / math.pow(10000, 2 * i / hd) for i in range(half)], np.float32)

    def ref(scale):
        r = x.copy()
        for h in range(nh):
            for i in range(half):
                ang = float(pos) * float(inv[i])
                c = np.float32(math.cos(ang)) * np.float32(scale)
                s_ = np.float32(math.sin(ang)) * np.float32(scale)
                x0, x1 = r[h * hd + i], r[h * hd + i + half]
                r[h * hd + i] = x0 * c - x1 * s_
                r[h * hd + i + half] = x0 * s_ + x1 * c
        return r

    for scale, want_scale in ((1.25, 1.25), (0.0, 1.0)):
        xd = g.dev(x)
        g.call("mantleHipApplyRoPEInplaceF32", g.ptr(xd), g.ptr(g.keep(inv)), pos, ctypes.c_float(scale), hd, half,
               nh, g.stream())
        np.testing.assert_allclose(g.host(xd), ref(want_scale), atol=1e-4, rtol=0)


def test_store_kv_f16_row_truncates(hip, oracle):
    """Float32ToFloat16 (internal/backend/simd/float16.go:7-46): truncation, FTZ, inf, NaN."""
    vals = np.array([1.0, -2.5, 0.1, 65504.0, 70000.0, 1e-6, -1e-8, np.inf, np.nan, 3.14159, -0.0, 6.1e-5],
                    dtype=np.float32)
    kv = vals.size
    cache = g.empty(3 * kv, torch.int16)
    g.call("mantleHipStoreKVF16Row", g.ptr(cache), g.ptr(g.keep(vals)), 2, kv, g.stream())
    got = g.host(cache).view(np.uint16)[2 * kv:]
    np.testing.assert_array_equal(got, _f16(oracle, vals))


# storeQ8 known answers (ops_runtime.go:132-168), as the oracle tests pin them:
# +-0.5 then truncation (0.49999997 + 0.5 rounds to 1.0 in fp32), a zero row,
# and a row whose 127/maxAbs overflows (amd64's NaN / out-of-range -> -127).
Q8_ROWS = [
    np.array([127.0, 2.5, -2.5, 0.49999997, -0.49999997, 1.5, 126.5, -127.0] * 2, np.float32),
    np.zeros(16, np.float32),
    np.array([1e-38, 0.0, -1e-38, 5e-39] * 4, np.float32),
]


@pytest.mark.parametrize("case", ["kat0", "kat1", "kat2", "rand1024", "rand4096", "rand48"])
def test_store_kv_q8_row_bitexact(hip, oracle, case):
    if case.startswith("kat"):
        k = Q8_ROWS[int(case[3:])]
        v = k[::-1].copy()
    else:
        n = int(case[4:])
        rng = np.random.default_rng(n)
        k = (rng.standard_normal(n) * 3).astype(np.float32)
        v = rng.standard_normal(n).astype(np.float32)
    kv, pos = k.size, 3
    ck = g.empty(5 * kv, torch.int8)
    cv = g.empty(5 * kv, torch.int8)
    ks = g.empty(5)
    vs = g.empty(5)
    g.call("mantleHipStoreKVQ8Row", g.ptr(ck), g.ptr(cv), g.ptr(ks), g.ptr(vs), g.ptr(g.keep(k)), g.ptr(g.keep(v)),
           pos, kv, g.stream())
    for dev, sc, src, name in ((ck, ks, k, "K"), (cv, vs, v, "V")):
        want_q, want_s = oracle.store_q8(src)
        np.testing.assert_array_equal(g.host(dev)[pos * kv:(pos + 1) * kv], want_q, err_msg=f"{case} {name} row")
        assert np.float32(g.host(sc)[pos]).view(np.uint32) == np.float32(want_s).view(np.uint32), f"{case} {name} scale"


@pytest.mark.parametrize("path", ["split", "fused"])
@pytest.mark.parametrize("n_head,kv_heads,head_dim,pos", [(16, 8, 128, 0), (16, 8, 128, 130), (32, 8, 128, 1100),
                                                         (8, 2, 64, 300), (16, 8, 128, 5000)])
def test_attention_q8_cache_bitexact(hip, oracle, path, n_head, kv_heads, head_dim, pos):
    """RunAttnHeads over the q8_0 cache (attnpool.go:100-102, :122-130): DotQ8 in
    the scalar order times the key's scale, V terms (p * q) * s in key order;
    rows written by storeQ8 (one scale per position over all kv heads)."""
    kv = kv_heads * head_dim
    rng = np.random.default_rng(pos + 11)
    q = rng.standard_normal(n_head * head_dim).astype(np.float32)
    ck = np.empty((pos + 1) * kv, np.int8)
    cv = np.empty((pos + 1) * kv, np.int8)
    ks = np.empty(pos + 1, np.float32)
    vs = np.empty(pos + 1, np.float32)
    for t in range(pos + 1):
        ck[t * kv:(t + 1) * kv], ks[t] = oracle.store_q8(rng.standard_normal(kv) * (1 + t % 7))
        cv[t * kv:(t + 1) * kv], vs[t] = oracle.store_q8(rng.standard_normal(kv))
    scale = np.float32(1.0 / np.sqrt(head_dim))
    g.call("mantleHipSetAttentionPath", ATTN_PATHS[path])
    try:
        out = g.empty(n_head * head_dim)
        scratch = g.empty(n_head * (pos + 1))
        g.call("mantleHipAttentionInnerQ8CacheF32", g.ptr(g.keep(q)), g.ptr(g.keep(ck)), g.ptr(g.keep(cv)),
               g.ptr(g.keep(ks)), g.ptr(g.keep(vs)), g.ptr(out), g.ptr(scratch), pos, 0, kv, head_dim, n_head,
               kv_heads, pos + 1, ctypes.c_float(scale), g.stream())
        got = g.host(out)
    finally:
        g.call("mantleHipSetAttentionPath", 0)
    g.assert_bitexact(got, oracle.attn_heads_q8(q, ck, cv, ks, vs, pos, kv, head_dim, n_head, kv_heads, float(scale)),
                      "q8 attention")


def test_attention_q8_cache_rejects_unsupported(hip):
    """The q8_0 cache needs head_dim 64/128 (the split kernels) and 16-byte rows."""
    q = np.zeros(16 * 96, np.float32)
    c = np.zeros(4 * 8 * 96, np.int8)
    s = np.zeros(4, np.float32)
    out = g.empty(16 * 96)
    scratch = g.empty(16 * 4)
    from mantle_amd import _lib
    rc = _lib.lib().mantleHipAttentionInnerQ8CacheF32(g.ptr(g.keep(q)), g.ptr(g.keep(c)), g.ptr(g.keep(c)),
                                                      g.ptr(g.keep(s)), g.ptr(g.keep(s)), g.ptr(out), g.ptr(scratch),
                                                      3, 0, 8 * 96, 96, 16, 8, 4, ctypes.c_float(0.1), g.stream())
    assert rc != 0
