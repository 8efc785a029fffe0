"""Causal GQA prefill attention on bf16 MFMA (config 3) against the CPU path.

Mantle prefills position by position: RoPE on q and k, then RunAttnHeads over
keys 0..t (internal/backend/simd/runtime_prefill.go:11-30, attnpool.go:77-153);
the oracle restates exactly that.  The MFMA kernel rounds the RoPE'd q / k and
the probabilities to bf16, so it is checked within the tolerance the path states
(max-abs 1e-3 plus rel 1e-2), not bit for bit; rows of a long prompt are checked
against a float64 evaluation of the same formula."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402

HD = 128
ATOL, RTOL = 1e-3, 1e-2


def bf16(x):
    """float32 -> (bf16 bits rounded to nearest even, their float32 values)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b, (b.astype(np.uint32) << 16).view(np.float32)


def make_inputs(seq, nh, kvh, seed=3):
    """Q / K / V bf16 N(0, 1) from one seeded generator (config 3)."""
    rng = np.random.default_rng(seed)
    qb, qf = bf16(rng.standard_normal(seq * nh * HD).astype(np.float32))
    kb, kf = bf16(rng.standard_normal(seq * kvh * HD).astype(np.float32))
    vb, vf = bf16(rng.standard_normal(seq * kvh * HD).astype(np.float32))
    return (qb, kb, vb), (qf.reshape(seq, nh * HD), kf.reshape(seq, kvh * HD), vf.reshape(seq, kvh * HD))


def rope_tables(oracle, seq):
    cs = [oracle.rope_tables(1e6, HD, t) for t in range(seq)]
    return (np.stack([c for c, _ in cs]).astype(np.float32), np.stack([s for _, s in cs]).astype(np.float32))


def workspace(seq, nh, kvh):
    n = ctypes.c_size_t()
    g.call("mantleHipAttentionPrefillWorkspaceSize", seq, nh, kvh, HD, ctypes.byref(n))
    return g.empty(n.value, dtype=torch.uint8), n.value


def run_gpu(bits, cos, sin, seq, nh, kvh, scale):
    qb, kb, vb = (g.keep(b) for b in bits)
    out = g.empty(seq * nh * HD)
    cp = g.ptr(g.keep(cos)) if cos is not None else None
    sp = g.ptr(g.keep(sin)) if sin is not None else None
    ws, nws = workspace(seq, nh, kvh)
    g.call("mantleHipAttentionPrefillBF16", g.ptr(qb), g.ptr(kb), g.ptr(vb), cp, sp, g.ptr(out), seq, nh, kvh, HD,
           ctypes.c_float(scale), g.ptr(ws), nws, g.stream())
    return g.host(out).reshape(seq, nh * HD)


def oracle_prefill(oracle, qf, kf, vf, cos, sin, seq, nh, kvh, scale):
    """Mantle's CPU prefill: per position, RoPE then RunAttnHeads over keys 0..t."""
    if cos is not None:
        kr = np.stack([oracle.apply_rope(kf[t], kvh, HD, cos[t], sin[t]) for t in range(seq)])
    else:
        kr = kf
    out = np.empty((seq, nh * HD), np.float32)
    for t in range(seq):
        qr = oracle.apply_rope(qf[t], nh, HD, cos[t], sin[t]) if cos is not None else qf[t]
        out[t] = oracle.attn_heads(2, qr, kr[: t + 1].ravel(), vf[: t + 1].ravel(), t, kvh * HD, HD, nh, kvh, scale)
    return out


def f64_rows(qf, kf, vf, cos, sin, rows, nh, kvh, scale):
    """float64 causal attention with the same RoPE pairs (i, i + 64), for selected query rows."""
    def rope(x, t, heads):
        x = x.astype(np.float64).reshape(heads, HD)
        c, s = cos[t].astype(np.float64), sin[t].astype(np.float64)
        x0, x1 = x[:, :64].copy(), x[:, 64:].copy()
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=1)
    n_keys = max(rows) + 1
    kr = np.stack([rope(kf[t], t, kvh) for t in range(n_keys)])  # [t][kvh][hd]
    v = vf[:n_keys].astype(np.float64).reshape(n_keys, kvh, HD)
    out = {}
    for t in rows:
        q = rope(qf[t], t, nh)
        o = np.empty((nh, HD))
        for h in range(nh):
            g_ = h * kvh // nh
            sc = kr[: t + 1, g_] @ q[h] * scale
            p = np.exp(sc - sc.max())
            p /= p.sum()
            o[h] = p @ v[: t + 1, g_]
        out[t] = o.ravel()
    return out


@pytest.mark.parametrize("seq,nh,kvh,rope", [(64, 16, 8, True), (200, 16, 8, True), (130, 4, 4, True),
                                             (96, 32, 8, True), (77, 16, 8, False)])
def test_prefill_matches_cpu_path(hip, oracle, seq, nh, kvh, rope):
    """GQA 2 and 4, plain multi-head, lengths off the 32/64 tiles, with and without RoPE."""
    bits, (qf, kf, vf) = make_inputs(seq, nh, kvh)
    cos, sin = rope_tables(oracle, seq) if rope else (None, None)
    scale = float(np.float32(1.0 / np.sqrt(HD)))
    got = run_gpu(bits, cos, sin, seq, nh, kvh, scale)
    want = oracle_prefill(oracle, qf, kf, vf, cos, sin, seq, nh, kvh, scale)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_prefill_long_prompt_rows_f64(hip, oracle):
    """2048 positions (config 3's middle size): first, last and interior rows vs float64."""
    seq, nh, kvh = 2048, 16, 8
    bits, (qf, kf, vf) = make_inputs(seq, nh, kvh)
    cos, sin = rope_tables(oracle, seq)
    scale = float(np.float32(1.0 / np.sqrt(HD)))
    got = run_gpu(bits, cos, sin, seq, nh, kvh, scale)
    rows = [0, 1, 31, 32, 63, 64, 1000, 2047]
    want = f64_rows(qf, kf, vf, cos, sin, rows, nh, kvh, scale)
    for t in rows:
        np.testing.assert_allclose(got[t], want[t], atol=ATOL, rtol=RTOL, err_msg=f"row {t}")
    assert np.isfinite(got).all()


def test_prefill_rejects_bad_shapes(hip):
    z = g.empty(16)
    p = g.ptr(z)
    f = ctypes.c_float(1.0)
    from mantle_amd import _lib
    L = _lib.lib()
    big = 1 << 30
    assert L.mantleHipAttentionPrefillBF16(p, p, p, None, None, p, 4, 16, 8, 64, f, p, big, None) != 0  # head_dim 64
    assert L.mantleHipAttentionPrefillBF16(p, p, p, None, None, p, 4, 16, 6, 128, f, p, big, None) != 0  # 16 % 6
    assert L.mantleHipAttentionPrefillBF16(p, p, p, p, None, p, 4, 16, 8, 128, f, p, big, None) != 0  # cos, no sin
    assert L.mantleHipAttentionPrefillBF16(p, p, p, None, None, p, 0, 16, 8, 128, f, p, big, None) != 0  # empty
    assert L.mantleHipAttentionPrefillBF16(p, p, p, None, None, p, 4, 16, 8, 128, f, p, 16, None) != 0  # workspace
    assert L.mantleHipAttentionPrefillBF16(p, p, p, None, None, p, 4, 16, 8, 128, f, None, big, None) != 0


@pytest.mark.parametrize("case", ["v_1e5", "k_1e5_q_1e-6", "q_1e5_k_1e-6", "all_1e-6", "mixed_tiles"])
def test_prefill_fp16_range(hip, oracle, case):
    """bf16 inputs outside fp16's range (|x| > 65504) or in its subnormals
    (|x| < 6.1e-5): the kernel scales each operand block by a power of two
    before its fp16 conversion, so it still matches the CPU path (fp32 on the
    bf16 values) within max-abs 1e-3 (relative to the output's scale) + rel 1e-2."""
    seq, nh, kvh = 130, 16, 8
    rng = np.random.default_rng(17)
    qs, ks, vs = {"v_1e5": (1, 1, 1e5), "k_1e5_q_1e-6": (1e-6, 1e5, 1), "q_1e5_k_1e-6": (1e5, 1e-6, 1),
                  "all_1e-6": (1e-6, 1e-6, 1e-6), "mixed_tiles": (1, 1, 1)}[case]
    q = rng.standard_normal(seq * nh * HD).astype(np.float32) * np.float32(qs)
    k = rng.standard_normal(seq * kvh * HD).astype(np.float32) * np.float32(ks)
    v = rng.standard_normal(seq * kvh * HD).astype(np.float32) * np.float32(vs)
    if case == "mixed_tiles":  # V tiles of very different magnitudes, one K tile past fp16's range
        v.reshape(seq, -1)[32:64] *= np.float32(3e5)
        v.reshape(seq, -1)[96:] *= np.float32(1e-5)
        k.reshape(seq, -1)[64:96] *= np.float32(2e5)
        q *= np.float32(1e-5)
    qb, qf = bf16(q)
    kb, kf = bf16(k)
    vb, vf = bf16(v)
    qf, kf, vf = qf.reshape(seq, nh * HD), kf.reshape(seq, kvh * HD), vf.reshape(seq, kvh * HD)
    cos, sin = rope_tables(oracle, seq)
    scale = float(np.float32(1.0 / np.sqrt(HD)))
    got = run_gpu((qb, kb, vb), cos, sin, seq, nh, kvh, scale)
    want = oracle_prefill(oracle, qf, kf, vf, cos, sin, seq, nh, kvh, scale)
    assert np.isfinite(want).all() and np.isfinite(got).all()
    # the absolute tolerance scales with the largest |v| a row's keys (0..t) reach
    vis = np.maximum.accumulate(np.abs(vf).max(axis=1))[:, None]
    bad = np.abs(got - want) > ATOL * vis + RTOL * np.abs(want)
    assert not bad.any(), f"{int(bad.sum())} outputs out of tolerance, first at {np.argwhere(bad)[0]}"

