"""Pins the CPU oracle: known-answer tests from Mantle's own test files,
closed forms that a plausible slip (dropped term, wrong lane order, wrong
index, wrong rounding) would break, and float64 references within tolerance."""
import math

import numpy as np
import pytest

from oracle import oracle as o


# ---------------------------------------------------------------- fp16 ----
@pytest.mark.parametrize("v,bits", [(1.0, 0x3C00), (0.04, 0x291E), (0.1, 0x2E66), (-0.1, 0xAE66), (65504.0, 0x7BFF),
                                    (65536.0, 0x7C00), (1e-8, 0x0000), (-1e-8, 0x8000), (6.1035156e-05, 0x0400),
                                    (float("inf"), 0x7C00), (float("nan"), 0x7E00)])
def test_f32_to_f16_truncating_kat(v, bits):
    """Float32ToFloat16 (internal/backend/simd/float16.go:7-46) truncates the
    mantissa and flushes f16-subnormal results to zero; 0.04 -> 0x291E is the
    scale TestRowToQuant uses (internal/backend/simd/matvec_quant_test.go:9-29)."""
    assert o.f32_to_f16(v) == bits


def test_f32_to_f16_truncates_never_rounds_up():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(20000) * 10).astype(np.float32)
    v = v[np.abs(v) > 1e-4]
    t = np.array([o.f32_to_f16(float(x)) for x in v], dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.all(np.abs(t) <= np.abs(v))
    assert np.all(np.abs(v - t) < np.abs(v) * 2.0 ** -10)


@pytest.mark.parametrize("bits,v", [(0x3C00, 1.0), (0x0001, 0.0), (0x03FF, 0.0), (0x8001, -0.0), (0x0400, 2.0 ** -14),
                                    (0x7BFF, 65504.0), (0x7C00, float("inf"))])
def test_f16_to_f32_ftz_kat(bits, v):
    """Float16ToFloat32 (internal/backend/core/float16.go:42-64): subnormals -> 0."""
    assert o.f16_to_f32(bits) == v


# -------------------------------------------------------------- layout ----
@pytest.mark.parametrize("rows,cols,size", [(3072, 1024, 1_695_744), (1024, 3072, 1_695_744), (2048, 1024, 1_130_496),
                                            (1024, 1024, 565_248), (1024, 2048, 1_130_496),
                                            (151936, 1024, 83_868_672), (2, 96, 64 + 64 + 96), (1, 1, 64 + 64 + 16)])
def test_payload_size(rows, cols, size):
    """QuantPayloadSize (pkg/mcf/quant_payload.go:15-113) at the BASELINE shapes."""
    assert o.payload_size(rows, cols) == size


# ------------------------------------------------------------ quantizer ----
def test_quantize_k4_kat_single_block():
    """One block, values k*0.1: block scale 0.7/7 = 0.1 = super; the stored super
    is the TRUNCATED f16 0x2E66, u6 = 32, q = k; dequant w = f16(0x2E66) * k."""
    k = np.array([(i % 15) - 7 for i in range(32)], dtype=np.float32)
    w = (k * np.float32(0.1)).astype(np.float32).reshape(1, 32)
    p = o.quantize_k4(w)
    assert int(p[0]) | (int(p[1]) << 8) == 0x2E66
    assert p[64] == 32
    nib = p[128:144]
    q = np.empty(32, dtype=np.int8)
    q[0::2] = (nib & 0xF).astype(np.int8)
    q[1::2] = (nib >> 4).astype(np.int8)
    q = np.where(q > 7, q - 16, q)
    np.testing.assert_array_equal(q, k.astype(np.int8))
    np.testing.assert_array_equal(o.dequant_k4(p, 1, 32)[0], (k * np.float32(o.f16_to_f32(0x2E66))).astype(np.float32))


def test_quantize_k4_kat_sub_scale_uses_unrounded_super():
    """Second block with max 0.35: s_b = 0.05, ratio to the fp32 super 0.1 is
    0.5 -> u6 = 16 and q = round(v / (0.1 * 16/32)) with the UNROUNDED super."""
    a = np.zeros(64, dtype=np.float32)
    a[0] = 0.7
    a[32:64] = np.array([((i % 15) - 7) * 0.05 for i in range(32)], dtype=np.float32)
    p = o.quantize_k4(a.reshape(1, 64))
    assert p[64] == 32 and p[65] == 16
    q = o.dequant_k4(p, 1, 64)[0, 32:] / np.float32(o.f16_to_f32(0x2E66) * 0.5)
    np.testing.assert_array_equal(np.round(q), [((i % 15) - 7) for i in range(32)])


def test_quantize_k4_error_bound_and_ranges():
    rng = np.random.default_rng(1)
    for rows, cols in [(7, 300), (16, 1024), (3, 33)]:
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        p = o.quantize_k4(w)
        bpr = (cols + 31) // 32
        spr = (bpr + 7) // 8
        sub_off = (rows * spr * 2 + 63) & ~63
        sub = p[sub_off:sub_off + rows * bpr]
        assert sub.max() <= 63 and sub.min() >= 1
        d = o.dequant_k4(p, rows, cols)
        s = np.repeat(o.block_scales(p, rows, cols), 32, axis=1)[:, :cols]
        # |w - q*s_unrounded| <= s/2 and the truncated super shifts q*s by < 7*s*2^-10
        assert np.all(np.abs(d - w) <= s * (0.5 + 8 * 2.0 ** -10) * 1.001 + 1e-12)


def test_quantize_k4_zero_and_padding():
    p = o.quantize_k4(np.zeros((2, 40), dtype=np.float32))
    assert not p.any()
    w = np.ones((1, 40), dtype=np.float32)
    d = o.dequant_k4(o.quantize_k4(w), 1, 40)
    np.testing.assert_allclose(d, w, rtol=2e-3)


# -------------------------------------------------------- int8 activations ----
def test_quantize_vec_kat():
    """quantizeVecBlocksInto (internal/backend/simd/matvec_quant.go:746-797):
    maxAbs 127 -> scale 1, ties round away from zero, zero block -> scale 0."""
    x = np.zeros(96, dtype=np.float32)
    x[0:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.49, 3.0]
    x[64:96] = np.float32(-7.0)
    q, s = o.quantize_vec(x)
    np.testing.assert_array_equal(s, [1.0, 0.0, np.float32(7.0) / np.float32(127.0)])
    np.testing.assert_array_equal(q[0:8], [127, 3, -3, 1, -1, 127, -126, 3])
    assert not q[32:64].any()
    np.testing.assert_array_equal(q[64:96], -127)


# -------------------------------------------------------------- GEMV ----
def _kat_payload(rows, cols):
    """TestQuantMatVecK4F32 fixture (internal/backend/cuda/native/runtime_test.go:425-470):
    super = fp16(1.0), u6 = 32, q = (i+b)%13-6."""
    bpr = (cols + 31) // 32
    q = np.array([[(i + b) % 13 - 6 for i in range(32)] for b in range(rows * bpr)], dtype=np.int8)
    p = np.zeros(o.payload_size(rows, cols), dtype=np.uint8)
    spr = (bpr + 7) // 8
    p[:rows * spr * 2].view(np.uint16)[:] = 0x3C00
    sub_off = (rows * spr * 2 + 63) & ~63
    data_off = (sub_off + rows * bpr + 63) & ~63
    p[sub_off:sub_off + rows * bpr] = 32
    nib = (q.astype(np.int16) & 0xF).astype(np.uint8)
    p[data_off:data_off + rows * bpr * 16] = (nib[:, 0::2] | (nib[:, 1::2] << 4)).reshape(-1)
    return p, q.reshape(rows, bpr * 32)[:, :cols]


def test_w4a32_kat():
    rows, cols = 2, 96
    p, q = _kat_payload(rows, cols)
    x = np.array([((i % 17) - 8) * 0.125 for i in range(cols)], dtype=np.float32)
    want = q.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_array_equal(o.matvec_w4a32(p, rows, cols, x), want.astype(np.float32))
    np.testing.assert_array_equal(o.dequant_k4(p, rows, cols), q.astype(np.float32))


def test_w4a8_closed_form_integer_activations():
    """Integer activations whose block max is 127 quantise exactly (scale 1), so
    the W4A8 result is the exact integer matmul."""
    rows, cols = 5, 256
    p, q = _kat_payload(rows, cols)
    rng = np.random.default_rng(2)
    x = rng.integers(-127, 128, size=cols).astype(np.float32)
    x[0::32] = 127.0
    want = (q.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(o.matvec_w4a8(p, rows, cols, x), want)


def test_w4a8_numpy_emulation():
    """Independent numpy formulation: int64 block dots of the decoded nibbles
    with the int8 activations, term = f32(dot) * f32(s_w*s_x), blocks added in
    order in float32."""
    rng = np.random.default_rng(3)
    rows, cols = 9, 200
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    p = o.quantize_k4(w)
    bpr = (cols + 31) // 32
    spr = (bpr + 7) // 8
    sub_off = (rows * spr * 2 + 63) & ~63
    data_off = (sub_off + rows * bpr + 63) & ~63
    nib = p[data_off:data_off + rows * bpr * 16].reshape(rows, bpr, 16)
    qw = np.empty((rows, bpr, 32), dtype=np.int64)
    qw[:, :, 0::2] = nib & 0xF
    qw[:, :, 1::2] = nib >> 4
    qw = np.where(qw > 7, qw - 16, qw)
    sup = p[:rows * spr * 2].view(np.uint16).reshape(rows, spr).astype(np.uint32)
    supf = np.where((sup & 0x7C00) == 0, 0, ((sup & 0x8000) << 16) | (((sup >> 10) & 0x1F) + 112) << 23
                    | ((sup & 0x3FF) << 13)).astype(np.uint32).view(np.float32)
    u6 = (p[sub_off:sub_off + rows * bpr].reshape(rows, bpr) & 0x3F).astype(np.float32)
    sw = (np.repeat(supf, 8, axis=1)[:, :bpr] * (u6 / np.float32(32))).astype(np.float32)
    qx, sx = o.quantize_vec(x)
    dots = np.einsum("rbi,bi->rb", qw, qx.reshape(bpr, 32).astype(np.int64))
    terms = dots.astype(np.float32) * (sw * sx[None, :]).astype(np.float32)
    y = np.zeros(rows, dtype=np.float32)
    for b in range(bpr):
        y = (y + terms[:, b]).astype(np.float32)
    np.testing.assert_array_equal(o.matvec_w4a8(p, rows, cols, x), y)


# ------------------------------------------------------- dot / rmsnorm ----
def test_dot_lane_order_kat():
    """Mantle's reduction orders differ and the bits show it:
    AVX-512 (ops_avx512.go:27-90) keeps 4 accumulators x 16 lanes over 64-wide
    steps, AVX2 (ops_avx2.go:25-51) 2 x 8 lanes over 16-wide steps, scalar adds in order."""
    b = np.ones(128, dtype=np.float32)
    a = np.zeros(128, dtype=np.float32)
    a[0], a[1], a[64] = 1e8, 1.0, -1e8         # lane 0 of acc0 in both SIMD orders
    assert [o.dot(i, a, b) for i in (0, 1, 2)] == [0.0, 1.0, 1.0]
    a = np.zeros(128, dtype=np.float32)
    a[0], a[1], a[32] = 1e8, 1.0, -1e8         # acc2 lane 0 for AVX-512, acc0 lane 0 for AVX2
    assert [o.dot(i, a, b) for i in (0, 1, 2)] == [0.0, 1.0, 0.0]


@pytest.mark.parametrize("isa", [0, 1, 2])
@pytest.mark.parametrize("n", [5, 128, 1000])
def test_dot_vs_float64(isa, n):
    rng = np.random.default_rng(n)
    a, b = rng.standard_normal((2, n)).astype(np.float32)
    assert abs(o.dot(isa, a, b) - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-4 * math.sqrt(n)


@pytest.mark.parametrize("isa", [0, 1, 2])
def test_rmsnorm_kat_and_float64(isa):
    x = np.full(1024, 2.0, dtype=np.float32)
    w = np.full(1024, 0.5, dtype=np.float32)
    np.testing.assert_array_equal(o.rmsnorm(isa, x, w, 0.0), np.full(1024, 0.5, dtype=np.float32))
    rng = np.random.default_rng(isa)
    for n in (7, 128, 1024, 3000):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = rng.standard_normal(n).astype(np.float32)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
        np.testing.assert_allclose(o.rmsnorm(isa, x, w, 1e-6), want, rtol=2e-6, atol=2e-6)


def test_rmsnorm_lane_order_kat():
    """The three RMSNorm reduction orders give different bits (rmsNormAVX512,
    ops_avx512.go:98-108: 16 FMA lanes over 16-wide steps, lanes added left to
    right; rmsNormSIMD, ops_avx2.go:66-76: 8 lanes; rmsNormScalar, ops.go:73-76:
    one running sum).  x = [4096, 1 x 31]: 4096^2 = 2^24, and 2^24 + 1 rounds
    back to 2^24 (ties to even), so a 1 added straight onto 2^24 is lost while
    ones summed in a lane first survive.  Hand-worked sums of squares:
      scalar  2^24 + 1 + ... + 1, every 1 lost            -> 16777216
      AVX2    lane 0: 2^24 (+1 lost x3); lanes 1-7 hold 4 -> 2^24 + 28
      AVX-512 lane 0: 2^24 (+1 lost);    lanes 1-15 hold 2 -> 2^24 + 30"""
    x = np.ones(32, dtype=np.float32)
    x[0] = 4096.0
    w = np.ones(32, dtype=np.float32)
    sums = {0: 16777216.0, 1: 16777216.0 + 28, 2: 16777216.0 + 30}
    outs = {}
    for isa, ssq in sums.items():
        mean = np.float32(ssq) / np.float32(32)
        scale = np.float32(1.0) / np.float32(math.sqrt(float(np.float32(mean + np.float32(0.0)))))
        want = (x * scale).astype(np.float32) * w
        outs[isa] = o.rmsnorm(isa, x, w, 0.0)
        np.testing.assert_array_equal(outs[isa], want)
    # the orders are distinguishable through the output bits
    assert outs[0][1] != outs[1][1] != outs[2][1] != outs[0][1]


def test_fast_exp_range_reduction_kat():
    """fastExp (ops.go:108-150) takes k = int32(x*ln2Inv + 0.5) (x*ln2Inv - 0.5
    for x < 0, truncated toward zero), fastExpVec (ops_avx2.go:98-128)
    RoundToEven(x*ln2Inv).  At x = 1.7328680 (float32), x*ln2Inv is exactly
    2.5: fastExp takes k = 3 (r = x - 3 ln2 < 0), fastExpVec k = 2 (r > 0),
    and the two approximations differ.  Same at -x with k = -3 / -2.  At
    x*ln2Inv = 3.5 both give k = 4."""
    f = np.float32
    ln2, ln2inv = f(0.693147180559945309417), f(1.44269504088896340736)
    x = f(1.732867956161499)
    assert f(x * ln2inv) == f(2.5)

    def with_k(xv, k, vec):
        r = f(xv - f(f(k) * ln2))
        r2 = f(r * r); r3 = f(r2 * r); r4 = f(r2 * r2); r5 = f(r4 * r)
        poly = f(f(f(f(f(f(1.0) + r) + f(r2 * f(0.5))) + f(r3 * f(0.16666667))) + f(r4 * f(0.041666667)))
                 + f(r5 * f(0.008333333)))
        return float(f(poly * f(2.0 ** k)))

    for sgn in (1, -1):
        xv = f(sgn * x)
        k_trunc, k_even = 3 * sgn, 2 * sgn
        assert o.fast_exp(float(xv)) == with_k(xv, k_trunc, False)
        assert o.fast_exp_vec(float(xv)) == with_k(xv, k_even, True)
        assert o.fast_exp(float(xv)) != o.fast_exp_vec(float(xv))
    x35 = f(3.5 / 1.44269504088896340736)
    while f(x35 * ln2inv) != f(3.5):
        x35 = np.nextafter(x35, f(10), dtype=np.float32)
    assert o.fast_exp(float(x35)) == with_k(x35, 4, False)
    assert o.fast_exp_vec(float(x35)) == with_k(x35, 4, True)


# -------------------------------------------------- exp / softmax / silu ----
def test_fast_exp_kat_and_accuracy():
    assert o.fast_exp(0.0) == 1.0
    assert o.fast_exp(89.0) == np.float32(3.4028235e38)
    assert o.fast_exp(-89.0) == 0.0
    for x in np.linspace(-20, 10, 4001, dtype=np.float32):
        assert abs(o.fast_exp(float(x)) / math.exp(float(x)) - 1) < 1e-3
        assert abs(o.fast_exp_vec(float(x)) / math.exp(float(x)) - 1) < 1e-3


def test_sigmoid_silu_kat():
    """TestSigmoidValues / TestSiluMatchesDefinition (internal/backend/simd/ops_test.go:5-33):
    both the 8-wide (fastSiluVec) and the scalar-tail (Silu) paths."""
    for v, sig in [(0.0, 0.5), (2.0, 0.8807971), (-2.0, 0.1192029)]:
        assert abs(o.fast_silu_vec(v) - v * sig) <= 1e-5 * max(1.0, abs(v))
        tail = o.silu_mul(np.full(9, v, dtype=np.float32), np.ones(9, dtype=np.float32))
        assert abs(tail[8] - v * sig) <= 1e-5 * max(1.0, abs(v))
    g = np.array([-4, -1, 0, 1, 4, -4, -1, 0, 1], dtype=np.float32)
    got = o.silu_mul(g, np.ones_like(g))
    np.testing.assert_allclose(got, g / (1 + np.exp(-g.astype(np.float64))), atol=1e-5)


@pytest.mark.parametrize("n", [1, 6, 160, 5000])
def test_softmax_vs_float64(n):
    """softmaxRef (internal/backend/cuda/native/runtime_test.go:821-845) within 1e-5."""
    x = (np.random.default_rng(n).standard_normal(n) * 4).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(o.softmax(x), e / e.sum(), atol=1e-5, rtol=1e-3)


# -------------------------------------------------------------- RoPE ----
def test_rope_identity_at_pos0_and_float64():
    hd, nh = 128, 3
    x = np.random.default_rng(0).standard_normal(hd * nh).astype(np.float32)
    c, s = o.rope_tables(1e6, hd, 0)
    np.testing.assert_array_equal(o.apply_rope(x, nh, hd, c, s), x)
    pos = 1234
    c, s = o.rope_tables(1e6, hd, pos)
    got = o.apply_rope(x, nh, hd, c, s).reshape(nh, hd)
    inv = 1.0 / (1e6 ** (np.arange(hd // 2) * 2.0 / hd))
    ang = pos * inv
    xr = x.reshape(nh, hd).astype(np.float64)
    lo, hi = xr[:, :hd // 2], xr[:, hd // 2:]
    want = np.concatenate([lo * np.cos(ang) - hi * np.sin(ang), lo * np.sin(ang) + hi * np.cos(ang)], axis=1)
    np.testing.assert_allclose(got, want, atol=1e-5)


# --------------------------------------------------------- attention ----
def _ref_attention(q, ck, cv, pos, kv_stride, hd, nh, kvh, scale, start=0):
    """referenceAttention (internal/backend/simd/attn_test.go:177-236) in float64."""
    out = np.zeros(nh * hd)
    for h in range(nh):
        g = h * kvh // nh
        qh = q[h * hd:(h + 1) * hd].astype(np.float64)
        ks = np.array([ck[t * kv_stride + g * hd: t * kv_stride + (g + 1) * hd] for t in range(start, pos + 1)])
        vs = np.array([cv[t * kv_stride + g * hd: t * kv_stride + (g + 1) * hd] for t in range(start, pos + 1)])
        sc = ks.astype(np.float64) @ qh * scale
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = p @ vs
    return out


def _fill(n, scale):  # fillTestData (internal/backend/simd/attn_test.go:240-244)
    return np.array([scale * np.float32((i % 29) - 14) for i in range(n)], dtype=np.float32)


@pytest.mark.parametrize("isa", [0, 1, 2])
def test_attention_kat_full(isa):
    """TestRunAttnHeadsMatchesReferenceFull (internal/backend/simd/attn_test.go:10-46)."""
    nh, kvh, hd, pos = 4, 2, 8, 5
    kv = kvh * hd
    q, ck, cv = _fill(nh * hd, 0.1), _fill((pos + 1) * kv, 0.2), _fill((pos + 1) * kv, 0.3)
    scale = np.float32(1.0 / math.sqrt(hd))
    got = o.attn_heads(isa, q, ck, cv, pos, kv, hd, nh, kvh, float(scale))
    np.testing.assert_allclose(got, _ref_attention(q, ck, cv, pos, kv, hd, nh, kvh, float(scale)), atol=1e-5)


def test_attention_kat_sliding_window():
    """TestRunAttnHeadsMatchesReferenceSlidingWindow (internal/backend/simd/attn_test.go:48-86)."""
    nh, kvh, hd, pos, window = 6, 3, 8, 9, 4
    start = pos - window + 1
    kv = kvh * hd
    q, ck, cv = _fill(nh * hd, 0.05), _fill((pos + 1) * kv, 0.07), _fill((pos + 1) * kv, 0.09)
    scale = float(np.float32(1.0 / math.sqrt(hd)))
    got = o.attn_heads(2, q, ck, cv, pos, kv, hd, nh, kvh, scale, start)
    np.testing.assert_allclose(got, _ref_attention(q, ck, cv, pos, kv, hd, nh, kvh, scale, start), atol=1e-5)


def test_argmax_first_max():
    x = np.array([1, 3, 3, -1, 3], dtype=np.float32)
    assert o.argmax(x) == 1
    assert o.argmax(np.array([-5.0], dtype=np.float32)) == 0


# ---- bf16 dense GEMV (internal/backend/simd/matvec.go:406-979) ----

@pytest.mark.parametrize("bits_in,bits_out", [(0x3F800000, 0x3F80), (0x3F808000, 0x3F80), (0x3F818000, 0x3F82),
                                              (0x3F808001, 0x3F81), (0xBF7FFFFF, 0xBF80), (0x00000000, 0x0000)])
def test_f32_to_bf16_round_nearest_even_kat(bits_in, bits_out):
    """pkg/mcf/pack.go:789-793: ties go to the even bf16, anything above rounds up."""
    f = np.frombuffer(np.uint32(bits_in).tobytes(), np.float32)[0]
    assert o.lib().mo_f32_to_bf16(float(f)) == bits_out


@pytest.mark.parametrize("cols", [8, 37, 100, 1000, 4104])
def test_bf16_matvec_exact_integer_kat(cols):
    """Small-integer bf16 weights and x in multiples of 1/8: every partial sum is
    exact in fp32, so all three orders must give the integer result."""
    rng = np.random.default_rng(cols)
    wi = rng.integers(-8, 9, size=(9, cols))
    xi = rng.integers(-16, 17, size=cols)
    wb = o.f32_to_bf16(wi.astype(np.float32))
    x = (xi / 8.0).astype(np.float32)
    want = (wi @ xi) / 8.0
    for isa in (o.ISA_SCALAR, o.ISA_AVX2, o.ISA_AVX512):
        np.testing.assert_array_equal(o.bf16_matvec(isa, wb, x), want.astype(np.float32))


def test_bf16_matvec_order_closed_form():
    """One row where the three orders differ, worked by hand from the Go source
    (x = 1): w_0 = 2^24, w_16 = -2^24, w_1..w_15 = 1.
      AVX-512 (32 lane chains, acc + acc_2 per lane): lane 0 holds 2^24 and -2^24 -> 0, lanes 1..15
        hold 1 -> 15.
      AVX2 (8 lane chains): lane 0 takes 2^24 + 1 (rounds to 2^24) - 2^24 = 0, lanes 1..7 take two 1s
        -> 14.
      scalar (8-term groups): 2^24 + 1 + ... stays 2^24, + 8 = 2^24 + 8, + (-2^24 + 0...) -> 8."""
    w = np.zeros((1, 32), np.float32)
    w[0, 0], w[0, 16], w[0, 1:16] = 2.0 ** 24, -2.0 ** 24, 1.0
    wb = o.f32_to_bf16(w)
    x = np.ones(32, np.float32)
    assert float(o.bf16_matvec(o.ISA_AVX512, wb, x)[0]) == 15.0
    assert float(o.bf16_matvec(o.ISA_AVX2, wb, x)[0]) == 14.0
    assert float(o.bf16_matvec(o.ISA_SCALAR, wb, x)[0]) == 8.0


@pytest.mark.parametrize("rows,cols", [(17, 256), (19, 10240)])
def test_bf16_matvec_simd_matches_scalar(rows, cols):
    """TestMatVecBF16MatchesScalar (internal/backend/simd/matvec_bf16_test.go:11-50):
    uniform(-1, 1) bf16 weights and x, every SIMD order within 5e-4 of the scalar
    one; and all within float64 rounding of the exact product."""
    rng = np.random.default_rng(1)
    wb = o.f32_to_bf16(((rng.random((rows, cols)) - 0.5) * 2).astype(np.float32))
    x = ((rng.random(cols) - 0.5) * 2).astype(np.float32)
    scalar = o.bf16_matvec(o.ISA_SCALAR, wb, x)
    exact = (wb.astype(np.uint32) << 16).view(np.float32).astype(np.float64) @ x.astype(np.float64)
    for isa in (o.ISA_AVX2, o.ISA_AVX512):
        assert np.abs(o.bf16_matvec(isa, wb, x) - scalar).max() <= 5e-4
    for isa in (o.ISA_SCALAR, o.ISA_AVX2, o.ISA_AVX512):
        assert np.abs(o.bf16_matvec(isa, wb, x) - exact).max() <= 1e-4 * np.sqrt(cols)


# ---- f16 KV cache (internal/backend/simd/attnpool.go:103-106, :127-135) ----

def _f16_bits(x):
    return np.array([o.f32_to_f16(float(v)) for v in np.ravel(x)], dtype=np.uint16)


def test_attn_f16_is_scalar_attention_on_the_decoded_cache():
    """DotF16 is dotScalarF16 whatever the ISA (ops.go:35-46) and the V sum reads
    Float16ToFloat32 values: over an f16 cache, RunAttnHeads equals the f32
    attention in the scalar order on the decoded values."""
    rng = np.random.default_rng(4)
    nh, kvh, hd, pos = 4, 2, 64, 70
    kv = kvh * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16 = _f16_bits(rng.standard_normal((pos + 1) * kv) * 3)
    v16 = _f16_bits(rng.standard_normal((pos + 1) * kv))
    kf = np.array([o.f16_to_f32(int(b)) for b in k16], np.float32)
    vf = np.array([o.f16_to_f32(int(b)) for b in v16], np.float32)
    got = o.attn_heads_f16(q, k16, v16, pos, kv, hd, nh, kvh, 0.125)
    np.testing.assert_array_equal(got, o.attn_heads(o.ISA_SCALAR, q, kf, vf, pos, kv, hd, nh, kvh, 0.125))


def test_attn_f16_dot_order_closed_form():
    """Worked by hand (hd 128, one head, keys 0 = all ones, 1 = all zeros, V rows
    1 and 0): q_0 = 2^24, q_64 = -2^24, q_1..63 = 1.  The scalar DotF16 of key 0
    loses every +1 against 2^24, then cancels to 0 -> scores equal -> out 0.5.
    (The AVX-512 f32 Dot pairs q_0 with q_64 in one lane and keeps the 63 ones.)"""
    hd = 128
    q = np.zeros(hd, np.float32)
    q[0], q[64], q[1:64] = 2.0 ** 24, -2.0 ** 24, 1.0
    k16 = np.concatenate([np.full(hd, 0x3C00, np.uint16), np.zeros(hd, np.uint16)])
    v16 = np.concatenate([np.full(hd, 0x3C00, np.uint16), np.zeros(hd, np.uint16)])
    got = o.attn_heads_f16(q, k16, v16, 1, hd, hd, 1, 1, 1.0)
    np.testing.assert_array_equal(got, np.full(hd, 0.5, np.float32))
    f32 = o.attn_heads(o.ISA_AVX512, q, np.repeat([1.0, 0.0], hd).astype(np.float32),
                       np.repeat([1.0, 0.0], hd).astype(np.float32), 1, hd, hd, 1, 1, 1.0)
    assert float(f32[0]) > 0.99  # score 63 vs 0


def test_attn_f16_vs_float64():
    """TestRunAttnHeadsMatchesReference's tolerance (attn_test.go:10-86, 1e-5) against
    float64 softmax attention over the f16-decoded cache."""
    rng = np.random.default_rng(5)
    nh, kvh, hd, pos = 8, 2, 128, 300
    kv = kvh * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k16 = _f16_bits(rng.standard_normal((pos + 1) * kv))
    v16 = _f16_bits(rng.standard_normal((pos + 1) * kv))
    kf = np.array([o.f16_to_f32(int(b)) for b in k16]).reshape(pos + 1, kvh, hd)
    vf = np.array([o.f16_to_f32(int(b)) for b in v16]).reshape(pos + 1, kvh, hd)
    got = o.attn_heads_f16(q, k16, v16, pos, kv, hd, nh, kvh, float(1 / np.sqrt(hd)))
    want = np.empty(nh * hd)
    for h in range(nh):
        g = h * kvh // nh
        s = kf[:, g] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        want[h * hd:(h + 1) * hd] = p @ vf[:, g]
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- q8_0 KV cache ----
# internal/backend/simd/ops_runtime.go:132-168 (storeQ8), attnpool.go:100-102, :122-130.

def test_store_q8_kat():
    """Worked by hand.  Row maxAbs 2: scale = 2/127, inv = 63.5, so 1 -> 63.5 + 0.5
    = 64; -0.5 -> -31.75 - 0.5 = -32.25 -> -32 (truncation); 0.25 -> 16.375 -> 16;
    2 -> 127.5 -> 127; -2 -> -127.  Row maxAbs 127 (inv 1): 2.5 -> 3 and -2.5 -> -3
    (half away from zero); 0.49999997 (= 0.5 - 2^-25) + 0.5 is 1 - 2^-25, a tie
    in fp32 that rounds to even 1.0, so it stores 1 where round() would give 0;
    126.5 -> 127; 1.5 -> 2."""
    q, s = o.store_q8(np.array([1.0, -0.5, 0.25, 2.0, -2.0, 0.0], np.float32))
    assert q.tolist() == [64, -32, 16, 127, -127, 0]
    assert np.float32(s) == np.float32(2.0) / np.float32(127.0)
    q, s = o.store_q8(np.array([127.0, 2.5, -2.5, 0.49999997, -0.49999997, 126.5, 1.5], np.float32))
    assert q.tolist() == [127, 3, -3, 1, -1, 127, 2]
    assert s == 1.0


def test_store_q8_zero_and_overflow_rows():
    """A zero row stores scale 0 and zeros (ops_runtime.go:147-153).  A row whose
    maxAbs is below 127 / FLT_MAX makes inv = 127/maxAbs overflow to +Inf: every
    v*inv is +-Inf or NaN (0 * Inf), which Go's float32 -> int32 on amd64
    (CVTTSS2SL) turns into INT32_MIN, clamped to -127 -- for every element."""
    q, s = o.store_q8(np.zeros(32, np.float32))
    assert s == 0.0 and not q.any()
    q, s = o.store_q8(np.array([1e-38, 0.0, -1e-38, 5e-39], np.float32))
    assert q.tolist() == [-127] * 4
    assert np.float32(s) == np.float32(1e-38) / np.float32(127.0)


def test_store_q8_round_trip_bound():
    """|q*scale - x| <= scale/2 (+ an ulp) for every element, and the row's
    largest element maps to +-127."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(1024) * 5).astype(np.float32)
    q, s = o.store_q8(x)
    err = np.abs(q.astype(np.float64) * s - x)
    assert err.max() <= s * 0.5 * (1 + 1e-5)
    assert abs(int(q[np.argmax(np.abs(x))])) == 127


def test_attn_q8_single_key_closed_form():
    """pos 0: the softmax of one score is exactly 1, so out = (1 * q_v) * s_v
    exactly, per head, from kv head h * kv_heads / n_head."""
    nh, kvh, hd = 4, 2, 64
    kv = kvh * hd
    rng = np.random.default_rng(13)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k8 = rng.integers(-127, 128, kv).astype(np.int8)
    v8 = rng.integers(-127, 128, kv).astype(np.int8)
    ks, vs = np.float32([0.03]), np.float32([0.0625])
    got = o.attn_heads_q8(q, k8, v8, ks, vs, 0, kv, hd, nh, kvh, 0.125)
    for h in range(nh):
        g = h * kvh // nh
        np.testing.assert_array_equal(got[h * hd:(h + 1) * hd], v8[g * hd:(g + 1) * hd].astype(np.float32) * vs[0])


def test_attn_q8_dot_order_closed_form():
    """Worked by hand as for DotF16 (hd 128, one head): q_0 = 2^24, q_64 = -2^24,
    q_1..63 = 1; key 0 = all ones (scale 1), key 1 = all zeros; V rows 1 and 0
    (scale 1).  DotQ8's scalar sum loses every +1 against 2^24 and cancels to 0,
    so both scores are 0, p = 0.5 each, out = 0.5."""
    hd = 128
    q = np.zeros(hd, np.float32)
    q[0], q[64], q[1:64] = 2.0 ** 24, -2.0 ** 24, 1.0
    k8 = np.concatenate([np.ones(hd, np.int8), np.zeros(hd, np.int8)])
    v8 = k8.copy()
    one = np.ones(2, np.float32)
    got = o.attn_heads_q8(q, k8, v8, one, one, 1, hd, hd, 1, 1, 1.0)
    np.testing.assert_array_equal(got, np.full(hd, 0.5, np.float32))


def test_attn_q8_vs_float64():
    """attn_test.go:10-86's tolerance (1e-5) against float64 softmax attention over
    the dequantised cache (q * scale per position)."""
    rng = np.random.default_rng(14)
    nh, kvh, hd, pos = 8, 2, 128, 300
    kv = kvh * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k8 = np.empty((pos + 1, kv), np.int8)
    v8 = np.empty((pos + 1, kv), np.int8)
    ks = np.empty(pos + 1, np.float32)
    vs = np.empty(pos + 1, np.float32)
    for t in range(pos + 1):
        k8[t], ks[t] = o.store_q8(rng.standard_normal(kv))
        v8[t], vs[t] = o.store_q8(rng.standard_normal(kv))
    got = o.attn_heads_q8(q, k8, v8, ks, vs, pos, kv, hd, nh, kvh, float(1 / np.sqrt(hd)))
    kf = (k8.astype(np.float64) * ks[:, None]).reshape(pos + 1, kvh, hd)
    vf = (v8.astype(np.float64) * vs[:, None]).reshape(pos + 1, kvh, hd)
    want = np.empty(nh * hd)
    for h in range(nh):
        g = h * kvh // nh
        s = kf[:, g] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        want[h * hd:(h + 1) * hd] = p @ vf[:, g]
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


def test_argmax_strict_greater_kat():
    """argmaxHost (runtime_greedy.go:70-82): best = x[0], replaced only by a
    strictly greater value, so ties keep the first index, -0 ties +0, a later
    NaN never wins and a NaN at index 0 is never replaced."""
    f = np.float32
    assert o.argmax(np.array([1, 3, 3, 2], dtype=f)) == 1
    assert o.argmax(np.array([f(-0.0), f(0.0)], dtype=f)) == 0
    assert o.argmax(np.array([-1, np.nan, 0.5, np.nan], dtype=f)) == 2
    assert o.argmax(np.array([np.nan, 1, 2], dtype=f)) == 0


# ------------------------------------------- mixed K / V caches, ring / window ----
def _mixed_caches(rng, rows, kv):
    kf = (rng.standard_normal(rows * kv) * 2).astype(np.float32)
    vf = rng.standard_normal(rows * kv).astype(np.float32)
    caches = {"f32": (kf, vf, None, None), "f16": (_f16_bits(kf), _f16_bits(vf), None, None)}
    k8 = np.empty(rows * kv, np.int8); v8 = np.empty(rows * kv, np.int8)
    ks = np.empty(rows, np.float32); vs = np.empty(rows, np.float32)
    for t in range(rows):
        k8[t * kv:(t + 1) * kv], ks[t] = o.store_q8(kf[t * kv:(t + 1) * kv])
        v8[t * kv:(t + 1) * kv], vs[t] = o.store_q8(vf[t * kv:(t + 1) * kv])
    caches["q8_0"] = (k8, v8, ks, vs)
    return caches


def _decoded(kind, c, which, kv):
    if kind == "f32":
        return c[0 if which == "k" else 1]
    if kind == "f16":
        return np.array([o.f16_to_f32(int(b)) for b in c[0 if which == "k" else 1]], np.float32)
    raw, sc = (c[0], c[2]) if which == "k" else (c[1], c[3])
    return (raw.astype(np.float64).reshape(-1, kv) * sc[:, None]).reshape(-1)


@pytest.mark.parametrize("kt", ["f32", "f16", "q8_0"])
@pytest.mark.parametrize("vt", ["f32", "f16", "q8_0"])
def test_attn_mixed_matches_single_type_and_float64(kt, vt):
    """RunAttnHeads with K and V caches of independent types (attnpool.go:100-135):
    equal types give exactly the single-type restatements; every pair agrees
    with float64 attention over the decoded caches within 1e-5
    (TestRunAttnHeadsMatchesReference's tolerance, attn_test.go:10-86)."""
    rng = np.random.default_rng(21)
    nh, kvh, hd, pos = 4, 2, 64, 90
    kv = kvh * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    cs = _mixed_caches(rng, pos + 1, kv)
    ck, cv = cs[kt], cs[vt]
    got = o.attn_heads_mixed(2, q, kt, ck[0], ck[2], vt, cv[1], cv[3], pos, 0, 0, kv, hd, nh, kvh, 0.125)
    if kt == vt == "f32":
        np.testing.assert_array_equal(got, o.attn_heads(2, q, ck[0], cv[1], pos, kv, hd, nh, kvh, 0.125))
    elif kt == vt == "f16":
        np.testing.assert_array_equal(got, o.attn_heads_f16(q, ck[0], cv[1], pos, kv, hd, nh, kvh, 0.125))
    elif kt == vt == "q8_0":
        np.testing.assert_array_equal(got, o.attn_heads_q8(q, ck[0], cv[1], ck[2], cv[3], pos, kv, hd, nh, kvh, 0.125))
    kd = _decoded(kt, ck, "k", kv).astype(np.float64).reshape(pos + 1, kvh, hd)
    vd = _decoded(vt, cv, "v", kv).astype(np.float64).reshape(pos + 1, kvh, hd)
    want = np.empty((nh, hd))
    for h in range(nh):
        g = h * kvh // nh
        s = kd[:, g, :] @ q[h * hd:(h + 1) * hd].astype(np.float64) * 0.125
        p = np.exp(s - s.max()); p /= p.sum()
        want[h] = p @ vd[:, g, :]
    np.testing.assert_allclose(got, want.reshape(-1), atol=1e-5, rtol=1e-5)


def test_attn_ring_and_window_placement():
    """RunAttnHeads' ring (attnpool.go:88-99: 0 < cacheLen < pos + 1 puts key t at
    slot t % cacheLen) and window start: a window of the last W keys read from a
    ring of W slots equals the same window read from a linear cache."""
    rng = np.random.default_rng(5)
    nh, kvh, hd, W, pos = 2, 1, 64, 16, 40
    kv = kvh * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    lin_k = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    lin_v = rng.standard_normal((pos + 1) * kv).astype(np.float32)
    ring_k = np.zeros(W * kv, np.float32); ring_v = np.zeros(W * kv, np.float32)
    for t in range(pos + 1):  # StoreKV at cachePos = t % cacheLen (ops_runtime.go:51-55)
        ring_k[(t % W) * kv:(t % W + 1) * kv] = lin_k[t * kv:(t + 1) * kv]
        ring_v[(t % W) * kv:(t % W + 1) * kv] = lin_v[t * kv:(t + 1) * kv]
    start = pos - W + 1
    a = o.attn_heads_mixed(2, q, "f32", ring_k, None, "f32", ring_v, None, pos, start, W, kv, hd, nh, kvh, 0.125)
    b = o.attn_heads(2, q, lin_k, lin_v, pos, kv, hd, nh, kvh, 0.125, start=start)
    np.testing.assert_array_equal(a, b)
