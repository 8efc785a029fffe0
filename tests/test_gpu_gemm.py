"""GPU parity of the int8-MFMA W4A8 product over many activation rows
(mantleHipQuantMatMulK4W4A8F32): every row bit-identical to the CPU W4A8
arithmetic (oracle matvec_w4a8) and to the batch GEMV entry."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402
from tests.test_gpu_k4 import _random_payload, _weights  # noqa: E402


def _matmul(payload, rows, cols, x):
    n = x.shape[0]
    bpr = cols // 32
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    xd = g.dev(x)
    y = g.empty(n * rows)
    qx = g.empty(n * cols, torch.int8)
    xs = g.empty(n * bpr)
    g.call("mantleHipQuantMatMulK4W4A8F32", qn, qs, qsub, g.ptr(xd), g.ptr(y), rows, bpr, cols, n, g.ptr(qx),
           g.ptr(xs), g.stream())
    return g.host(y).reshape(n, rows), (keep, qn, qs, qsub, xd)


@pytest.mark.parametrize("rows,cols,n", [(16, 256, 1), (37, 256, 3), (64, 1024, 8), (100, 1024, 17),
                                         (3072, 1024, 64), (1024, 3072, 33), (2048, 1024, 130), (2560, 9728, 9),
                                         (300, 4096, 8), (64, 8192, 4), (70, 3072, 2)])
def test_w4a8_matmul_bitexact(hip, oracle, rows, cols, n):
    from mantle_amd import mcf
    print(f"matmul {rows}x{cols} n={n}", flush=True)
    payload = mcf.quantize_k4(_weights(rows, cols, 4))
    x = mcf.fill_normal(n * cols, 500 + n, 1.0).reshape(n, cols)
    x[0, 32:64] = 0.0          # a zero block: scale 0, skipped
    if n > 2:
        x[2, :] = 0.0          # an all-zero row
    got, _ = _matmul(payload, rows, cols, x)
    oracle.set_threads(8)
    for v in range(n):
        g.assert_bitexact(got[v], oracle.matvec_w4a8(payload, rows, cols, x[v]), f"matmul {rows}x{cols} v={v}")


@pytest.mark.parametrize("rows,cols,n", [(37, 256, 5), (2048, 1024, 20)])
def test_w4a8_matmul_random_bytes(hip, oracle, rows, cols, n):
    """Arbitrary payload bytes (nibble -8, zero/subnormal super, u6 = 0)."""
    payload = _random_payload(rows, cols, rows + n)
    x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    got, _ = _matmul(payload, rows, cols, x)
    for v in range(n):
        g.assert_bitexact(got[v], oracle.matvec_w4a8(payload, rows, cols, x[v]), f"random bytes v={v}")


@pytest.mark.parametrize("rows,cols", [(151936, 1024), (3072, 1024)])
def test_w4a8_matmul_matches_gemv(hip, rows, cols):
    """At batch 8 the matrix-core product equals the lane GEMV's, bit for bit."""
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 2))
    n, bpr = 8, cols // 32
    x = mcf.fill_normal(n * cols, 91, 1.0).reshape(n, cols)
    got, (keep, qn, qs, qsub, xd) = _matmul(payload, rows, cols, x)
    y = g.empty(n * rows)
    qx = g.empty(n * cols, torch.int8)
    xs = g.empty(n * bpr)
    g.call("mantleHipQuantMatVecK4W4A8F32", qn, qs, qsub, g.ptr(xd), g.ptr(y), rows, bpr, cols, n, g.ptr(qx),
           g.ptr(xs), g.stream())
    np.testing.assert_array_equal(got.view(np.uint32), g.host(y).reshape(n, rows).view(np.uint32))


def test_w4a8_matmul_rejects(hip):
    """blocksPerRow not a multiple of 8, n < 1: invalid value, nothing launched."""
    from mantle_amd import _lib
    f = _lib.lib().mantleHipQuantMatMulK4W4A8F32
    p = 256
    assert f(p, p, p, p, p, 4, 3, 96, 1, p, p, 0) != 0
    assert f(p, p, p, p, p, 4, 8, 256, 0, p, p, 0) != 0


@pytest.mark.parametrize("n", [3, 24])
def test_w4a8_matmul_nonfinite_scales(hip, oracle, n):
    """Infinite / NaN super scales next to zero activation blocks: a chunk with a
    scale that is not finite takes the skip test (a zero scale skips the block,
    as the CPU loop does); NaN where the oracle has NaN, every other value bit-exact."""
    rows, cols = 96, 512
    payload = _random_payload(rows, cols, 7 + n)
    bpr = cols // 32
    spr = (bpr + 7) // 8
    sup = payload[: rows * spr * 2].view(np.uint16)
    sup[::5] = 0x7C00        # +inf
    sup[1::7] = 0xFC00       # -inf
    sup[2::11] = 0x7E00      # NaN
    x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    x[:, 0:32] = 0.0         # block 0 of every vector: scale 0 against the inf supers
    x[0, 96:160] = 0.0
    got, _ = _matmul(payload, rows, cols, x)
    for v in range(n):
        want = oracle.matvec_w4a8(payload, rows, cols, x[v])
        np.testing.assert_array_equal(np.isnan(got[v]), np.isnan(want))
        ok = ~np.isnan(want)
        g.assert_bitexact(got[v][ok], want[ok], f"nonfinite v={v}")


def _extreme_x(n, cols, seed):
    """Activation rows whose block scales (max|x| / 127) fall below 2^-100 and
    above 2^100 in some blocks, beside ordinary ones."""
    x = np.random.default_rng(seed).standard_normal((n, cols)).astype(np.float32)
    x[:, 32:64] *= np.float32(1e-33)    # scale ~1e-35: the matrix-core kernels' exact fallback
    x[:, 96:128] *= np.float32(3e32)    # scale ~1e31
    x[0, 160:192] *= np.float32(1e-38)  # subnormal activations
    x[-1, 192:224] = np.float32(3e38)   # scale near the fp32 maximum
    return x


@pytest.mark.parametrize("n", [3, 24])
def test_w4a8_matmul_extreme_activation_scales(hip, oracle, n):
    """Activation block scales outside [2^-100, 2^100] send a chunk to the exact
    form of the term (the fast form takes the block dot against s_w / 16):
    still bit-identical to the CPU arithmetic, infinities and NaN included."""
    rows, cols = 80, 512
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 9))
    x = _extreme_x(n, cols, 40 + n)
    got, _ = _matmul(payload, rows, cols, x)
    for v in range(n):
        want = oracle.matvec_w4a8(payload, rows, cols, x[v])
        np.testing.assert_array_equal(np.isnan(got[v]), np.isnan(want))
        ok = ~np.isnan(want)
        g.assert_bitexact(got[v][ok], want[ok], f"extreme scales v={v}")


def test_w4a8_gemv8_extreme_activation_scales(hip, oracle):
    """The same at batch 8 on a tall matrix (the matrix-core pair-form GEMV)."""
    rows, cols, batch = 16384, 1024, 8
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 10))
    x = _extreme_x(batch, cols, 77)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    bpr = cols // 32
    xd = g.dev(x)
    y = g.empty(batch * rows)
    qx = g.empty(batch * cols, torch.int8)
    xs = g.empty(batch * bpr)
    g.call("mantleHipQuantMatVecK4W4A8F32", qn, qs, qsub, g.ptr(xd), g.ptr(y), rows, bpr, cols, batch, g.ptr(qx),
           g.ptr(xs), g.stream())
    got = g.host(y).reshape(batch, rows)
    oracle.set_threads(8)
    for b in range(batch):
        want = oracle.matvec_w4a8(payload, rows, cols, x[b])
        np.testing.assert_array_equal(np.isnan(got[b]), np.isnan(want))
        ok = ~np.isnan(want)
        g.assert_bitexact(got[b][ok], want[ok], f"gemv8 extreme scales b={b}")
