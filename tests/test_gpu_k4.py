"""GPU parity of the k4 kernels against the CPU oracle (bit-exact where the
reference arithmetic is integer / exact, tolerance for W4A32)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402

SHAPES = [(2, 96), (37, 100), (64, 1000), (3072, 1024), (1024, 3072), (2048, 1024), (151936, 1024),
          # Qwen3-4B / 8B row widths: 80, 128, 304 (pieced) and 384 (pieced) blocks; 20000 rows: large launch
          (6144, 2560), (2560, 4096), (2560, 9728), (20000, 2560), (4096, 12288), (20000, 4096)]


def _weights(rows, cols, seed):
    from mantle_amd import mcf
    return mcf.fill_normal(rows * cols, seed).reshape(rows, cols)


def _random_payload(rows, cols, seed):
    """Arbitrary bytes in every region: nibble -8, u6 = 0, super = 0 / subnormal / large."""
    from oracle import oracle as o
    rng = np.random.default_rng(seed)
    p = rng.integers(0, 256, size=o.payload_size(rows, cols), dtype=np.uint8)
    bpr = (cols + 31) // 32
    spr = (bpr + 7) // 8
    sup = p[: rows * spr * 2].view(np.uint16)
    choices = np.array([0x0000, 0x0001, 0x03FF, 0x2E66, 0x3C00, 0x1400, 0x0800], dtype=np.uint16)
    sup[:] = choices[rng.integers(0, len(choices), size=sup.size)]
    return p


@pytest.fixture(scope="module")
def ws():
    torch.cuda.init()
    return {}


def test_device_present(hip):
    import ctypes
    n = ctypes.c_int()
    g.call("mantleHipGetDeviceCount", ctypes.byref(n))
    assert n.value >= 1


def test_dequant_kat(hip, oracle):
    """TestDequantizeK4ToF16 (internal/backend/cuda/native/runtime_test.go:612-706):
    unit super/sub scales, q = (i+b)%13-6 => w == q exactly."""
    rows, cols = 2, 64
    bpr = 2
    q = np.array([[(i + b) % 13 - 6 for i in range(32)] for b in range(rows * bpr)], dtype=np.int8)
    payload = np.zeros(oracle.payload_size(rows, cols), dtype=np.uint8)
    sup = payload[:rows * 2].view(np.uint16)
    sup[:] = 0x3C00
    sub_off = 64
    payload[sub_off:sub_off + rows * bpr] = 32
    data_off = 128
    nib = (q.astype(np.int16) & 0xF).astype(np.uint8)
    payload[data_off:data_off + rows * bpr * 16] = (nib[:, 0::2] | (nib[:, 1::2] << 4)).reshape(-1)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    o16 = g.empty(rows * cols, torch.float16)
    o32 = g.empty(rows * cols)
    g.call("mantleHipDequantizeK4ToF16", qn, qs, qsub, g.ptr(o16), rows, bpr, cols, g.stream())
    g.call("mantleHipDequantizeK4ToF32", qn, qs, qsub, g.ptr(o32), rows, bpr, cols, g.stream())
    want = q.reshape(rows, cols).astype(np.float32)
    np.testing.assert_array_equal(g.host(o16).astype(np.float32).reshape(rows, cols), want)
    np.testing.assert_array_equal(g.host(o32).reshape(rows, cols), want)
    np.testing.assert_array_equal(oracle.dequant_k4(payload, rows, cols), want)


@pytest.mark.parametrize("rows,cols", [(37, 100), (64, 1000), (1024, 3072)])
@pytest.mark.parametrize("kind", ["packed", "random_bytes"])
def test_dequant_bitexact(hip, oracle, rows, cols, kind):
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 11)) if kind == "packed" else _random_payload(rows, cols, 5)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    out = g.empty(rows * cols)
    g.call("mantleHipDequantizeK4ToF32", qn, qs, qsub, g.ptr(out), rows, (cols + 31) // 32, cols, g.stream())
    g.assert_bitexact(g.host(out).reshape(rows, cols), oracle.dequant_k4(payload, rows, cols), f"dequant {kind}")


@pytest.mark.parametrize("n", [1, 31, 32, 100, 1024, 3072])
def test_quantize_vec_bitexact(hip, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if n >= 64:
        x[32:64] = 0.0                      # zero block -> scale 0
        x[0:4] = [2.5 / 127 * 127, -1.0, 0.5, -0.5]
    xd = g.dev(x)
    blocks = (n + 31) // 32
    qx = g.empty(blocks * 32, torch.int8)
    xs = g.empty(blocks)
    g.call("mantleHipQuantizeVecBlocksF32", g.ptr(xd), n, g.ptr(qx), g.ptr(xs), g.stream())
    wq, ws = oracle.quantize_vec(x)
    np.testing.assert_array_equal(g.unpermute_qx(g.host(qx)), wq)
    g.assert_bitexact(g.host(xs), ws, "xscales")


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("batch", [1, 8])
def test_w4a8_gemv_bitexact(hip, oracle, rows, cols, batch):
    """The parity GEMV reproduces Mantle's CPU W4A8 arithmetic bit for bit."""
    from mantle_amd import mcf
    print(f"w4a8 {rows}x{cols} B={batch}", flush=True)
    payload = mcf.quantize_k4(_weights(rows, cols, 2))
    x = mcf.fill_normal(batch * cols, 1000 + rows, 1.0).reshape(batch, cols)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    bpr = (cols + 31) // 32
    xd = g.dev(x)
    y = g.empty(batch * rows)
    qx = g.empty(batch * bpr * 32, torch.int8)
    xs = g.empty(batch * bpr)
    g.call("mantleHipQuantMatVecK4W4A8F32", qn, qs, qsub, g.ptr(xd), g.ptr(y), rows, bpr, cols, batch, g.ptr(qx),
           g.ptr(xs), g.stream())
    got = g.host(y).reshape(batch, rows)
    oracle.set_threads(8)
    for b in range(batch):
        g.assert_bitexact(got[b], oracle.matvec_w4a8(payload, rows, cols, x[b]), f"w4a8 {rows}x{cols} b={b}")


@pytest.mark.parametrize("rows,cols", [(37, 100), (64, 1000), (2048, 1024)])
def test_w4a8_gemv_random_bytes(hip, oracle, rows, cols):
    """Arbitrary payload bytes (nibble -8, zero/subnormal super, u6 = 0) stay bit-exact."""
    payload = _random_payload(rows, cols, rows)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    bpr = (cols + 31) // 32
    y = g.empty(rows)
    qx = g.empty(bpr * 32, torch.int8)
    xs = g.empty(bpr)
    g.call("mantleHipQuantMatVecK4W4A8F32", qn, qs, qsub, g.ptr(g.keep(x)), g.ptr(y), rows, bpr, cols, 1, g.ptr(qx),
           g.ptr(xs), g.stream())
    g.assert_bitexact(g.host(y), oracle.matvec_w4a8(payload, rows, cols, x), "w4a8 random bytes")


def test_w4a32_gemv_kat(hip):
    """TestQuantMatVecK4F32 (internal/backend/cuda/native/runtime_test.go:425-527)."""
    rows, cols, bpr = 2, 96, 3
    q = np.array([[(i + b) % 13 - 6 for i in range(32)] for b in range(rows * bpr)], dtype=np.int8)
    from oracle import oracle as o
    payload = np.zeros(o.payload_size(rows, cols), dtype=np.uint8)
    payload[:rows * 2].view(np.uint16)[:] = 0x3C00
    payload[64:64 + rows * bpr] = 32
    nib = (q.astype(np.int16) & 0xF).astype(np.uint8)
    payload[128:128 + rows * bpr * 16] = (nib[:, 0::2] | (nib[:, 1::2] << 4)).reshape(-1)
    x = np.array([((i % 17) - 8) * 0.125 for i in range(cols)], dtype=np.float32)
    want = (q.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    y = g.empty(rows)
    g.call("mantleHipQuantMatVecK4F32", qn, qs, qsub, g.ptr(g.keep(x)), g.ptr(y), rows, bpr, cols, g.stream())
    np.testing.assert_allclose(g.host(y), want, atol=1e-4, rtol=0)
    np.testing.assert_allclose(o.matvec_w4a32(payload, rows, cols, x), want, atol=1e-4, rtol=0)


@pytest.mark.parametrize("rows,cols", [(3072, 1024), (1024, 3072), (2048, 1024), (151936, 1024), (70001, 1024), (1001, 3072)])
def test_w4a32_gemv_tolerance(hip, oracle, rows, cols):
    """W4A32 (fp32 activations): within max-abs 1e-3 / rel 1e-2 of the oracle."""
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 2))
    x = mcf.fill_normal(cols, 77, 1.0)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    y = g.empty(rows)
    g.call("mantleHipQuantMatVecK4F32", qn, qs, qsub, g.ptr(g.keep(x)), g.ptr(y), rows, (cols + 31) // 32, cols,
           g.stream())
    oracle.set_threads(8)
    want = oracle.matvec_w4a32(payload, rows, cols, x)
    got = g.host(y)
    err = np.abs(got - want)
    assert np.all((err <= 1e-3) | (err <= 1e-2 * np.abs(want))), float(err.max())


@pytest.mark.parametrize("rows,cols", [(3072, 1024), (1024, 3072), (2048, 1024), (151936, 1024)])
def test_w4a32_gemv_batch8(hip, oracle, rows, cols):
    """Batched W4A32 (config 2 at B = 8, fp32 activations, on f16 matrix cores with
    x in two f16 parts): each column within max-abs 1e-3 / rel 1e-2 of the oracle,
    as is its own batch-1 launch (the lane kernel)."""
    from mantle_amd import mcf
    payload = mcf.quantize_k4(_weights(rows, cols, 2))
    B, bpr = 8, (cols + 31) // 32
    x = mcf.fill_normal(B * cols, 78, 1.0)
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    dx = g.keep(x)
    y = g.empty(B * rows)
    g.call("mantleHipQuantMatVecK4F32Batched", qn, qs, qsub, g.ptr(dx), g.ptr(y), rows, bpr, cols, B, g.stream())
    got = g.host(y).reshape(B, rows)
    oracle.set_threads(8)
    for b in range(B):
        want = oracle.matvec_w4a32(payload, rows, cols, x[b * cols:(b + 1) * cols])
        err = np.abs(got[b] - want)
        assert np.all((err <= 1e-3) | (err <= 1e-2 * np.abs(want))), (b, float(err.max()))
    for b in (0, 7):
        y1 = g.empty(rows)
        g.call("mantleHipQuantMatVecK4F32Batched", qn, qs, qsub, g.ptr(dx) + 4 * b * cols, g.ptr(y1), rows, bpr, cols,
               1, g.stream())
        err = np.abs(g.host(y1) - got[b])
        assert np.all((err <= 1e-3) | (err <= 1e-2 * np.abs(got[b]))), (b, float(err.max()))


@pytest.mark.parametrize("batch", [2, 3, 5, 8])
@pytest.mark.parametrize("scale", [1.0, 1e5, 1e-6])
def test_w4a32_gemv_batches_range(hip, oracle, batch, scale):
    """Batches 2..8 and activations far outside fp16's range (the per-vector
    power-of-two factor): within max-abs 1e-3 * scale / rel 1e-2 of the oracle."""
    from mantle_amd import mcf
    rows, cols = 1000, 2048
    payload = mcf.quantize_k4(_weights(rows, cols, 6))
    bpr = cols // 32
    x = (np.random.default_rng(batch).standard_normal((batch, cols)) * scale).astype(np.float32)
    x[0, 100:200] *= 1e-3  # small values beside large ones in one vector
    keep, qn, qs, qsub = g.k4_dev(payload, rows, cols)
    y = g.empty(batch * rows)
    g.call("mantleHipQuantMatVecK4F32Batched", qn, qs, qsub, g.ptr(g.keep(x)), g.ptr(y), rows, bpr, cols, batch,
           g.stream())
    got = g.host(y).reshape(batch, rows)
    for b in range(batch):
        want = oracle.matvec_w4a32(payload, rows, cols, x[b])
        err = np.abs(got[b] - want)
        assert np.all((err <= 1e-3 * scale) | (err <= 1e-2 * np.abs(want))), (b, float(err.max()))
