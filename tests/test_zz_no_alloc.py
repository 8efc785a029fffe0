"""The allocation-free W4A8 GEMV entry point (mantleHipQuantMatVecK4W4A8F32NoAlloc)
against the scratch-taking one it mirrors: bit-identical outputs on two calls in
a row, the second with a smaller input (the library array keeps the first
call's contents), and the size limit rejected before any launch."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402


def _payload(rows, cols, seed):
    from mantle_amd import mcf
    w = mcf.fill_normal(rows * cols, seed).reshape(rows, cols)
    p = mcf.quantize_k4(w.astype(np.float32))
    return mcf.k4_regions(p, rows, cols)


def _both(rows, cols, batch, seed):
    sup, sub, nib = _payload(rows, cols, seed)
    x = np.random.default_rng(seed).standard_normal(batch * cols).astype(np.float32)
    bpr = (cols + 31) // 32
    dn, dsup, dsub, dx = g.keep(nib), g.keep(sup), g.keep(sub), g.keep(x)
    y0 = g.empty(batch * rows)
    y1 = g.empty(batch * rows)
    qx = g.empty(batch * bpr * 32, torch.int8)
    xs = g.empty(batch * bpr)
    g.call("mantleHipQuantMatVecK4W4A8F32", g.ptr(dn), g.ptr(dsup), g.ptr(dsub), g.ptr(dx), g.ptr(y0), rows, bpr, cols,
           batch, g.ptr(qx), g.ptr(xs), g.stream())
    g.call("mantleHipQuantMatVecK4W4A8F32NoAlloc", g.ptr(dn), g.ptr(dsup), g.ptr(dsub), g.ptr(dx), g.ptr(y1), rows,
           bpr, cols, batch, g.stream())
    return g.host(y0), g.host(y1)


def test_no_alloc_gemv_matches_scratch_entry(hip):
    for rows, cols, batch, seed in [(3072, 12288, 8, 1), (1000, 1024, 1, 2)]:  # the second call is smaller
        want, got = _both(rows, cols, batch, seed)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"{rows}x{cols} b{batch}")


def test_no_alloc_gemv_rejects_oversize(hip):
    from mantle_amd import _lib
    L = _lib.lib()
    f = ctypes.c_void_p(0x1000)
    assert L.mantleHipQuantMatVecK4W4A8F32NoAlloc(f, f, f, f, f, 4, 385, 12320, 1, None) == 1  # > 12288 columns
    assert L.mantleHipQuantMatVecK4W4A8F32NoAlloc(f, f, f, f, f, 4, 32, 1024, 9, None) == 1  # batch > 8
