"""Raw-bf16 weights on the GPU vs the CPU oracle: the bf16 GEMV
(internal/backend/simd/matvec.go:406-979, fp32 activations) bit-exact in each
of Mantle's three reduction orders, and whole greedy decode steps of bf16
models bit-identical (logits and residual stream)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import gpu_util as g  # noqa: E402
from tests import models  # noqa: E402

ISAS = [2, 1, 0]


def _bf16(oracle, rows, cols, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_bf16(((rng.random((rows, cols)) - 0.5) * 2 * scale).astype(np.float32))


# (17, 256) and (19, 10240) are TestMatVecBF16MatchesScalar's shapes
# (internal/backend/simd/matvec_bf16_test.go:17-24); 1000 / 1016 columns leave a
# 16-element and an 8-element remainder after the 32-element steps; the rest
# are Qwen3-8B rows (4096, 12288 columns).
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("rows,cols", [(17, 256), (19, 10240), (5, 1000), (33, 1016), (1024, 4096), (300, 12288)])
def test_bf16_gemv_bitexact(hip, oracle, isa, rows, cols):
    w = _bf16(oracle, rows, cols, rows * 7 + cols)
    x = ((np.random.default_rng(cols).random(cols) - 0.5) * 2).astype(np.float32)
    y = g.empty(rows)
    g.call("mantleHipSetParityISA", isa)
    try:
        g.call("mantleHipMatVecBF16F32", g.ptr(g.keep(w)), g.ptr(g.keep(x)), g.ptr(y), rows, cols, g.stream())
        got = g.host(y)
    finally:
        g.call("mantleHipSetParityISA", 2)
    g.assert_bitexact(got, oracle.bf16_matvec(isa, w, x), f"bf16 gemv isa {isa}")


def test_bf16_gemv_order_closed_form(hip, oracle):
    """The hand-worked row of the oracle test: 15 / 14 / 8 for AVX-512 / AVX2 / scalar."""
    w = np.zeros((1, 32), np.float32)
    w[0, 0], w[0, 16], w[0, 1:16] = 2.0 ** 24, -2.0 ** 24, 1.0
    wb = oracle.f32_to_bf16(w)
    x = np.ones(32, np.float32)
    for isa, want in ((2, 15.0), (1, 14.0), (0, 8.0)):
        y = g.empty(1)
        g.call("mantleHipSetParityISA", isa)
        g.call("mantleHipMatVecBF16F32", g.ptr(g.keep(wb)), g.ptr(g.keep(x)), g.ptr(y), 1, 32, g.stream())
        assert float(g.host(y)[0]) == want, isa
    g.call("mantleHipSetParityISA", 2)


def test_bf16_gemv_rejects_bad_shapes(hip):
    from mantle_amd import _lib
    L = _lib.lib()
    z = g.empty(64)
    p = g.ptr(z)
    assert L.mantleHipMatVecBF16F32(p, p, p, 4, 12, None) != 0    # cols % 8
    assert L.mantleHipMatVecBF16F32(p, p, p, 0, 16, None) != 0    # no rows
    assert L.mantleHipMatVecBF16F32(None, p, p, 4, 16, None) != 0
    assert L.mantleHipMatVecBF16F32(p + 2, p, p, 4, 16, None) != 0  # unaligned weights


@pytest.mark.parametrize("isa", ["avx512", "avx2", "scalar"])
@pytest.mark.parametrize("shape", ["tiny", "wide4b"])
def test_bf16_model_logits_bitexact(hip, tmp_models, shape, isa):
    """Greedy steps of bf16-weight models: logits and residual stream bit-identical
    to the oracle's; "wide4b" has Qwen3-4B's row widths (2560 / 4096 / 9728) and a
    20000-row lm_head."""
    import mantle_amd
    isa_id = {"avx512": 2, "avx2": 1, "scalar": 0}[isa]
    cfg = dict(models.TINY if shape == "tiny" else models.WIDE4B, weights="bf16")
    if shape == "wide4b" and isa != "avx512":
        pytest.skip("the wide model runs in Mantle's default order only (CPU oracle time)")
    path = models.pack(str(tmp_models / f"{shape}_bf16.mcf"), 11, cfg)
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=48, parity_isa=isa)
    om = models.oracle_model(path, cfg, 48, isa_id)
    steps = 20 if shape == "tiny" else 4
    try:
        tok = 3
        for step in range(steps):
            logits = rt.forward_token(tok)
            nxt, want = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
            np.testing.assert_array_equal(rt.hidden().view(np.uint32), om.hidden().view(np.uint32))
            assert int(np.argmax(logits)) == nxt
            tok = nxt
    finally:
        rt.close()
        om.close()


def test_bf16_model_greedy_tokens_graph(hip, tmp_models):
    """generate_greedy (captured step graph, device-side argmax) equals the oracle's tokens."""
    import mantle_amd
    cfg = dict(models.LANE, weights="bf16")
    path = models.pack(str(tmp_models / "lane_bf16.mcf"), 12, cfg)
    p = models.prompt(9, cfg["vocab"], 2)
    rt = mantle_amd.new_backend().load_model(path, max_context=64)
    try:
        got = rt.generate_greedy(p, 32)
    finally:
        rt.close()
    om = models.oracle_model(path, cfg, 64)
    try:
        want = om.generate_greedy(p, 32)
    finally:
        om.close()
    assert got == want
