"""End-to-end greedy decode on the GPU vs the CPU oracle: identical tokens,
bit-identical logits and residual stream."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import models  # noqa: E402


@pytest.fixture(scope="module")
def tiny_path(tmp_models):
    return models.pack(str(tmp_models / "tiny.mcf"), 0, models.TINY)


@pytest.fixture(scope="module")
def lane_path(tmp_models):
    return models.pack(str(tmp_models / "lane.mcf"), 3, models.LANE)


@pytest.mark.parametrize("isa", ["avx512", "avx2", "scalar"])
@pytest.mark.parametrize("shape", ["tiny", "lane"])
def test_greedy_logits_bitexact(hip, tiny_path, lane_path, shape, isa):
    """Every step's logits and residual stream bit-identical to the oracle in
    each of Mantle's three reduction orders; "tiny" runs the tile GEMV, "lane"
    (1024-wide rows) the lane-chain GEMV with its fused RMSNorm prologue."""
    import mantle_amd
    isa_id = {"avx512": 2, "avx2": 1, "scalar": 0}[isa]
    path, cfg = (tiny_path, models.TINY) if shape == "tiny" else (lane_path, models.LANE)
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=96, parity_isa=isa)
    om = models.oracle_model(path, cfg, 96, isa_id)
    steps = 40 if shape == "tiny" else 12
    try:
        tok = 17
        for step in range(steps):
            logits = rt.forward_token(tok)
            nxt, want = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
            np.testing.assert_array_equal(rt.hidden().view(np.uint32), om.hidden().view(np.uint32))
            assert int(np.argmax(logits)) == nxt
            tok = nxt
        assert rt.pos == steps
    finally:
        rt.close()
        om.close()


@pytest.mark.parametrize("shape", ["wide4b", "wide8b"])
def test_wide_rows_logits_bitexact(hip, tmp_models, shape):
    """Qwen3-4B / 8B row widths: 80/128-block rows whole, 304/384-block rows
    (the down projections) in double-buffered pieces, 20000 logits rows on the
    large-matrix launch -- logits and residual stream bit-identical per step."""
    import mantle_amd
    cfg = models.WIDE4B if shape == "wide4b" else models.WIDE8B
    path = models.pack(str(tmp_models / f"{shape}.mcf"), 7, cfg)
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=32)
    om = models.oracle_model(path, cfg, 32)
    try:
        tok = 5
        for step in range(6):
            logits = rt.forward_token(tok)
            nxt, want = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
            np.testing.assert_array_equal(rt.hidden().view(np.uint32), om.hidden().view(np.uint32))
            tok = nxt
    finally:
        rt.close()
        om.close()


@pytest.mark.parametrize("path", ["split", "fused"])
def test_lane_f16_kv_cache_bitexact(hip, lane_path, path):
    """`mantle run`'s default --cache-type-k/v f16 (cmd/mantle/run.go:183-195): 100
    fused steps with the f16 cache (transposed V) on both split paths, logits
    bit-identical to the oracle's f16-cache decode."""
    import mantle_amd
    from mantle_amd import _lib
    _lib.call("mantleHipSetAttentionPath", {"split": 0, "fused": 3}[path])
    try:
        rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=128, kv_cache="f16")
        cfg = dict(models.LANE, kv_cache="f16")
        om = models.oracle_model(lane_path, cfg, 128)
        toks = models.prompt(100, models.LANE["vocab"], 6)
        for step, tok in enumerate(toks):
            logits = rt.forward_token(tok)
            _, want = om.forward_greedy(tok, want_logits=True)
            if step % 10 == 9 or step < 3:
                np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
        rt.close()
        om.close()
    finally:
        _lib.call("mantleHipSetAttentionPath", 0)


@pytest.mark.parametrize("path", ["split", "fused"])
def test_lane_q8_kv_cache_bitexact(hip, lane_path, path):
    """--cache-type-k/v q8_0 (loader.go:645-663): 400 steps (the transposed int8
    V ring wraps past 320 keys; 420 positions pad to 432 per column), logits
    bit-identical to the oracle's q8_0-cache decode on both split settings
    (both take the two-launch form with a separate append)."""
    import mantle_amd
    from mantle_amd import _lib
    _lib.call("mantleHipSetAttentionPath", {"split": 0, "fused": 3}[path])
    try:
        rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=420, kv_cache="q8_0")
        om = models.oracle_model(lane_path, dict(models.LANE, kv_cache="q8_0"), 420)
        toks = models.prompt(400, models.LANE["vocab"], 8)
        for step, tok in enumerate(toks):
            logits = rt.forward_token(tok)
            _, want = om.forward_greedy(tok, want_logits=True)
            if step % 25 == 24 or step < 3 or step == len(toks) - 1:
                np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
        rt.close()
        om.close()
    finally:
        _lib.call("mantleHipSetAttentionPath", 0)


@pytest.mark.parametrize("kv,pv_lds", [("f32", "1"), ("f32", "0"), ("f16", "1"), ("q8_0", "1")])
def test_lane_v_sum_staged_in_lds(hip, lane_path, kv, pv_lds, monkeypatch):
    """The V sum with V staged in LDS by loader waves (widened there: f16
    through the flushing conversion, int8 exactly), chunks of 256 keys (600
    steps: three chunks, the last partial; 650 positions pad the columns), and
    the register-ring form (MANTLE_HIP_PV_LDS=0): logits bit-identical to the
    oracle for each cache type."""
    import mantle_amd
    monkeypatch.setenv("MANTLE_HIP_PV_LDS", pv_lds)
    rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=650, kv_cache=kv)
    om = models.oracle_model(lane_path, dict(models.LANE, kv_cache=kv), 650)
    try:
        toks = models.prompt(600, models.LANE["vocab"], 10)
        for step, tok in enumerate(toks):
            logits = rt.forward_token(tok)
            _, want = om.forward_greedy(tok, want_logits=True)
            if step % 50 == 49 or step in (0, 255, 256, 257, 511, 512, 599):
                np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
    finally:
        rt.close()
        om.close()


@pytest.mark.parametrize("path", ["fused", "split", "single", "general"])
def test_lane_long_context_attention_paths(hip, lane_path, path):
    """140 fused steps (past two 64-key chunks, the step's own K/V row inside
    a later chunk) on each attention variant: logits bit-identical to the oracle."""
    import mantle_amd
    from mantle_amd import _lib
    _lib.call("mantleHipSetAttentionPath", {"split": 0, "single": 1, "general": 2, "fused": 3}[path])
    try:
        rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=160)
        om = models.oracle_model(lane_path, models.LANE, 160)
        toks = models.prompt(140, models.LANE["vocab"], 5)
        for step, tok in enumerate(toks):
            logits = rt.forward_token(tok)
            _, want = om.forward_greedy(tok, want_logits=True)
            if step % 10 == 9 or step >= 128:
                np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
        rt.close()
        om.close()
    finally:
        _lib.call("mantleHipSetAttentionPath", 0)


def test_tiny_generate_graph_matches_eager(hip, tiny_path):
    import mantle_amd
    p = models.prompt(9, models.TINY["vocab"], 1)
    rt = mantle_amd.new_backend().load_model(tiny_path, max_context=128)
    om = models.oracle_model(tiny_path, models.TINY, 128)
    try:
        want = om.generate_greedy(p, 64)
        got = rt.generate_greedy(p, 64)
        assert got == want
        rt.reset()
        rt.set_use_graph(False)
        assert rt.generate_greedy(p, 64) == want
        rt.reset()
        rt.set_use_graph(True)
        nxt = rt.prefill_tokens(p)
        assert nxt == want[0]
        seq = [nxt]
        for _ in range(7):
            seq.append(rt.forward_token_greedy(seq[-1]))
        assert seq == want[:8]
    finally:
        rt.close()
        om.close()


def test_load_from_memory_image_matches_path(hip, tiny_path):
    import mantle_amd
    p = models.prompt(5, models.TINY["vocab"], 2)
    a = mantle_amd.new_backend().load_model(tiny_path, max_context=32)
    b = mantle_amd.new_backend().load_model_image(open(tiny_path, "rb").read(), max_context=32)
    try:
        assert a.generate_greedy(p, 12) == b.generate_greedy(p, 12)
    finally:
        a.close()
        b.close()


def test_context_limit_and_bad_token(hip, tiny_path):
    import mantle_amd
    rt = mantle_amd.new_backend().load_model(tiny_path, max_context=4)
    try:
        with pytest.raises(mantle_amd.HipError):
            rt.forward_token_greedy(models.TINY["vocab"])
        rt.prefill_tokens([1, 2, 3, 4])
        with pytest.raises(mantle_amd.HipError):
            rt.forward_token_greedy(1)
        rt.reset()
        assert rt.pos == 0
        rt.forward_token_greedy(1)
    finally:
        rt.close()


@pytest.mark.parametrize("kv_cache", ["f32", "f16", "q8_0"])
def test_qwen3_0_6b_first_64_tokens(hip, tmp_models, kv_cache):
    """Qwen3-0.6B shape, weights seed 0, 31-token prompt seed 1:
    the first 64 greedy tokens equal the CPU oracle's, with Mantle's f32 cache
    (the loader default), its f16 cache (`mantle run`'s default) and q8_0."""
    import mantle_amd
    from mantle_amd.mcf import QWEN3_0_6B
    from oracle import oracle as o
    path = models.pack(str(tmp_models / "qwen3_0_6b_k4.mcf"), 0, QWEN3_0_6B)
    p = models.prompt(31, QWEN3_0_6B["vocab"], 1)
    rt = mantle_amd.new_backend().load_model(path, max_context=128, kv_cache=kv_cache)
    try:
        got = rt.generate_greedy(p, 64)
    finally:
        rt.close()
    o.set_threads(16)
    om = models.oracle_model(path, dict(QWEN3_0_6B, kv_cache=kv_cache), 128)
    try:
        want = om.generate_greedy(p, 64)
    finally:
        om.close()
    assert got == want


@pytest.mark.parametrize("kt,vt", [("f32", "f16"), ("f16", "f32"), ("f32", "q8_0"), ("q8_0", "f32"),
                                   ("f16", "q8_0"), ("q8_0", "f16")])
@pytest.mark.parametrize("ctx", [200, 650])
def test_lane_mixed_kv_cache_types(hip, lane_path, kt, vt, ctx):
    """--cache-type-k and --cache-type-v chosen independently
    (cmd/mantle/run.go:183-195; StoreKV / RunAttnHeads handle each cache by
    its own type, ops_runtime.go:112-131, attnpool.go:100-135): logits
    bit-identical to the oracle with the same pair, on the register-ring V
    sum (200 positions) and the LDS-staged one (650)."""
    import mantle_amd
    rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=ctx, kv_cache_k=kt, kv_cache_v=vt)
    om = models.oracle_model(lane_path, dict(models.LANE, kv_cache_k=kt, kv_cache_v=vt), ctx)
    try:
        n = 150 if ctx == 200 else 300
        toks = models.prompt(n, models.LANE["vocab"], 11)
        for step, tok in enumerate(toks):
            logits = rt.forward_token(tok)
            _, want = om.forward_greedy(tok, want_logits=True)
            if step % 25 == 24 or step in (0, 63, 64, 65, n - 1):
                np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
    finally:
        rt.close()
        om.close()


def test_load_from_tensor_views_matches_mcf_load(hip, lane_path):
    """mantleHipModelLoadTensors (a Go LoadModel feeding mcfstore.File's
    ReadTensorRaw payloads and the config.json section) builds the same model
    as loading the MCF file: identical logits per step."""
    import mantle_amd
    from mantle_amd.mcf import MCFFile
    f = MCFFile(lane_path)
    items = [(n, t["dtype"], t["shape"], f.raw(n).copy()) for n, t in f.tensors.items()]
    cfg_json = f.section(0x0100)
    a = mantle_amd.new_backend().load_model(lane_path, max_context=48)
    b = mantle_amd.new_backend().load_model_tensors(cfg_json, reversed(items), max_context=48)
    try:
        tok = 5
        for _ in range(8):
            la, lb = a.forward_token(tok), b.forward_token(tok)
            np.testing.assert_array_equal(la.view(np.uint32), lb.view(np.uint32))
            tok = int(np.argmax(la))
    finally:
        a.close()
        b.close()
        f.close()


def test_prefill_tokens_logits_and_effective_context(hip, lane_path):
    """PrefillTokens([]int) ([]float32, error) (internal/inference/engine.go:28-30):
    the last prompt position's logits equal the oracle's; SetEffectiveContextLength
    (internal/backend/core/instance.go:325-339) shrinks the caches before the first
    token without changing a result, and is refused mid-sequence."""
    import mantle_amd
    from mantle_amd import _lib
    prompt = models.prompt(40, models.LANE["vocab"], 12)
    rt = mantle_amd.new_backend().load_model(lane_path, max_context=400)
    om = models.oracle_model(lane_path, models.LANE, 400)
    try:
        rt.set_effective_context_length(64)
        assert rt.max_context == 64
        logits = rt.prefill_tokens_logits(prompt)
        want = None
        for t in prompt:
            _, want = om.forward_greedy(t, want_logits=True)
        np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32))
        assert _lib.lib().mantleHipModelSetEffectiveContextLength(rt._handle(), 128) == 1  # pos != 0
        tok = int(np.argmax(logits))
        for _ in range(20):  # up to position 60 of the 64
            lg = rt.forward_token(tok)
            nxt, w = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(lg.view(np.uint32), w.view(np.uint32))
            tok = nxt
        rt.reset()
        rt.set_effective_context_length(0)  # back to the load-time 400
        assert rt.max_context == 400
        assert rt.forward_token_greedy(prompt[0]) >= 0
    finally:
        rt.close()
        om.close()


def test_update_rope_recomputes_tables(hip, lane_path):
    """core.Runtime.UpdateRoPE (internal/backend/core/interfaces.go:14-18): with a
    new RoPE base the logits follow the oracle built with that base; with the
    same base nothing changes."""
    import mantle_amd
    rt = mantle_amd.new_backend().load_model(lane_path, max_context=32)
    om = models.oracle_model(lane_path, dict(models.LANE, rope_base=5e4), 32)
    try:
        rt.update_rope(0.0)
        rt.update_rope(5e4)
        assert rt.model_config()["rope_base"] == 5e4
        tok = 9
        for _ in range(6):
            lg = rt.forward_token(tok)
            nxt, w = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(lg.view(np.uint32), w.view(np.uint32))
            tok = nxt
    finally:
        rt.close()
        om.close()
