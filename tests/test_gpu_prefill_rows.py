"""Batched prompt prefill (all prompt rows per projection on int8 MFMA, the
attention rows on the decode kernels) against the per-token steps: the last
row's logits, the residual stream and the decode steps after it bit-identical,
for every KV cache type, across several passes of rows; and against the CPU
oracle directly."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import models  # noqa: E402


@pytest.fixture(scope="module")
def lane_path(tmp_models):
    return models.pack(str(tmp_models / "lane_rows.mcf"), 3, models.LANE)


@pytest.fixture(scope="module")
def tiny_path(tmp_models):
    return models.pack(str(tmp_models / "tiny_rows.mcf"), 0, models.TINY)


def _run(path, ctx, prompt, steps, env, **kw):
    import mantle_amd
    old = os.environ.get("MANTLE_HIP_PREFILL")
    if env:
        os.environ["MANTLE_HIP_PREFILL"] = env
    else:
        os.environ.pop("MANTLE_HIP_PREFILL", None)
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=ctx, **kw)
    try:
        out = [rt.prefill_tokens_logits(prompt), rt.hidden()]
        tok = int(np.argmax(out[0]))
        for _ in range(steps):
            lg = rt.forward_token(tok)
            out.append(lg)
            tok = int(np.argmax(lg))
        assert rt.pos == len(prompt) + steps
        return out
    finally:
        rt.close()
        if old is None:
            os.environ.pop("MANTLE_HIP_PREFILL", None)
        else:
            os.environ["MANTLE_HIP_PREFILL"] = old


@pytest.mark.parametrize("kt,vt", [("f32", "f32"), ("f16", "f16"), ("q8_0", "q8_0"), ("f32", "q8_0"),
                                   ("q8_0", "f16")])
@pytest.mark.parametrize("n,ctx", [(37, 96), (300, 650), (300, 32768)])
def test_prefill_rows_match_steps(hip, lane_path, kt, vt, n, ctx):
    """(300, 32768): the scores of 32768-key rows cap a pass at 256 rows, so the prompt takes two passes."""
    print(f"prefill rows kv {kt}/{vt} n={n} ctx={ctx}", flush=True)
    prompt = models.prompt(n, models.LANE["vocab"], 21 + n)
    rows = _run(lane_path, ctx, prompt, 6, None, kv_cache_k=kt, kv_cache_v=vt)
    steps = _run(lane_path, ctx, prompt, 6, "steps", kv_cache_k=kt, kv_cache_v=vt)
    for i, (a, b) in enumerate(zip(rows, steps)):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"output {i}")


def test_prefill_rows_tiny_vs_oracle(hip, tiny_path):
    """The tile-GEMV model shape (256-wide rows), prompt then decode, against the oracle."""
    prompt = models.prompt(50, models.TINY["vocab"], 5)
    got = _run(tiny_path, 80, prompt, 4, None)
    om = models.oracle_model(tiny_path, models.TINY, 80)
    try:
        want = None
        for t in prompt:
            _, want = om.forward_greedy(t, want_logits=True)
        np.testing.assert_array_equal(got[0].view(np.uint32), want.view(np.uint32))
        np.testing.assert_array_equal(got[1].view(np.uint32), om.hidden().view(np.uint32))
        tok = int(np.argmax(want))
        for i in range(4):
            nxt, w = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(got[2 + i].view(np.uint32), w.view(np.uint32), err_msg=f"step {i}")
            tok = nxt
    finally:
        om.close()


def test_generate_greedy_rows_match_steps(hip, lane_path):
    """GenerateGreedy's prompt takes the batched rows: the same tokens as the per-token steps."""
    import mantle_amd
    prompt = models.prompt(90, models.LANE["vocab"], 8)
    outs = []
    for env in (None, "steps"):
        if env:
            os.environ["MANTLE_HIP_PREFILL"] = env
        rt = mantle_amd.new_backend("hip").load_model(lane_path, max_context=160)
        try:
            outs.append(rt.generate_greedy(prompt, 40))
        finally:
            rt.close()
            os.environ.pop("MANTLE_HIP_PREFILL", None)
    assert outs[0] == outs[1]


def test_prefill_rows_gqa4_wide_rows(hip, tmp_models):
    """Four query heads per kv head (Qwen3-4B's 32 / 8) and 2560 / 9728-wide rows."""
    path = models.pack(str(tmp_models / "wide4b_rows.mcf"), 1, models.WIDE4B)
    prompt = models.prompt(70, models.WIDE4B["vocab"], 4)
    rows = _run(path, 128, prompt, 3, None)
    steps = _run(path, 128, prompt, 3, "steps")
    for i, (a, b) in enumerate(zip(rows, steps)):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"output {i}")


HD64 = dict(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, head_dim=64, ffn=1024, vocab=1000,
            rope_base=1e6, eps=1e-6, tie_embeddings=1)


@pytest.mark.parametrize("kt,vt", [("f32", "f32"), ("f16", "q8_0")])
def test_prefill_rows_head_dim_64(hip, tmp_models, kt, vt):
    """head_dim 64 (one column wave per head in the V sum): rows equal the per-token steps."""
    path = models.pack(str(tmp_models / "hd64_rows.mcf"), 2, HD64)
    prompt = models.prompt(90, HD64["vocab"], 6)
    rows = _run(path, 160, prompt, 4, None, kv_cache_k=kt, kv_cache_v=vt)
    steps = _run(path, 160, prompt, 4, "steps", kv_cache_k=kt, kv_cache_v=vt)
    for i, (a, b) in enumerate(zip(rows, steps)):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"output {i}")
