"""The BASELINE configs at their full sizes on the GPU, against the CPU oracle
or float64 where the oracle would take minutes:

* config 3 (prefill attention): S = 512 whole vs Mantle's position-by-position
  CPU prefill, S = 8192 rows (first, interior, last) vs float64;
* config 4 (Qwen3-4B k4, 36 blocks, vocab 151936, seed 4): greedy tokens after
  a short prompt identical to the oracle's;
* config 5 (Qwen3-8B, seed 5, k4 and raw bf16): logits bit-identical per step.

The models are packed once per box under MANTLE_BENCH_DIR (bench.py's files)."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tests import models  # noqa: E402
from tests import test_gpu_prefill as pf  # noqa: E402

MODEL_DIR = os.environ.get("MANTLE_BENCH_DIR", "/tmp/mantle_bench")


def _threads():
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, n))


def _model(name, seed, weights):
    from mantle_amd import mcf
    cfg = dict(getattr(mcf, name), weights=weights)
    os.makedirs(MODEL_DIR, exist_ok=True)
    tag = {"QWEN3_4B": "qwen3-4b", "QWEN3_8B": "qwen3-8b"}[name]
    path = os.path.join(MODEL_DIR, f"{tag}_{weights}_seed{seed}.mcf")
    mcf.pack_cached(path, seed, cfg)
    return path, cfg


def test_prefill_512_whole_vs_cpu_path(hip, oracle):
    """Config 3 at S = 512: every output vs the per-position CPU path."""
    seq, nh, kvh = 512, 16, 8
    bits, (qf, kf, vf) = pf.make_inputs(seq, nh, kvh)
    cos, sin = pf.rope_tables(oracle, seq)
    scale = float(np.float32(1.0 / np.sqrt(pf.HD)))
    got = pf.run_gpu(bits, cos, sin, seq, nh, kvh, scale)
    oracle.set_threads(_threads())
    want = pf.oracle_prefill(oracle, qf, kf, vf, cos, sin, seq, nh, kvh, scale)
    np.testing.assert_allclose(got, want, atol=pf.ATOL, rtol=pf.RTOL)


def test_prefill_8192_rows_vs_float64(hip, oracle):
    """Config 3 at S = 8192: the first, tile-edge, interior and last rows vs float64."""
    seq, nh, kvh = 8192, 16, 8
    bits, (qf, kf, vf) = pf.make_inputs(seq, nh, kvh)
    cos, sin = pf.rope_tables(oracle, seq)
    scale = float(np.float32(1.0 / np.sqrt(pf.HD)))
    got = pf.run_gpu(bits, cos, sin, seq, nh, kvh, scale)
    rows = [0, 1, 31, 32, 127, 128, 2047, 4095, 4096, 6001, 8190, 8191]
    want = pf.f64_rows(qf, kf, vf, cos, sin, rows, nh, kvh, scale)
    for t in rows:
        np.testing.assert_allclose(got[t], want[t], atol=pf.ATOL, rtol=pf.RTOL, err_msg=f"row {t}")
    assert np.isfinite(got).all()


def test_qwen3_4b_greedy_tokens(hip):
    """Config 4 at full size (36 blocks, d 2560, ffn 9728, 32/8 heads, vocab
    151936, seed 4): after an 8-token prompt the first 16 greedy tokens equal
    the oracle's."""
    import mantle_amd
    from oracle import oracle as o
    path, cfg = _model("QWEN3_4B", 4, "k4")
    p = models.prompt(8, cfg["vocab"], 1)
    rt = mantle_amd.new_backend().load_model(path, max_context=64)
    try:
        got = rt.generate_greedy(p, 16)
    finally:
        rt.close()
    o.set_threads(_threads())
    om = models.oracle_model(path, cfg, 64)
    try:
        want = om.generate_greedy(p, 16)
    finally:
        om.close()
    assert got == want


@pytest.mark.parametrize("weights", ["k4", "bf16"])
def test_qwen3_8b_logits_bitexact(hip, weights):
    """Config 5 at full size (36 blocks, d 4096, ffn 12288, untied lm_head, seed
    5), k4 and raw bf16 weights: three steps' logits bit-identical to the oracle."""
    import mantle_amd
    from oracle import oracle as o
    path, cfg = _model("QWEN3_8B", 5, weights)
    rt = mantle_amd.new_backend().load_model(path, max_context=16)
    o.set_threads(_threads())
    om = models.oracle_model(path, cfg, 16)
    try:
        tok = 7
        for step in range(3):
            logits = rt.forward_token(tok)
            nxt, want = om.forward_greedy(tok, want_logits=True)
            np.testing.assert_array_equal(logits.view(np.uint32), want.view(np.uint32), err_msg=f"step {step}")
            tok = nxt
    finally:
        rt.close()
        om.close()
