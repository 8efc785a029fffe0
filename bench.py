"""bench.py -- decode tok/s @ batch 1 and k4 GEMV HBM GB/s on one MI355X.

Workload (BASELINE.json configs[0] shape, the metric's model): Qwen3-0.6B-shaped
decoder (28 blocks, d 1024, FFN 3072, 16/8 heads, hd 128, vocab 151936), random
N(0,0.02) weights from seed 0 packed to MCF k4, a 31-token prompt (seed 1),
then greedy decode.  A "step" is one decode token.  Inputs are resident in HBM
before the timed region; the timed steps run back to back from the captured
HIP graph with the device-side argmax feeding the next step.

Also measured (not the headline value): BASELINE configs[1] k4 GEMV shapes at
batch 1 and 8, each launch on a different copy of the weights (>= 1 GiB
rotation, so the 256 MB MALL cannot serve them), timed with HIP events on the
launch stream; the lm_head GEMV (151936 x 1024) is the `roofline` kernel.
The CPU baseline is the C restatement of Mantle's CPU path (oracle/) timed on
this host on a bounded sample of the same decode.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA
PROMPT_LEN = 31


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_microbench(shapes, batches, iters=200, rotate_bytes=1 << 30, modes=("w4a8",)):
    """k4 GEMV per-launch HIP events: "w4a8" on pre-quantised activations (the decode
    GEMV, MatVecWithQuant on a PrepareQuantVec result), "w4a32" on the fp32 activations
    themselves (config 2's N(0,1) x, tolerance-checked arithmetic)."""
    import numpy as np
    import torch

    from mantle_amd import _lib, mcf

    stream = torch.cuda.current_stream()
    out = []
    for rows, cols in shapes:
        w = mcf.fill_normal(rows * cols, 2 + rows).reshape(rows, cols)
        payload = mcf.quantize_k4(w)
        del w
        psize = payload.nbytes
        copies = max(2, -(-rotate_bytes // psize))
        base = torch.from_numpy(payload).to("cuda:0")
        bufs = [base] + [base.clone() for _ in range(copies - 1)]
        bpr = (cols + 31) // 32
        spr = (bpr + 7) // 8
        sub_off = (rows * spr * 2 + 63) & ~63
        data_off = (sub_off + rows * bpr + 63) & ~63
        for batch, mode in [(b, m) for m in modes for b in batches]:
            x = torch.randn(batch, cols, device="cuda:0", generator=torch.Generator("cuda:0").manual_seed(2))
            qx = torch.empty(batch * bpr * 32, dtype=torch.int8, device="cuda:0")
            xs = torch.empty(batch * bpr, dtype=torch.float32, device="cuda:0")
            y = torch.empty(batch * rows, dtype=torch.float32, device="cuda:0")
            for b in range(batch):
                _lib.call("mantleHipQuantizeVecBlocksF32", x[b].data_ptr(), cols,
                          qx.data_ptr() + b * bpr * 32, xs.data_ptr() + 4 * b * bpr, stream.cuda_stream)

            def launch(i):
                p = bufs[i % copies].data_ptr()
                if mode == "w4a8":
                    _lib.call("mantleHipQuantMatVecK4W4A8QF32", p + data_off, p, p + sub_off, qx.data_ptr(),
                              xs.data_ptr(), y.data_ptr(), rows, bpr, cols, batch, stream.cuda_stream)
                else:
                    _lib.call("mantleHipQuantMatVecK4F32Batched", p + data_off, p, p + sub_off, x.data_ptr(),
                              y.data_ptr(), rows, bpr, cols, batch, stream.cuda_stream)

            for i in range(copies + 5):
                launch(i)
            # back-to-back launches between two HIP events on the launch stream:
            # the average is the kernel's duration plus the dispatch gap
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(iters):
                launch(i)
            e1.record(stream)
            torch.cuda.synchronize()
            avg_s = e0.elapsed_time(e1) * 1e-3 / iters
            # one launch per event pair, for the spread
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(32)]
            for i, (a, b) in enumerate(evs):
                a.record(stream)
                launch(i)
                b.record(stream)
            torch.cuda.synchronize()
            single = np.array([a.elapsed_time(b) for a, b in evs]) * 1e-3
            algo_bytes = psize + 4 * cols * batch + 4 * rows * batch
            out.append(dict(rows=rows, cols=cols, batch=batch, mode=mode, payload_bytes=psize, algo_bytes=algo_bytes,
                            avg_us=avg_s * 1e6, single_launch_median_us=float(np.median(single)) * 1e6,
                            gbs=algo_bytes / avg_s / 1e9, frac=algo_bytes / avg_s / 1e9 / PEAK_HBM_GBS,
                            rotation_copies=copies, launches=iters))
            log(f"gemv {mode} {rows}x{cols} B={batch}: {avg_s*1e6:.2f} us avg, {algo_bytes/avg_s/1e9:.0f} GB/s")
        del bufs, base
        torch.cuda.empty_cache()
    return out


def copy_calibration(nbytes=256 << 20, reps=5):
    """A plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: {reps} x {nbytes} B device-to-device copies")


def measured_copy_gbs(nbytes=1 << 30, reps=10):
    """HBM bandwidth a plain device-to-device copy reaches (bytes read + written per second):
    the measured ceiling beside the 8 TB/s spec peak."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    b.copy_(a)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (s.elapsed_time(e) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    log(f"copy kernel: {gbs:.0f} GB/s ({nbytes} B read + written per copy)")
    return gbs


def prefill_microbench(seqs=(512, 2048, 8192), nh=16, kvh=8, hd=128, reps=20):
    """Config 3: causal GQA attention prefill (bf16 q / k / v N(0,1), seed 3, RoPE base 1e6) on MFMA,
    and the pre-attention RMSNorm over seq x 2048 rows (unit-mean gains); HIP events on the launch stream."""
    import ctypes

    import numpy as np
    import torch

    from mantle_amd import _lib

    stream = torch.cuda.current_stream()
    gen = torch.Generator("cuda:0").manual_seed(3)
    out = []
    for S in seqs:
        q = torch.randn(S * nh * hd, device="cuda:0", generator=gen).to(torch.bfloat16)
        k = torch.randn(S * kvh * hd, device="cuda:0", generator=gen).to(torch.bfloat16)
        v = torch.randn(S * kvh * hd, device="cuda:0", generator=gen).to(torch.bfloat16)
        inv = 1.0 / (1e6 ** (np.arange(0, hd, 2, dtype=np.float64) / hd))  # loader.go:1604-1612
        ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
        cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to("cuda:0")
        sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to("cuda:0")
        o = torch.empty(S * nh * hd, device="cuda:0")
        scale = ctypes.c_float(1.0 / np.sqrt(hd))
        nws = ctypes.c_size_t()
        _lib.call("mantleHipAttentionPrefillWorkspaceSize", S, nh, kvh, hd, ctypes.byref(nws))
        ws = torch.empty(nws.value, dtype=torch.uint8, device="cuda:0")

        def attn():
            _lib.call("mantleHipAttentionPrefillBF16", q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(),
                      sin.data_ptr(), o.data_ptr(), S, nh, kvh, hd, scale, ws.data_ptr(), nws.value,
                      stream.cuda_stream)

        x = torch.randn(S * 2048, device="cuda:0", generator=gen)
        w = 1.0 + 0.1 * torch.randn(2048, device="cuda:0", generator=gen)  # unit-mean gains
        y = torch.empty_like(x)

        def norm():
            _lib.call("mantleHipRMSNormBatchedF32", y.data_ptr(), x.data_ptr(), w.data_ptr(), ctypes.c_float(1e-6),
                      2048, S, stream.cuda_stream)

        def timed(fn):
            for _ in range(3):
                fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / reps

        t_attn, t_norm = timed(attn), timed(norm)
        flops = 4 * hd * nh * S * (S + 1) / 2
        tf = flops / (t_attn * 1e-6) / 1e12
        nbytes = S * 2048 * 8 + 2048 * 4
        gbs = nbytes / (t_norm * 1e-6) / 1e9
        out.append(dict(seq=S, attention_us=round(t_attn, 2), algo_flops=flops, tflops=round(tf, 1),
                        mfma_frac=round(tf / PEAK_MFMA_F16_TFLOPS, 4),
                        rmsnorm_us=round(t_norm, 2), rmsnorm_bytes=nbytes, rmsnorm_gbs=round(gbs, 1),
                        rmsnorm_frac=round(gbs / PEAK_HBM_GBS, 4)))
        log(f"prefill attention S={S}: {t_attn:.1f} us, {tf:.1f} TFLOP/s ({tf / PEAK_MFMA_F16_TFLOPS:.1%} of "
            f"{PEAK_MFMA_F16_TFLOPS:.0f}); rmsnorm {S}x2048: {t_norm:.2f} us, {gbs:.0f} GB/s")
        del q, k, v, o, x, y, ws
    return out


def traffic_from_profile():
    """HBM bytes per launch of the roofline kernel, as measured by the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/), or None."""
    path = os.path.join(ROOT, "profiles", "k4_gemv_lm_head_151936x1024_pmc.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1].strip())
    except OSError:
        return None
    return None


def host_cpu():
    """CPU model, logical CPUs, the CPUs this process may run on, and the ISA
    Mantle's CPU path would dispatch to (AVX-512 if avx512f, else AVX2,
    internal/backend/simd/tensor_cpu.go:18-24)."""
    model, flags = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    isa = "avx512" if "avx512f" in flags else ("avx2" if "avx2" in flags else "scalar")
    return dict(model=model, nproc=os.cpu_count() or 1, usable=usable, isa=isa)


def cpu_baseline(path, cfg, prompt, steps=128, steps_1t=8):
    """The oracle (C restatement of Mantle's CPU path) on this host: the prompt
    token by token, then `steps` greedy decode steps on every usable core
    (rows and heads split over threads as matVecWithQuant splits rows,
    internal/backend/simd/matvec.go:175-208), then `steps_1t` more on one thread."""
    from oracle import oracle as o
    from tests import models

    hc = host_cpu()
    threads = hc["usable"]
    m = models.oracle_model(path, cfg, PROMPT_LEN + steps + steps_1t + 2)
    try:
        o.set_threads(threads)
        t0 = time.perf_counter()
        nxt = None
        for t in prompt:
            nxt = m.forward_greedy(t)
        t_prefill = time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(steps):
            nxt = m.forward_greedy(nxt)
        dt = time.perf_counter() - t0
        o.set_threads(1)
        t0 = time.perf_counter()
        for _ in range(steps_1t):
            nxt = m.forward_greedy(nxt)
        dt1 = time.perf_counter() - t0
    finally:
        m.close()
    return dict(value=round(steps / dt, 3), unit="tok/s", cores=threads, kind="port",
                value_1thread=round(steps_1t / dt1, 3),
                cpu_model=hc["model"], nproc=hc["nproc"], host_isa=hc["isa"], reduction_order="avx512",
                steps=steps, steps_1thread=steps_1t, prefill_tok_s=round(PROMPT_LEN / t_prefill, 3),
                sample=f"Qwen3-0.6B k4 (config 1): {PROMPT_LEN}-token prompt, then {steps} greedy decode steps on "
                       f"{threads} threads (all CPUs this process may use; nproc {hc['nproc']}), then {steps_1t} "
                       f"more on 1 thread; oracle/ C restatement of Mantle's archsimd path in the AVX-512 "
                       f"reduction order (host dispatch would pick {hc['isa']}), {hc['model']}")


def cpu_gemv_baseline(shapes=((151936, 1024), (3072, 1024), (1024, 3072), (2048, 1024)), threads=None,
                      rotate_bytes=1 << 30, min_s=1.0):
    """Config 2 on the host: the oracle's W4A8 GEMV (MatVecWithQuant: the activation's
    int8 quantisation and the ordered block sums) at batch 1 on every usable core,
    the same weights (seed 2) and x ~ N(0,1); weight copies rotated over >= 1 GiB so
    the last-level cache cannot serve them; GB/s of algorithmic bytes."""
    import numpy as np

    from mantle_amd import mcf
    from oracle import oracle as o

    threads = threads or host_cpu()["usable"]
    o.set_threads(threads)
    out = []
    for rows, cols in shapes:
        payload = mcf.quantize_k4(mcf.fill_normal(rows * cols, 2 + rows).reshape(rows, cols))
        copies = max(2, -(-rotate_bytes // payload.nbytes))
        bufs = [payload] + [payload.copy() for _ in range(copies - 1)]
        x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
        o.matvec_w4a8(bufs[0], rows, cols, x)
        n, t0 = 0, time.perf_counter()
        while n < copies or time.perf_counter() - t0 < min_s:
            o.matvec_w4a8(bufs[n % copies], rows, cols, x)
            n += 1
        dt = (time.perf_counter() - t0) / n
        algo = mcf.payload_size(rows, cols) + 4 * cols + 4 * rows
        out.append(dict(rows=rows, cols=cols, batch=1, avg_us=round(dt * 1e6, 1), gbs=round(algo / dt / 1e9, 2),
                        threads=threads, launches=n))
        log(f"cpu gemv w4a8 {rows}x{cols}: {dt * 1e3:.2f} ms, {algo / dt / 1e9:.2f} GB/s on {threads} threads")
        del bufs
    return out


def weight_bytes_per_token(cfg):
    """Weight bytes one decode token streams: every block matrix plus the lm_head
    (the tied embedding when tie_embeddings), norms as fp32; k4 payloads, or 2
    bytes per weight with cfg["weights"] == "bf16"."""
    from mantle_amd.mcf import payload_size
    d, f, hd = cfg["d_model"], cfg["ffn"], cfg["head_dim"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    if cfg.get("weights") == "bf16":
        payload_size = lambda r, c: 2 * r * c  # noqa: E731
    layer = (payload_size(qd, d) + 2 * payload_size(kvd, d) + payload_size(d, qd) + 2 * payload_size(f, d)
             + payload_size(d, f) + 4 * (2 * d + 2 * hd))
    return cfg["n_layers"] * layer + payload_size(cfg["vocab"], d) + 4 * d


def prompt_prefill_bench(path, lengths=(512, 2048), reps=3):
    """Prompt prefill on the batched path (every projection one int8-MFMA GEMM
    over the prompt rows, attention rows per kv head; bit-identical to the
    per-token steps): best of `reps` timed PrefillTokens calls per length, each
    after a Reset, on a runtime sized for the longest prompt."""
    import mantle_amd
    from mantle_amd import mcf
    from mantle_amd.mcf import QWEN3_0_6B
    out = []
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=max(lengths) + 8)
    try:
        for n in lengths:
            prompt = mcf.uniform_tokens(n, QWEN3_0_6B["vocab"], 2)
            rt.prefill_tokens(prompt[:16])  # first-call allocations outside the timing
            best = None
            for _ in range(reps):
                rt.reset()
                t0 = time.perf_counter()
                rt.prefill_tokens(prompt)
                dt = time.perf_counter() - t0
                best = dt if best is None or dt < best else best
            out.append(dict(tokens=n, ms=round(best * 1e3, 3), tok_s=round(n / best, 1)))
            log(f"prompt prefill {n} tokens: {best * 1e3:.2f} ms, {n / best:.0f} tok/s")
    finally:
        rt.close()
    return out


def decode_run(rt, prompt, warmup, steps):
    """Token-by-token prefill of `prompt` (as Mantle runs k4 prefill; the first
    token also captures the step graph), then `warmup` untimed and `steps` timed
    greedy decode steps.  Returns (decode seconds, prefill tok/s)."""
    import torch
    rt.prefill_tokens(prompt[:1])
    rt.synchronize()
    t0 = time.perf_counter()
    for i in range(1, len(prompt), 1024):  # progress on long prompts
        rt.prefill_tokens(prompt[i:i + 1024])
        rt.synchronize()
        if len(prompt) > 4096:
            log(f"prefill {min(i + 1024, len(prompt))}/{len(prompt)} tokens, {time.perf_counter() - t0:.1f} s")
    prefill_tps = (len(prompt) - 1) / (time.perf_counter() - t0)
    if warmup:
        rt.decode_steps(warmup)
    rt.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rt.decode_steps(steps)
    rt.synchronize()
    torch.cuda.synchronize()
    return time.perf_counter() - t0, prefill_tps


# Configs 4 and 5 (reported, not the headline): larger decoders after a long prompt.
LARGE_MODELS = {"qwen3-4b": ("QWEN3_4B", 4, 2048), "qwen3-8b": ("QWEN3_8B", 5, 16384)}


def large_model_run(args):
    import mantle_amd
    from mantle_amd import mcf
    name, seed, plen = LARGE_MODELS[args.model]
    cfg = dict(getattr(mcf, name), weights=args.weights)
    plen = args.prompt or plen
    os.makedirs(args.model_dir, exist_ok=True)
    path = os.path.join(args.model_dir, f"{args.model}_{args.weights}_seed{seed}.mcf")
    t0 = time.perf_counter()
    mcf.pack_cached(path, seed, cfg)
    log(f"model ready in {time.perf_counter() - t0:.1f} s: {path}")
    prompt = mcf.uniform_tokens(plen, cfg["vocab"], 1)
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=plen + args.warmup + args.steps + 8,
                                                  kv_cache=args.kv_cache)
    try:
        dt, prefill_tps = decode_run(rt, prompt, args.warmup, args.steps)
    finally:
        rt.close()
    tps = args.steps / dt
    wb = weight_bytes_per_token(cfg)
    kv_elem = {"f16": 2, "q8_0": 1}.get(args.kv_cache, 4)
    kv_mid = 2 * cfg["n_layers"] * cfg["n_kv_heads"] * cfg["head_dim"] * kv_elem * (plen + args.warmup + args.steps // 2)
    log(f"{args.model} {args.weights} kv {args.kv_cache}: decode {tps:.1f} tok/s, prefill {prefill_tps:.1f} tok/s")
    print(json.dumps({
        "metric": f"decode tok/s @batch1, {args.model} {args.weights} after a {plen}-token prompt, {args.kv_cache} KV cache",
        "value": round(tps, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16 weights x fp32 activations, fp32 accumulation" if args.weights == "bf16"
                  else "k4 weights x int8 activations, int32 block dots, fp32 accumulation"),
        "data": f"synthetic: random-init N(0,0.02) weights seed {seed} packed to MCF {args.weights}, {plen} uniform "
                f"token ids seed 1",
        "config": {"workload": f"{args.model}-shape {args.weights} greedy decode, batch 1 (BASELINE config {seed})",
                   "prompt_tokens": plen, "parallelism": "none (1 GPU)"},
        "prefill_tok_s": round(prefill_tps, 2),
        "weight_bytes_per_token": wb,
        "kv_bytes_per_token_mid": kv_mid,
        "effective_gbs": round((wb + kv_mid) * tps / 1e9, 1),
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemv", action="store_true", help="skip the GEMV microbench")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 prefill attention microbench")
    ap.add_argument("--prefill-only", action="store_true", help="only the config-3 prefill microbench (for rocprofv3)")
    ap.add_argument("--prompt-prefill-only", action="store_true",
                    help="only the batched prompt prefill of the config-1 model (for rocprofv3)")
    ap.add_argument("--gemv-batch", type=int, default=1, help="--gemv-only: the batch of the logits-shape GEMV")
    ap.add_argument("--gemv-mode", default="w4a8", choices=["w4a8", "w4a32"],
                    help="--gemv-only: int8 (CPU-parity) or fp32 activations")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the lm_head GEMV microbench and a copy calibration (for rocprofv3 --pmc runs)")
    ap.add_argument("--model", default="qwen3-0.6b", choices=["qwen3-0.6b", *LARGE_MODELS],
                    help="qwen3-4b / qwen3-8b: configs 4 / 5, a decode line of their own (not the headline)")
    ap.add_argument("--prompt", type=int, default=0, help="prompt length for --model qwen3-4b / qwen3-8b")
    ap.add_argument("--kv-cache", default="f32", choices=["f32", "f16", "q8_0"],
                    help="KV cache element type for --model qwen3-4b / qwen3-8b (f16: `mantle run`'s default)")
    ap.add_argument("--weights", default="k4", choices=["k4", "bf16"],
                    help="weight format for --model qwen3-4b / qwen3-8b (config 5 runs both)")
    ap.add_argument("--model-dir", default=os.environ.get("MANTLE_BENCH_DIR", "/tmp/mantle_bench"))
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "single-GPU build: bench.py measures one MI355X; --gpus > 1 is not supported "
                                   "(the path would shard the GEMV rows and the attention by kv head, one process per GPU)"}))
        sys.exit(2)

    import torch

    import mantle_amd
    from mantle_amd import mcf
    from mantle_amd.mcf import QWEN3_0_6B

    if args.model != "qwen3-0.6b":
        large_model_run(args)
        return

    if args.prefill_only:
        print(json.dumps({"prefill": prefill_microbench()}), flush=True)
        return

    if args.gemv_only:
        g = gemv_microbench([(151936, 1024)], [args.gemv_batch], iters=50, modes=(args.gemv_mode,))[0]
        copy_calibration()
        print(json.dumps({"gemv": g}), flush=True)
        return

    os.makedirs(args.model_dir, exist_ok=True)
    path = os.path.join(args.model_dir, "qwen3_0_6b_k4_seed0.mcf")
    t0 = time.perf_counter()
    mcf.pack_cached(path, 0, QWEN3_0_6B)
    log(f"model ready in {time.perf_counter() - t0:.1f} s: {path}")
    if args.prompt_prefill_only:
        print(json.dumps({"prompt_prefill": prompt_prefill_bench(path)}), flush=True)
        return
    prompt = mcf.uniform_tokens(PROMPT_LEN, QWEN3_0_6B["vocab"], 1)
    max_ctx = PROMPT_LEN + args.warmup + args.steps + 8
    rt = mantle_amd.new_backend("hip").load_model(path, max_context=max_ctx)
    try:
        dt, prefill_tps = decode_run(rt, prompt, args.warmup, args.steps)
    finally:
        rt.close()
    tps = args.steps / dt
    log(f"decode: {tps:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token), prefill {prefill_tps:.1f} tok/s")

    prompt_prefill = prompt_prefill_bench(path)
    gemv = []
    if not args.no_gemv:
        gemv = gemv_microbench([(151936, 1024), (3072, 1024), (1024, 3072), (2048, 1024)], [1, 8],
                               modes=("w4a8", "w4a32"))
    prefill = [] if args.no_prefill else prefill_microbench()
    head = next((g for g in gemv if g["rows"] == 151936 and g["batch"] == 1 and g["mode"] == "w4a8"), None)
    roofline = None
    if head:
        roofline = dict(bound="hbm", achieved=round(head["gbs"], 1), peak=PEAK_HBM_GBS, unit="GB/s",
                        frac=round(head["frac"], 4), traffic=traffic_from_profile(),
                        kernel="k4_gemv_lane_kernel<0,8,4,1,4,0,1,0> (W4A8 store, 8 lanes/row, 4-wave one-unit workgroups) 151936x1024 B=1",
                        avg_launch_us=round(head["avg_us"], 3), algo_bytes_per_launch=head["algo_bytes"])
        copy = measured_copy_gbs()
        roofline["measured_copy_gbs"] = round(copy, 1)
        roofline["frac_of_measured_copy"] = round(head["gbs"] / copy, 4)
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(path, QWEN3_0_6B, prompt)
            cpu["gemv"] = cpu_gemv_baseline()
            log(f"cpu baseline: {cpu['value']:.3f} tok/s on {cpu['cores']} threads, "
                f"{cpu['value_1thread']:.3f} tok/s on 1 ({cpu['cpu_model']})")
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline failed: {e!r}")
    bytes_per_token = weight_bytes_per_token(QWEN3_0_6B)
    line = {
        "metric": "decode tok/s @batch1 + k4 GEMV HBM GB/s (% of peak), Qwen3-0.6B-shape k4",
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        # the CPU leg measured on this host (no published number exists for this metric on this hardware)
        "vs_baseline": round(tps / cpu["value"], 2) if cpu else None,
        "dtype": "k4 weights x int8 activations, int32 block dots, fp32 accumulation",
        "data": "synthetic: random-init N(0,0.02) weights seed 0 packed to MCF k4, 31 uniform token ids seed 1",
        "config": {"workload": "Qwen3-0.6B-shape k4 greedy decode, batch 1 (28 blocks, d1024, ffn3072, 16/8 heads, "
                               "hd128, vocab151936)", "prompt_tokens": PROMPT_LEN, "parallelism": "none (1 GPU)"},
        # batched prompt prefill, 512-token prompt (the decode run's 31-token prompt: prefill_31_tok_s)
        "prefill_tok_s": prompt_prefill[0]["tok_s"],
        "prefill_31_tok_s": round(prefill_tps, 2),
        "prompt_prefill": prompt_prefill,
        "effective_weight_gbs": round(bytes_per_token * tps / 1e9, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gemv": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in g.items()} for g in gemv],
        "prefill_attention": prefill,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
