"""Per-kernel phase breakdown of one decode step (latency study).

    python -m mantle_amd.build --phase-trace     # once: libmantle_hip_trace.so
    python -m mantle_amd.phase_trace [--steps N] [--model qwen3-0.6b|qwen3-4b] [--prompt P]

Runs the Qwen3-0.6B-shape k4 decode (or the 4B shape) on the phase-trace
build of the library, whose kernels stamp workgroup 0's wall clock (100 MHz)
at fixed points, and prints, per kernel of the decoder layer, the mean offset
of each stamp from that workgroup's start and the start-to-start time to the
next kernel.  Stamps: lane GEMVs 1 loads issued, 2 activation arrived,
6 RMSNorm scale known, 3 int8 activation staged (prologue done), 4 first unit
summed, 5 workgroup 0 done; V-sum launch 1 softmax done, 2 V sum and store
done; the score launch only its start.
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
KINDS = ["QKV GEMV (RMSNorm prologue)", "attention scores", "softmax + V sum", "Wo GEMV + residual",
         "gate/up GEMV (RMSNorm, SiLU*up)", "down GEMV + residual"]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--model-dir", default=os.environ.get("MANTLE_BENCH_DIR", "/tmp/mantle_bench"))
    ap.add_argument("--model", default="qwen3-0.6b", choices=("qwen3-0.6b", "qwen3-4b"))
    ap.add_argument("--prompt", type=int, default=31, help="prompt tokens before the traced decode steps")
    ap.add_argument("--raw", type=int, default=0, help="also print the first N stamped launches of the last step")
    args = ap.parse_args()
    trace = os.path.join(HERE, "libmantle_hip_trace.so")
    if not os.path.exists(trace):
        sys.exit("build the trace library first: python -m mantle_amd.build --phase-trace")
    os.environ["MANTLE_HIP_LIB"] = trace
    from . import _lib
    _lib.LIB_PATH = trace
    from . import mcf
    from .backend import new_backend
    os.makedirs(args.model_dir, exist_ok=True)
    cfg, seed, name = ((mcf.QWEN3_0_6B, 0, "qwen3_0_6b_k4_seed0.mcf") if args.model == "qwen3-0.6b"
                       else (mcf.QWEN3_4B, 4, "qwen3_4b_k4_seed4.mcf"))
    path = mcf.pack_cached(os.path.join(args.model_dir, name), seed, cfg)
    rt = new_backend().load_model(path, max_context=max(512, args.prompt + args.steps + 16))
    fn = _lib.lib().mantleHipDebugPhaseTrace
    fn.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_uint)]
    buf = np.zeros(8192 * 8, dtype=np.uint64)
    n = C.c_uint()
    try:
        rt.prefill_tokens(mcf.uniform_tokens(args.prompt, cfg["vocab"], 1))
        rt.synchronize()
        fn(buf.ctypes.data, 8192, C.byref(n))
        n0 = n.value
        rt.decode_steps(args.steps)
        rt.synchronize()
        fn(buf.ctypes.data, 8192, C.byref(n))
        n1 = n.value
    finally:
        rt.close()
    per = (n1 - n0) // args.steps
    t = buf[:n1 * 8].reshape(n1, 8).astype(np.int64)
    steps = min(5, args.steps)
    rows = t[n1 - steps * per:].reshape(steps, per, 8)
    L = cfg["n_layers"]
    if args.raw:
        last = rows[-1]
        for i in list(range(min(args.raw, per - 1))) + list(range(max(args.raw, per - 4), per)):
            st = [f"{(last[i, c] - last[i, 0]) * 0.01:.2f}" if last[i, c] > 0 else "-" for c in (1, 2, 6, 3, 4, 5)]
            nxt = f"{(last[i + 1, 0] - last[i, 0]) * 0.01:.2f} us" if i + 1 < per else "-"
            print(f"launch {i}: start-to-next {nxt}, stamps", " ".join(st))
    head = per - 6 * L - 1  # stamped launches before the first layer (embed)
    start = rows[:, :, 0]
    s2s = np.diff(start, axis=1) * 0.01  # us
    if args.raw and steps > 1:
        cross = (rows[1:, 0, 0] - rows[:-1, per - 1, 0]) * 0.01
        print(f"last launch of a step to the first of the next: {cross.mean():.2f} us")
    print(f"stamped launches per step: {per}; step start-to-start "
          f"{(start[:, -1] - start[:, 0]).mean() * 0.01:.1f} us over the last {steps} steps")
    print("| kernel | start-to-start us | " + " | ".join(f"stamp {k}" for k in (1, 2, 6, 3, 4, 5)) + " |")
    print("|---|---:|" + "---:|" * 6)
    for kind in range(6):
        idx = [head + 6 * l + kind for l in range(L)]
        sel = rows[:, idx, :]
        off = lambda c: ((sel[:, :, c] - sel[:, :, 0]) * 0.01).mean()  # noqa: E731
        cells = []
        for c in (1, 2, 6, 3, 4, 5):
            v = off(c)
            cells.append(f"{v:.2f}" if (sel[:, :, c] > 0).all() and v >= 0 else "-")
        ss = s2s[:, [i for i in idx if i < per - 1]].mean()
        print(f"| {KINDS[kind]} | {ss:.2f} | " + " | ".join(cells) + " |")


if __name__ == "__main__":
    main()
