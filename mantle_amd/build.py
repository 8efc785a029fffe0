"""Build libmantle_hip.so for gfx950 in-tree (hipcc, no build system needed).

    python -m mantle_amd.build                 # the product library
    python -m mantle_amd.build --phase-trace   # libmantle_hip_trace.so: the same kernels with
                                               # workgroup-0 phase timestamps (mantle_amd.phase_trace)

The shared library lands next to this file so that it travels with the
repository snapshot to the GPU box.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmantle_hip.so")
TRACE_LIB = os.path.join(HERE, "libmantle_hip_trace.so")
OBJ_DIR = os.path.join(HERE, "_build")
SOURCES = ["gemv_lane_store.hip", "gemv_lane_fused.hip", "gemv_lane_b8.hip", "gemv_w4a32.hip", "gemm_w4a8.hip", "gemm_w4a32.hip", "gemv_bf16.hip", "attention.hip", "prefill_attention.hip", "kernels.hip", "runtime.cpp", "capi.cpp",
           "mcf.cpp"]
ARCH = os.environ.get("MANTLE_HIP_ARCH", "gfx950")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall",
    # no implicit FMA anywhere: the CPU-parity kernels depend on it
    "-ffp-contract=off",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source flags.  attention.hip runs with f16 (and f64) denormals flushed:
# its f16 KV cache reads convert with v_cvt_f32_f16, which then flushes
# subnormal inputs to signed zero as Mantle's Float16ToFloat32 does; fp32 stays
# IEEE (denormals kept) like everywhere else.
EXTRA = {
    "attention.hip": ["-fdenormal-fp-math=preserve-sign", "-Xclang", "-fdenormal-fp-math-f32=ieee",
                      "-DMANTLE_F16_INPUT_FTZ=1"],
    # matrix-core results straight into VGPRs: the int32 dots are read by VALU
    # arithmetic at once, and AGPR results would cost a copy each
    "gemm_w4a32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # f16 inputs flushed as in attention.hip: the weight super-scales decode
    # through v_cvt_f32_f16 with Mantle's subnormal-to-zero
    "gemm_w4a8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fdenormal-fp-math=preserve-sign", "-Xclang",
                      "-fdenormal-fp-math-f32=ieee"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str, obj_dir: str = OBJ_DIR, defines: tuple = ()) -> str:
    obj = os.path.join(obj_dir, src + ".o")
    cmd = [hipcc(), *COMMON, *defines, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".hip"):
        cmd.insert(1, "-xhip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True, phase_trace: bool = False) -> str:
    obj_dir = OBJ_DIR + ("_trace" if phase_trace else "")
    lib = TRACE_LIB if phase_trace else LIB
    defines = ("-DMANTLE_PHASE_TRACE",) if phase_trace else ()
    os.makedirs(obj_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), SOURCES))
    tmp = lib + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(phase_trace="--phase-trace" in sys.argv[1:])
