"""CPU tests of the product's host side: the k4 producer, the MCF writer and
reader, the C ABI's symbol table and its host-side argument validation (no GPU
compute is called here)."""
import ctypes as C
import json
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import mantle_amd
from mantle_amd import _lib, mcf
from oracle import oracle as o
from tests import models

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mantle_hip.h")


def test_header_symbols_exported():
    """Every function include/mantle_hip.h declares is exported by libmantle_hip.so."""
    decl = set(re.findall(r"\b(mantleHip\w+)\s*\(", open(HEADER).read()))
    assert decl, "no declarations parsed"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\b(mantleHip\w+)\b", out.stdout))
    assert decl <= exported, sorted(decl - exported)
    assert decl == set(_lib.exported_symbols()), sorted(decl ^ set(_lib.exported_symbols()))
    _lib.lib()  # every binding resolves


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 33), (7, 300), (64, 1024), (5, 3000), (2, 96)])
def test_product_quantizer_matches_oracle(rows, cols):
    w = mcf.fill_normal(rows * cols, rows * 1000 + cols).reshape(rows, cols)
    w[0, 0] = 0.0
    np.testing.assert_array_equal(mcf.quantize_k4(w), o.quantize_k4(w))
    assert mcf.payload_size(rows, cols) == o.payload_size(rows, cols)


def test_product_quantizer_edge_tensors():
    for w in (np.zeros((2, 64), np.float32), np.full((1, 32), -3.0, np.float32),
              np.array([[1e-30, -2e-30] * 16], np.float32), np.array([[60000.0] + [1.0] * 31], np.float32)):
        np.testing.assert_array_equal(mcf.quantize_k4(w), o.quantize_k4(w))
    with pytest.raises(_lib.HipError):
        mcf.quantize_k4(np.array([[np.nan] * 32], np.float32))


def test_fill_normal_moments_and_determinism():
    a = mcf.fill_normal(200001, 42, 0.02)
    assert np.array_equal(a, mcf.fill_normal(200001, 42, 0.02))
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert not np.array_equal(a, mcf.fill_normal(200001, 43, 0.02))


def test_mcf_container_layout(tmp_path):
    """Independent parse of the written file: header (pkg/mcf/header.go), sorted
    section directory, sorted tensor index, 64-aligned payloads inside TensorData,
    QuantInfo records (pkg/mcf/quantinfo.go)."""
    cfg = dict(models.TINY)
    path = models.pack(str(tmp_path / "t.mcf"), 9, cfg)
    b = open(path, "rb").read()
    magic, major, minor, hsize, nsec, diroff, fsize, flags = struct.unpack_from("<4sHHIIQQQ", b, 0)
    assert magic == b"MCF\0" and major == 1 and hsize == 40 and fsize == len(b) and flags & 1
    secs = [struct.unpack_from("<IIQQ", b, diroff + 24 * i) for i in range(nsec)]
    types = [s[0] for s in secs]
    assert types == sorted(types) and {2, 3, 4, 0x100} <= set(types)
    for t, v, off, size in secs:
        assert off % 8 == 0 and off + size <= diroff
    sec = {s[0]: s for s in secs}
    cj = json.loads(b[sec[0x100][2]:sec[0x100][2] + sec[0x100][3]])
    assert cj["model_type"] == "qwen3" and cj["head_dim"] == cfg["head_dim"]
    ioff = sec[3][2]
    ver, fl, count, ndims, eoff, doff, soff, ssz = struct.unpack_from("<IIIIQQQQ", b, ioff)
    assert ver == 1 and fl & 1
    names, td = [], sec[4]
    for i in range(count):
        noff, nlen, dt, rank, dimoff, _, off, size = struct.unpack_from("<IIIIIIQQ", b, ioff + eoff + 40 * i)
        name = b[ioff + soff + noff: ioff + soff + noff + nlen].decode()
        names.append(name)
        shape = struct.unpack_from(f"<{rank}Q", b, ioff + doff + 8 * dimoff)
        assert td[2] <= off and off + size <= td[2] + td[3] and off % 64 == 0
        if dt == mcf.DTYPE_K4:
            assert size == o.payload_size(*shape)
        else:
            assert dt == mcf.DTYPE_F32 and size == 4 * shape[0]
            assert np.all(np.frombuffer(b[off:off + size], np.float32) == 1.0)
    assert names == sorted(names)
    qh = struct.unpack_from("<II", b, sec[2][2])
    assert qh[0] == 1 and qh[1] == sum(1 for n in names if n.endswith("proj.weight") or "embed" in n)


def _fnv1a(s: str) -> int:
    h = 0xcbf29ce484222325
    for ch in s.encode():
        h = ((h ^ ch) * 0x100000001b3) & ((1 << 64) - 1)
    return h


def test_mcf_payloads_are_quantized_seeded_weights(tmp_path):
    """The packed k4 payload of each tensor equals quantize_k4 of the seeded
    N(0,0.02) weights (seed = splitmix64(model_seed ^ fnv1a(name)))."""
    cfg = dict(models.TINY)
    path = models.pack(str(tmp_path / "t.mcf"), 11, cfg)
    with mcf.MCFFile(path) as f:
        for name in ("model.layers.1.mlp.down_proj.weight", "model.embed_tokens.weight"):
            r, c = f.tensors[name]["shape"]
            w = mcf.fill_normal(r * c, models.splitmix64(11 ^ _fnv1a(name)), 0.02).reshape(r, c)
            np.testing.assert_array_equal(f.raw(name), o.quantize_k4(w))


def test_mcf_reader_rejects_corruption(tmp_path):
    path = models.pack(str(tmp_path / "t.mcf"), 1, dict(models.TINY))
    b = bytearray(open(path, "rb").read())
    bad = tmp_path / "bad.mcf"
    for mutate in (lambda x: x.__setitem__(0, ord("X")), lambda x: x.__setitem__(slice(24, 32), b"\0" * 8),
                   lambda x: x.__delitem__(slice(len(x) - 10, len(x)))):
        c = bytearray(b)
        mutate(c)
        bad.write_bytes(bytes(c))
        with pytest.raises(_lib.HipError):
            mcf.MCFFile(str(bad))
    with pytest.raises(_lib.HipError):
        mcf.MCFFile(str(tmp_path / "missing.mcf"))


def test_host_validation_rejects_bad_arguments():
    """Null pointers / bad dims return hipErrorInvalidValue (1) before any launch
    (the contract of internal/backend/cuda/native/ops_validation_test.go)."""
    L = _lib.lib()
    fake = C.c_void_p(0x1000)
    assert L.mantleHipQuantMatVecK4F32(None, None, None, None, None, 4, 1, 32, None) == 1
    assert L.mantleHipQuantMatVecK4F32(fake, fake, fake, fake, fake, 4, 2, 32, None) == 1  # bpr != ceil(cols/32)
    assert L.mantleHipQuantMatVecK4W4A8F32(fake, fake, fake, fake, fake, 4, 1, 32, 9, fake, fake, None) == 1
    assert L.mantleHipQuantMatVecK4W4A8QF32(fake, fake, fake, fake, fake, fake, 0, 1, 32, 1, None) == 1
    assert L.mantleHipRMSNormF32(None, fake, fake, C.c_float(1e-6), 8, None) == 1
    assert L.mantleHipRMSNormF32(fake, fake, fake, C.c_float(1e-6), 0, None) == 1
    assert L.mantleHipAttentionInnerF32Cache(fake, fake, fake, fake, fake, 5, 6, 16, 8, 4, 2, 6, C.c_float(1), None) == 1  # start > pos
    assert L.mantleHipAttentionInnerF32Cache(fake, fake, fake, fake, fake, 5, 0, 16, 8, 4, 3, 6, C.c_float(1), None) == 1
    assert L.mantleHipApplyRoPEInplaceTableF32(fake, fake, fake, 8, 5, 1, None) == 1
    assert L.mantleHipSoftmaxRowsF32(fake, 0, 4, None) == 1
    assert L.mantleHipArgMaxF32(fake, 0, fake, None) == 1
    assert L.mantleHipSetParityISA(7) == 1
    # q8_0 cache: rows past 4096 values, a null row, a start past pos, head_dim 96 (no split kernel)
    assert L.mantleHipStoreKVQ8Row(fake, fake, fake, fake, fake, fake, 0, 5000, None) == 1
    assert L.mantleHipStoreKVQ8Row(fake, fake, fake, fake, None, fake, 0, 1024, None) == 1
    assert L.mantleHipStoreKVQ8Row(fake, fake, fake, fake, fake, fake, 0, 0, None) == 1
    assert L.mantleHipAttentionInnerQ8CacheF32(fake, fake, fake, fake, fake, fake, fake, 5, 6, 1024, 128, 16, 8, 6,
                                               C.c_float(1), None) == 1
    assert L.mantleHipAttentionInnerQ8CacheF32(fake, fake, fake, fake, fake, fake, fake, 5, 0, 768, 96, 16, 8, 6,
                                               C.c_float(1), None) == 1
    # the reference signatures (softmax.h:70-104): no scratch argument
    assert L.mantleHipAttentionInnerF16CacheF32(fake, fake, fake, fake, 5, 6, 1024, 128, 16, 8, 0, C.c_float(1),
                                                None) == 1
    assert L.mantleHipAttentionInnerMixedCacheF32(fake, fake, fake, fake, fake, None, fake, fake, 1, 0, 5, 0, 1024, 128,
                                                  16, 8, 0, C.c_float(1), None) == 1  # q8_0 K without scales
    assert L.mantleHipApplyRoPEInplaceF32(None, fake, 3, C.c_float(1), 128, 64, 2, None) == 1
    assert L.mantleHipApplyRoPEInplaceF64FreqF32(fake, fake, 3, C.c_float(1), 128, 65, 2, None) == 1  # 2*half > hd
    assert L.mantleHipSetKVCacheType(3) == 1
    assert L.mantleHipSetKVCacheType(2) == 0 and L.mantleHipGetKVCacheType() == 2
    assert L.mantleHipSetKVCacheType(0) == 0
    assert L.mantleHipGetErrorString(1)


def test_model_load_errors_without_gpu(tmp_path):
    with pytest.raises(_lib.HipError):
        mantle_amd.new_backend("hip").load_model(str(tmp_path / "missing.mcf"))
    with pytest.raises(ValueError):
        mantle_amd.new_backend("cuda")
    assert mantle_amd.new_backend("HIP").name() == "hip"


def test_model_image_rejects_corrupt_bytes():
    with pytest.raises(_lib.HipError):
        mantle_amd.new_backend().load_model_image(b"MCF\0" + b"\0" * 100)


def test_bench_rejects_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "single-GPU" in r.stdout
