"""Pins the oracle's Qwen3 decode wiring (layer order, GQA head map, q/k norm,
RoPE, KV cache, tied lm_head) against an independent float64 forward pass over
the same dequantised weights.  The oracle quantises activations to int8 per
32-block (Mantle's W4A8), so agreement is to a tolerance, not bit-exact."""
import numpy as np

from oracle import oracle as o
from tests import models


def _f64_forward(f, cfg, tokens):
    from mantle_amd.mcf import DTYPE_F32
    L, d, nh, kvh, hd = cfg["n_layers"], cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    eps = cfg["eps"]

    def t(name):
        info = f.tensors[name]
        raw = f.raw(name)
        if info["dtype"] == DTYPE_F32:
            return raw.view(np.float32).astype(np.float64)
        r, c = info["shape"]
        return o.dequant_k4(raw, r, c).astype(np.float64)

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * g

    emb = t("model.embed_tokens.weight")
    W = [{k: t(f"model.layers.{l}.{k}") for k in (
        "input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
        "self_attn.k_norm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")}
         for l in range(L)]
    fnorm = t("model.norm.weight")
    inv = 1.0 / (cfg["rope_base"] ** (np.arange(hd // 2) * 2.0 / hd))
    K = [[] for _ in range(L)]
    V = [[] for _ in range(L)]
    out = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        c, s = np.cos(pos * inv), np.sin(pos * inv)

        def rope(v):
            lo, hi = v[:hd // 2].copy(), v[hd // 2:].copy()
            return np.concatenate([lo * c - hi * s, lo * s + hi * c])

        for l in range(L):
            w = W[l]
            h = rms(x, w["input_layernorm.weight"])
            q = (w["self_attn.q_proj.weight"] @ h).reshape(nh, hd)
            k = (w["self_attn.k_proj.weight"] @ h).reshape(kvh, hd)
            v = (w["self_attn.v_proj.weight"] @ h).reshape(kvh, hd)
            q = np.array([rope(rms(qq, w["self_attn.q_norm.weight"])) for qq in q])
            k = np.array([rope(rms(kk, w["self_attn.k_norm.weight"])) for kk in k])
            K[l].append(k)
            V[l].append(v)
            ks, vs = np.array(K[l]), np.array(V[l])
            a = np.zeros((nh, hd))
            for hh in range(nh):
                g = hh * kvh // nh
                sc = ks[:, g] @ q[hh] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                a[hh] = (p / p.sum()) @ vs[:, g]
            x = x + w["self_attn.o_proj.weight"] @ a.reshape(-1)
            h2 = rms(x, w["post_attention_layernorm.weight"])
            gt = w["mlp.gate_proj.weight"] @ h2
            up = w["mlp.up_proj.weight"] @ h2
            x = x + w["mlp.down_proj.weight"] @ (gt / (1 + np.exp(-gt)) * up)
        out.append(emb @ rms(x, fnorm))
    return out


def test_oracle_model_matches_float64_forward(tmp_path):
    from mantle_amd.mcf import MCFFile
    cfg = dict(models.TINY)
    path = models.pack(str(tmp_path / "tiny.mcf"), 3, cfg)
    tokens = models.prompt(12, cfg["vocab"], 4)
    m = models.oracle_model(path, cfg, 32)
    got = [m.forward_greedy(t, want_logits=True)[1] for t in tokens]
    m.close()
    with MCFFile(path) as f:
        want = _f64_forward(f, cfg, tokens)
    for step, (g, w) in enumerate(zip(got, want)):
        rel = np.linalg.norm(g - w) / np.linalg.norm(w)
        assert rel < 2e-2, (step, rel)
        assert np.corrcoef(g, w)[0, 1] > 0.999


def test_oracle_model_reset_replays_identically(tmp_path):
    cfg = dict(models.TINY)
    path = models.pack(str(tmp_path / "tiny.mcf"), 5, cfg)
    m = models.oracle_model(path, cfg, 32)
    a = m.generate_greedy([1, 2, 3], 8)
    m.reset()
    b = m.generate_greedy([1, 2, 3], 8)
    m.close()
    assert a == b
