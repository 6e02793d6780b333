"""numpy restatement of zlm's decode-layer glue -- TEST INFRASTRUCTURE ONLY.

The ops between the GEMVs of one Qwen3 decode layer (reference
src/architectures/impl/qwen3/block.zig:20-41), used to check the HIP glue
kernels and the whole decode step.  Projections go through the C oracle's
production GEMV (``oracle.matvec``).  Only tests, ``smoke()`` and bench.py's
CPU leg import this module.
"""
from __future__ import annotations

import numpy as np

from oracle import matvec


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """rmsNorm (transformer/norm.zig:26-37): x * (1/sqrt(mean(x^2) + eps)) * w, f32."""
    x = np.asarray(x, np.float32)
    inv = np.float32(1.0) / np.sqrt(np.float32(np.mean(x.astype(np.float64) ** 2)) + np.float32(eps))
    return (x * inv * np.asarray(w, np.float32)).astype(np.float32)


def rope_half(head: np.ndarray, pos: int, freq_base: float) -> np.ndarray:
    """Rotate-half RoPE (rope.zig:4-33; frequencies as RopeTable, :46-104):
    inv_i = base^(-2i/hd), angle = pos*inv_i, (x_i, x_{i+hd/2}) ->
    (x_i c - x_{i+hd/2} s, x_i s + x_{i+hd/2} c).  The angle is formed as the
    reference forms it, in f32 (RopeTable.init's f32 pow, RopeTable.ensure's
    f32 product t * inv_freq[i]): at position 32767 that differs from the exact
    angle by up to ~2e-3 rad.  Its cos / sin and the rotation are float64."""
    head = np.asarray(head, np.float64)
    hd = head.size
    half = hd // 2
    fi = np.arange(half, dtype=np.float32)
    inv = np.power(np.float32(freq_base), np.float32(-2.0) * fi / np.float32(hd)).astype(np.float32)
    ang = (np.float32(pos) * inv).astype(np.float32).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = head[:half], head[half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c])


def write_kv(k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, pos: int) -> None:
    """writeKv (attention.zig:6-28): caches [n_kv][max_seq][hd] f16, row `pos` of each head."""
    n_kv, _, hd = k_cache.shape
    k_cache[:, pos, :] = np.asarray(k, np.float32).reshape(n_kv, hd).astype(np.float16)
    v_cache[:, pos, :] = np.asarray(v, np.float32).reshape(n_kv, hd).astype(np.float16)


def attend(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, n_heads: int, pos: int,
           scale: float) -> np.ndarray:
    """Attention of every q head over positions 0..pos (attention.zig:86-170,
    GQA kv_head = q_head / (n_heads / n_kv)): softmax(q.k * scale) . V, in
    float64 over the f16 cache values."""
    n_kv, _, hd = k_cache.shape
    group = n_heads // n_kv
    q = np.asarray(q, np.float64).reshape(n_heads, hd)
    out = np.zeros((n_heads, hd), np.float64)
    for h in range(n_heads):
        kh = h // group
        K = k_cache[kh, : pos + 1].astype(np.float64)
        V = v_cache[kh, : pos + 1].astype(np.float64)
        s = (K @ q[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V
    return out.reshape(-1)


def qk_norm_rope(qkv: np.ndarray, q_norm_w: np.ndarray, k_norm_w: np.ndarray, n_heads: int, n_kv: int, hd: int,
                 eps: float, freq_base: float, pos: int):
    """qkNormHeads (norm.zig:116-126) on q and k, then rope on each head
    (block.zig:24-29); returns (q, k, v) flat."""
    nq = n_heads * hd
    nk = n_kv * hd
    q = np.asarray(qkv[:nq], np.float32).reshape(n_heads, hd)
    k = np.asarray(qkv[nq:nq + nk], np.float32).reshape(n_kv, hd)
    v = np.asarray(qkv[nq + nk:nq + 2 * nk], np.float32)
    qo = np.concatenate([rope_half(rms_norm(q[h], q_norm_w, eps), pos, freq_base) for h in range(n_heads)])
    ko = np.concatenate([rope_half(rms_norm(k[h], k_norm_w, eps), pos, freq_base) for h in range(n_kv)])
    return qo.astype(np.float32), ko.astype(np.float32), v


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """ActivationKind.silu.apply (activation.zig:8-13) in float64."""
    g = np.asarray(g, np.float64)
    return (g / (1.0 + np.exp(-g))) * np.asarray(u, np.float64)


def decode_step(cfg, layers, out_norm, lm_head, lm_type, proj_type, x_in, pos, k_caches, v_caches, matvec=matvec):
    """One token through the Qwen3 layer sequence (block.zig:20-41) and the
    tail (:43-46).  `layers[i]` holds raw GGUF bytes 'qkv' (q;k;v rows), 'o',
    'gate', 'up', 'down' and f32 'attn_norm', 'ffn_norm', 'q_norm', 'k_norm'.
    Caches are updated in place.  Returns the logits (f32).  `matvec` is the
    production GEMV (the C oracle's, or its bit-identical pooled form for
    model-sized weights)."""
    hd, nh, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    h = np.asarray(x_in, np.float32).copy()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for i, L in enumerate(layers):
        n = rms_norm(h, L["attn_norm"], cfg.eps)
        qkv = matvec(proj_type, L["qkv"], cfg.hidden, (nh + 2 * nkv) * hd, n)
        q, k, v = qk_norm_rope(qkv, L["q_norm"], L["k_norm"], nh, nkv, hd, cfg.eps, cfg.freq_base, pos)
        write_kv(k, v, k_caches[i], v_caches[i], pos)
        att = attend(q, k_caches[i], v_caches[i], nh, pos, scale).astype(np.float32)
        h = (h + matvec(proj_type, L["o"], nh * hd, cfg.hidden, att)).astype(np.float32)
        n = rms_norm(h, L["ffn_norm"], cfg.eps)
        g = matvec(proj_type, L["gate"], cfg.hidden, cfg.ffn, n)
        u = matvec(proj_type, L["up"], cfg.hidden, cfg.ffn, n)
        mid = silu_mul(g, u).astype(np.float32)
        h = (h + matvec(proj_type, L["down"], cfg.ffn, cfg.hidden, mid)).astype(np.float32)
    n = rms_norm(h, out_norm, cfg.eps)
    return matvec(lm_type, lm_head, cfg.hidden, cfg.vocab, n)
