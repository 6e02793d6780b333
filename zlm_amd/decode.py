"""Batch-1 decode step of a Qwen3-shaped model on the HIP backend, activations
resident in HBM from the token's embedding row to the logits.

The layer sequence is the reference's Qwen3 block (reference
src/architectures/impl/qwen3/block.zig:20-41, tail :43-46); every projection
runs through this backend's GEMV kernels, fused where the sequence allows:

    h <- x_in                                        (the token's embedding row)
    per layer:
      qkv  = W_qkv . RMSNorm(h, attn_norm)           GEMV, norm form (q;k;v rows)
      attn = attention(RoPE(RMSNorm_head(q)), K, V)  q/k head norm + RoPE, K/V append
                                                     at pos and split-K attention in
                                                     one launch, the merge in a second
      h    = h + W_o . attn                          GEMV, residual form
      mid  = silu(W_gate . n) * (W_up . n),  n = RMSNorm(h, ffn_norm)
                                                     GEMV, normed gate_up form
      h    = h + W_down . mid                        GEMV, residual form
    logits = W_lm . RMSNorm(h, out_norm)             GEMV, norm form

The q, k and v projections are one resident (their rows concatenated), the
layout this backend keeps in HBM for one launch instead of three.  The
position lives in device memory, so a step captured once into a HIP graph
replays for any position.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from zlm_amd import device as zd


@dataclass(frozen=True)
class DecodeConfig:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq: int
    eps: float = 1e-6
    freq_base: float = 1_000_000.0
    proj_type: int = zd.Q4_0
    lm_type: int = zd.Q8_0

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


# Qwen3-8B shapes, Q4_0 projections, Q8_0 lm_head, fp16 KV of 2048.
QWEN3_8B = DecodeConfig(n_layers=36, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288,
                        vocab=151936, max_seq=2048)

_BLOCK = {zd.Q4_0: (32, 18), zd.Q8_0: (32, 34)}


def weight_bytes(cfg: DecodeConfig) -> int:
    """Bytes of every weight a step streams (GGUF block bytes)."""
    pe, pb = _BLOCK[cfg.proj_type]
    le, lb = _BLOCK[cfg.lm_type]
    per_layer = (cfg.qkv_rows * cfg.hidden + cfg.hidden * cfg.n_heads * cfg.head_dim + 2 * cfg.ffn * cfg.hidden
                 + cfg.hidden * cfg.ffn) // pe * pb
    return cfg.n_layers * per_layer + cfg.vocab * cfg.hidden // le * lb


def kv_bytes(cfg: DecodeConfig, context: int) -> int:
    """K and V bytes attention reads at `context` positions (fp16)."""
    return cfg.n_layers * 2 * cfg.n_kv_heads * context * cfg.head_dim * 2


@dataclass
class _Layer:
    qkv: zd.Resident
    o: zd.Resident
    gate: zd.Resident
    up: zd.Resident
    down: zd.Resident
    attn_norm: int
    ffn_norm: int
    q_norm: int
    k_norm: int
    k_cache: int
    v_cache: int


class DecodeModel:
    """Weights, KV caches and activation buffers of one model in HBM.

    ``host`` (optional) gives the weights as raw GGUF bytes and f32 norm
    vectors, per layer: 'qkv', 'o', 'gate', 'up', 'down', 'attn_norm',
    'ffn_norm', 'q_norm', 'k_norm', and optionally the f16 caches 'k_cache' /
    'v_cache' ([n_kv_heads][max_seq][head_dim], zeros when absent); plus
    'lm_head' and 'out_norm'.  Without it
    the projections are synthesised in HBM (q4_0 scales |N(0,1)|*0.02, q8_0
    |N(0,1)|*0.01) and the norm weights are 1 + 0.1 N(0,1)."""

    def __init__(self, dev: zd.Device, cfg: DecodeConfig, host: Optional[dict] = None, seed: int = 0x5A4C4D02):
        if not dev.available():
            raise RuntimeError("decode needs an available HIP device")
        self.dev, self.cfg = dev, cfg
        self._owned: list[int] = []
        self._res: list[zd.Resident] = []
        rng = np.random.default_rng(seed)
        c = cfg

        def vec(a: np.ndarray) -> int:
            a = np.ascontiguousarray(a, np.float32)
            p = dev.dev_malloc(max(16, a.nbytes))
            dev.dev_upload(p, a)
            self._owned.append(p)
            return p

        def buf(nbytes: int) -> int:
            p = dev.dev_malloc(max(16, nbytes))
            self._owned.append(p)
            return p

        def res(name: str, rows: int, k: int, qtype: int, layer: Optional[dict], salt: int) -> zd.Resident:
            if layer is not None:
                r = dev.upload_resident(layer[name])
            else:
                be, _ = _BLOCK[qtype]
                scale = 0.02 if qtype == zd.Q4_0 else 0.01
                r = dev.synth_resident(qtype, rows * k // be, seed * 1315423911 + salt, scale)
            if r is None:
                raise RuntimeError(f"resident {name}: {dev.last_error()}")
            self._res.append(r)
            return r

        def norm(layer: Optional[dict], name: str, n: int) -> int:
            if layer is not None:
                return vec(layer[name])
            return vec(1.0 + 0.1 * rng.standard_normal(n))

        self.layers: list[_Layer] = []
        cache_elems = c.n_kv_heads * c.max_seq * c.head_dim
        for i in range(c.n_layers):
            L = host["layers"][i] if host else None
            s = 16 * (i + 1)
            kc, vc = buf(cache_elems * 2), buf(cache_elems * 2)
            if host is None:  # a history in the caches, as after `context` earlier tokens
                dev.synth_f16(kc, cache_elems, seed + s + 7, 1.0)
                dev.synth_f16(vc, cache_elems, seed + s + 8, 1.0)
            else:
                for cache, name in ((kc, "k_cache"), (vc, "v_cache")):
                    hist = L.get(name)
                    if hist is None:
                        hist = np.zeros(cache_elems, np.float16)
                    elif hist.dtype != np.float16 or hist.size != cache_elems:
                        raise ValueError(f"layer {i} {name}: {cache_elems} f16 values expected")
                    dev.dev_upload(cache, np.ascontiguousarray(hist).reshape(-1))
            self.layers.append(_Layer(
                qkv=res("qkv", c.qkv_rows, c.hidden, c.proj_type, L, s + 1),
                o=res("o", c.hidden, c.n_heads * c.head_dim, c.proj_type, L, s + 2),
                gate=res("gate", c.ffn, c.hidden, c.proj_type, L, s + 3),
                up=res("up", c.ffn, c.hidden, c.proj_type, L, s + 4),
                down=res("down", c.hidden, c.ffn, c.proj_type, L, s + 5),
                attn_norm=norm(L, "attn_norm", c.hidden), ffn_norm=norm(L, "ffn_norm", c.hidden),
                q_norm=norm(L, "q_norm", c.head_dim), k_norm=norm(L, "k_norm", c.head_dim),
                k_cache=kc, v_cache=vc))
        self.lm_head = res("lm_head", c.vocab, c.hidden, c.lm_type, host, 3)
        self.out_norm = norm(host, "out_norm", c.hidden)
        self.x_in = buf(c.hidden * 4)
        self.h = buf(c.hidden * 4)
        self.qkv = buf(c.qkv_rows * 4)
        self.attn = buf(c.n_heads * c.head_dim * 4)
        self.mid = buf(c.ffn * 4)
        self.logits = buf(c.vocab * 4)
        self.pos = buf(16)
        self.scale = 1.0 / math.sqrt(c.head_dim)

    def host_copy(self) -> dict:
        """The model's weights, norms and caches as host arrays, in the `host`
        format the constructor takes (raw GGUF bytes, f32 norms, f16 caches
        [n_kv_heads][max_seq][head_dim]); for checking a model synthesised in
        HBM against the CPU kernels.  Only before the first step (a resident's
        first op converts its raw bytes to the device layout)."""
        d, c = self.dev, self.cfg

        def f32(p: int, n: int) -> np.ndarray:
            out = np.empty(n, np.float32)
            d.dev_download(out, p)
            return out

        def f16(p: int) -> np.ndarray:
            out = np.empty((c.n_kv_heads, c.max_seq, c.head_dim), np.float16)
            d.dev_download(out, p)
            return out

        layers = []
        for L in self.layers:
            layers.append({
                "qkv": d.resident_read_raw(L.qkv), "o": d.resident_read_raw(L.o),
                "gate": d.resident_read_raw(L.gate), "up": d.resident_read_raw(L.up),
                "down": d.resident_read_raw(L.down),
                "attn_norm": f32(L.attn_norm, c.hidden), "ffn_norm": f32(L.ffn_norm, c.hidden),
                "q_norm": f32(L.q_norm, c.head_dim), "k_norm": f32(L.k_norm, c.head_dim),
                "k_cache": f16(L.k_cache), "v_cache": f16(L.v_cache)})
        return {"layers": layers, "lm_head": d.resident_read_raw(self.lm_head),
                "out_norm": f32(self.out_norm, c.hidden)}

    # -- one step --------------------------------------------------------------
    def window_for(self, pos: int) -> int:
        """The attention window a step at `pos` needs: the smallest power of
        two >= pos + 1 (at least 128), capped at max_seq."""
        w = 128
        while w < pos + 1:
            w *= 2
        return min(w, self.cfg.max_seq)

    def enqueue_step(self, window: Optional[int] = None) -> None:
        """Enqueue one token's step on the device stream (no waits).  The
        attention reads positions [0, window) of the caches (default: all of
        them); the step's position must be below the window."""
        d, c = self.dev, self.cfg
        window = c.max_seq if window is None else window
        q, lm = zd.quant(c.proj_type), zd.quant(c.lm_type)

        def ok(flag: bool, what: str) -> None:
            if not flag:
                raise RuntimeError(f"{what}: {d.last_error()}")

        ok(d.dev_copy_enqueue(self.h, self.x_in, c.hidden * 4), "embed")
        for L in self.layers:
            ok(d.gemv_op_enqueue(zd.FORM_NORM, q, L.qkv, c.qkv_rows, c.hidden, self.h, self.qkv,
                                 norm_w=L.attn_norm, eps=c.eps), "qkv")
            ok(d.attention_decode_window_enqueue(self.qkv, L.q_norm, L.k_norm, c.n_heads, c.n_kv_heads,
                                                 c.head_dim, c.eps, c.freq_base, self.pos, L.k_cache, L.v_cache,
                                                 c.max_seq, window, self.scale, self.attn), "attention")
            ok(d.gemv_op_enqueue(zd.FORM_RESID, q, L.o, c.hidden, c.n_heads * c.head_dim, self.attn, self.h,
                                 res=self.h), "o")
            ok(d.gemv_op_enqueue(zd.FORM_NORMPAIR, q, L.gate, c.ffn, c.hidden, self.h, self.mid, w_up=L.up,
                                 norm_w=L.ffn_norm, eps=c.eps, act=zd.SILU), "gate_up")
            ok(d.gemv_op_enqueue(zd.FORM_RESID, q, L.down, c.hidden, c.ffn, self.mid, self.h, res=self.h), "down")
        ok(d.gemv_op_enqueue(zd.FORM_NORM, lm, self.lm_head, c.vocab, c.hidden, self.h, self.logits,
                             norm_w=self.out_norm, eps=c.eps), "lm_head")

    def set_input(self, x_in: np.ndarray, pos: int) -> None:
        self.dev.dev_upload(self.x_in, np.ascontiguousarray(x_in, np.float32))
        self.dev.dev_upload(self.pos, np.array([pos, 0, 0, 0], np.int32))

    def step(self, x_in: np.ndarray, pos: int, window: Optional[int] = None) -> np.ndarray:
        """One eager step for token row `x_in` at `pos` (attention window:
        default all of the caches); returns the logits."""
        self.set_input(x_in, pos)
        self.enqueue_step(window)
        out = np.zeros(self.cfg.vocab, np.float32)
        self.dev.dev_download(out, self.logits)
        return out

    def logits_host(self) -> np.ndarray:
        out = np.zeros(self.cfg.vocab, np.float32)
        self.dev.dev_download(out, self.logits)
        return out

    def capture(self, window: Optional[int] = None) -> int:
        """Record one step into a HIP graph (run a step eagerly first so every
        layout and scratch buffer exists).  A serving loop captures one graph
        per window bucket (window_for) and replays the one for each position,
        so a step reads only the KV it needs."""
        if not self.dev.capture_begin():
            raise RuntimeError(self.dev.last_error())
        try:
            self.enqueue_step(window)
        finally:
            g = self.dev.capture_end()
        if g is None:
            raise RuntimeError(f"capture failed: {self.dev.last_error()}")
        return g

    def free(self) -> None:
        for r in self._res:
            self.dev.free_resident(r)
        for p in self._owned:
            self.dev.dev_free(p)
        self._res, self._owned = [], []
