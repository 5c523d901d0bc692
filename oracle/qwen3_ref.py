"""numpy restatement of the int8 Qwen3-style decode step -- TEST INFRASTRUCTURE ONLY.

Follows the reference model structure (ip/models/qwen3_0_6b/architecture.py:
21-221: fused qkv with bias, rotate-half RoPE, GQA, pre-norm block, fused
gate_up + SwiGLU, lm_head, greedy argmax) at the BASELINE config-2 shape
(head_dim 128), with the reference's kernel defects fixed as documented in
mod_amd/csrc/decode.hip: causal attention over the cache, no dropped residual,
RoPE applied per head count.

Every linear is the W8 per-channel GEMV: y = s_w * (W_int8 @ x) (+ bias).
Computation runs in float64 (``dtype=np.float64``) or float32 for the
full-size config where float64 dequantized weights would not fit comfortably.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Qwen3Config:
    n_layers: int = 28
    hidden: int = 1024
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 3072
    vocab: int = 151936
    max_seq: int = 384
    rms_eps: float = 1e-6
    rope_theta: float = 10000.0
    kv_dtype: str = "float32"     # "float16": k and v rounded to fp16 (RNE) when cached


def _kv_round(v, cfg):
    """The value the KV cache holds: v itself, or v rounded to fp16."""
    return v.astype(np.float16).astype(v.dtype) if cfg.kv_dtype == "float16" else v


def rope_tables(cfg: Qwen3Config, dtype=np.float64):
    half = cfg.head_dim // 2
    j = np.arange(half, dtype=np.float64)
    inv = cfg.rope_theta ** (-(2 * j) / cfg.head_dim)
    ang = np.arange(cfg.max_seq, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(dtype), np.sin(ang).astype(dtype)


def _lin(x, W, s, b, dt):
    y = (W.astype(dt) @ x.astype(dt)) * s.astype(dt)
    if b is not None:
        y = y + b.astype(dt)
    return y


def _rms(x, w, eps, dt):
    x = x.astype(dt)
    return x * (1.0 / np.sqrt(np.mean(x * x) + eps)) * w.astype(dt)


def _rope(v, c, s):
    half = v.shape[-1] // 2
    r, im = v[..., :half], v[..., half:]
    return np.concatenate([r * c - im * s, r * s + im * c], axis=-1)


class Qwen3Ref:
    """Incremental decoder with a KV cache; step(id) returns the logits."""

    def __init__(self, cfg: Qwen3Config, w: dict, dtype=np.float64):
        self.cfg, self.w, self.dt = cfg, w, dtype
        self.cos, self.sin = rope_tables(cfg, dtype)
        L, nkv, D = cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
        self.kc = np.zeros((L, cfg.max_seq, nkv, D), dtype)
        self.vc = np.zeros((L, cfg.max_seq, nkv, D), dtype)
        self.pos = 0

    def step(self, tok: int) -> np.ndarray:
        c, w, dt, pos = self.cfg, self.w, self.dt, self.pos
        H, D, nq, nkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
        x = w["embed"][tok].astype(dt)
        for l, Lw in enumerate(w["layers"]):
            h = _rms(x, Lw["in_norm"], c.rms_eps, dt)
            qkv = _lin(h, Lw["w_qkv"], Lw["s_qkv"], Lw.get("b_qkv"), dt)
            q = qkv[: nq * D].reshape(nq, D)
            k = qkv[nq * D: (nq + nkv) * D].reshape(nkv, D)
            v = qkv[(nq + nkv) * D:].reshape(nkv, D)
            q = _rope(q, self.cos[pos], self.sin[pos])
            k = _rope(k, self.cos[pos], self.sin[pos])
            self.kc[l, pos] = _kv_round(k, c)
            self.vc[l, pos] = _kv_round(v, c)
            K = self.kc[l, : pos + 1]            # [t, nkv, D]
            V = self.vc[l, : pos + 1]
            grp = nq // nkv
            out = np.empty((nq, D), dt)
            for hh in range(nq):
                kv = hh // grp
                sc = (K[:, kv, :] @ q[hh]) / np.sqrt(D)
                p = np.exp(sc - sc.max())
                p = p / p.sum()
                out[hh] = p @ V[:, kv, :]
            x = x + _lin(out.reshape(-1), Lw["w_o"], Lw["s_o"], None, dt)
            h = _rms(x, Lw["post_norm"], c.rms_eps, dt)
            gu = _lin(h, Lw["w_gu"], Lw["s_gu"], None, dt)
            g, u = gu[: c.intermediate], gu[c.intermediate:]
            a = g / (1.0 + np.exp(-g)) * u
            x = x + _lin(a, Lw["w_down"], Lw["s_down"], None, dt)
        h = _rms(x, w["final_norm"], c.rms_eps, dt)
        logits = _lin(h, w["lm_head"], w["s_lm_head"], None, dt)
        self.pos += 1
        return logits


def forward_all(cfg: Qwen3Config, w: dict, ids, want, dtype=np.float64) -> np.ndarray:
    """Teacher-forced logits of a whole id sequence in one batched pass:
    position i sees ids[0..i] (causal attention), exactly the computation of
    Qwen3Ref.step at every position, done as matrix products over all
    positions at once. Returns the logits of the positions in `want`
    ([len(want), vocab]); pinned against step() in the oracle tests."""
    c, dt = cfg, dtype
    H, D, nq, nkv, I = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads, c.intermediate
    ids = np.asarray(ids)
    T = len(ids)
    cos, sin = rope_tables(c, dt)
    cos, sin = cos[:T][:, None, :], sin[:T][:, None, :]
    causal = np.triu(np.ones((T, T), bool), 1)

    def lin(x, W, s, b):
        y = (x @ W.astype(dt).T) * s.astype(dt)
        return y if b is None else y + b.astype(dt)

    def rms(x, g):
        return x * (1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + c.rms_eps)) * g.astype(dt)

    x = w["embed"][ids].astype(dt)
    grp = nq // nkv
    for Lw in w["layers"]:
        qkv = lin(rms(x, Lw["in_norm"]), Lw["w_qkv"], Lw["s_qkv"], Lw.get("b_qkv"))
        q = _rope(qkv[:, : nq * D].reshape(T, nq, D), cos, sin)
        k = _kv_round(_rope(qkv[:, nq * D: (nq + nkv) * D].reshape(T, nkv, D), cos, sin), c)
        v = _kv_round(qkv[:, (nq + nkv) * D:].reshape(T, nkv, D), c)
        out = np.empty((T, nq, D), dt)
        for hh in range(nq):
            kv = hh // grp
            sc = (q[:, hh, :] @ k[:, kv, :].T) / np.sqrt(D)
            sc[causal] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p = p / p.sum(axis=1, keepdims=True)
            out[:, hh, :] = p @ v[:, kv, :]
        x = x + lin(out.reshape(T, nq * D), Lw["w_o"], Lw["s_o"], None)
        gu = lin(rms(x, Lw["post_norm"]), Lw["w_gu"], Lw["s_gu"], None)
        g, u = gu[:, :I], gu[:, I:]
        x = x + lin(g / (1.0 + np.exp(-g)) * u, Lw["w_down"], Lw["s_down"], None)
    h = rms(x[np.asarray(want)], w["final_norm"])
    return lin(h, w["lm_head"], w["s_lm_head"], None)


def greedy(cfg: Qwen3Config, w: dict, prompt, n_new: int, dtype=np.float64):
    """Greedy decode: returns (ids, logits of every step)."""
    ref = Qwen3Ref(cfg, w, dtype)
    ids = list(prompt)
    all_logits = []
    for pos in range(len(prompt) + n_new - 1):
        lg = ref.step(ids[pos])
        all_logits.append(lg)
        if pos + 1 >= len(prompt):
            ids.append(int(np.argmax(lg)))
    return ids, all_logits
