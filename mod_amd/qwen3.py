"""Host side of the int8 Qwen3-style decoder (BASELINE config 2 shape).

``Qwen3Int8Decoder`` uploads int8 weights (numpy) into library-owned HBM
tensors and drives the native decoder (pio_qwen3_* in libtensor_ops_rocm.so).
Three ways to run steps, sharing one KV cache and position:
  "eager"       the step's kernels launched one by one,
  "graph"       one device-driven step captured once as a HIP graph and
                replayed per token,
  "persistent"  every step of the call in one kernel launch (Qwen3-0.6B
                layer shape only; see ``persistent_supported``).
Replaces Qwen3ForCausalLM.generate (ip/models/qwen3_0_6b/architecture.py:
183-221), whose loop makes ~30 ctypes calls and allocations per layer per token.
"""
from __future__ import annotations

import ctypes
from dataclasses import asdict, dataclass
from typing import Dict, List, Optional

import numpy as np

from . import ops
from .backend import Tensor
from .ops import RocmError, check, lib


@dataclass
class Qwen3Config:
    """Defaults = BASELINE config 2 (Qwen3-0.6B shape, head_dim 128)."""
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
    kv_dtype: str = "float32"     # KV cache element type: "float32" or "float16"

    def weight_bytes(self) -> Dict[str, int]:
        """Int8 weight and fp32 scale bytes streamed per decode token."""
        H, D, I = self.hidden, self.head_dim, self.intermediate
        nqkv = (self.n_heads + 2 * self.n_kv_heads) * D
        per_layer = nqkv * H + H * self.n_heads * D + 2 * I * H + H * I
        scales_layer = 4 * (nqkv + H + 2 * I + H)
        return {
            "int8": self.n_layers * per_layer + self.vocab * H,
            "scales": self.n_layers * scales_layer + 4 * self.vocab,
            "bias_norms": self.n_layers * 4 * (nqkv + 2 * H) + 4 * H,
        }

    def kv_bytes_per_pos(self) -> int:
        """K and V bytes read per cached position per token."""
        return self.n_layers * 2 * self.n_kv_heads * self.head_dim * (2 if self.kv_dtype == "float16" else 4)


class _CConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                              "head_dim", "intermediate", "vocab", "max_seq")] + \
               [("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("kv_dtype", ctypes.c_int)]


_KV_CODES = {"float32": 0, "float16": 1}


class _CLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("in_norm", "w_qkv", "s_qkv", "b_qkv", "w_o", "s_o",
                                                 "post_norm", "w_gu", "s_gu", "w_down", "s_down")]


LAYER_KEYS = ("in_norm", "w_qkv", "s_qkv", "b_qkv", "w_o", "s_o", "post_norm", "w_gu", "s_gu",
              "w_down", "s_down")


def random_weights(cfg: Qwen3Config, seed: int = 0, qkv_bias: bool = True) -> dict:
    """Random-init int8 weights of the config's architecture (numpy, host).
    int8 weights ~ randint(-127, 127); scales ~ U(0.001, 0.02) scaled by
    1/sqrt(K/1024) so activations stay O(1) through the layers; norms ~ 1."""
    rng = np.random.default_rng(seed)
    H, D, I, V = cfg.hidden, cfg.head_dim, cfg.intermediate, cfg.vocab
    nqkv = (cfg.n_heads + 2 * cfg.n_kv_heads) * D

    def lin(n, k):
        w = rng.integers(-127, 127, size=(n, k), dtype=np.int8)
        s = (rng.uniform(0.001, 0.02, size=n) * np.sqrt(1024.0 / k) * 0.1).astype(np.float32)
        return w, s

    layers = []
    for _ in range(cfg.n_layers):
        L = {}
        L["in_norm"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        L["w_qkv"], L["s_qkv"] = lin(nqkv, H)
        L["b_qkv"] = (0.1 * rng.standard_normal(nqkv)).astype(np.float32) if qkv_bias else None
        L["w_o"], L["s_o"] = lin(H, cfg.n_heads * D)
        L["post_norm"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        L["w_gu"], L["s_gu"] = lin(2 * I, H)
        L["w_down"], L["s_down"] = lin(H, I)
        layers.append(L)
    embed = rng.standard_normal((V, H), dtype=np.float32)
    lm, s_lm = lin(V, H)
    return {"embed": embed, "final_norm": np.ones(H, np.float32), "lm_head": lm,
            "s_lm_head": (s_lm * 10).astype(np.float32), "layers": layers}


def _hf(i: int, leaf: str) -> str:
    return f"model.layers.{i}.{leaf}"


def weights_from_checkpoint(path, cfg: Qwen3Config, device: str = "rocm:0",
                            strict: bool = True) -> dict:
    """Decoder weights from a safetensors checkpoint under the Hugging Face
    Qwen names (``model.layers.{i}.self_attn.q_proj.weight`` ...), as device
    tensors for ``Qwen3Int8Decoder``.

    Each linear is read either in the int8 format (I8 ``.weight`` plus F32
    ``.weight_scale``) or as F32 / F16 / BF16 and quantized per output channel
    on the GPU. q/k/v and gate/up are fused by stacking rows (q, k, v; gate,
    up), or read fused from ``qkv_proj`` / ``gate_up_proj`` (the reference
    layout, ip/models/qwen3_0_6b/architecture.py:24,47). Per-channel scales make
    stacking rows before or after quantization give the same int8 weights.
    ``lm_head`` falls back to the embedding (tied weights). With ``strict``,
    a checkpoint tensor the decoder has no place for (e.g. per-head q/k norms,
    which this decoder does not apply) is an error rather than silently unused.
    """
    from .weights import Checkpoint, FLOAT_DTYPES, SCALE_SUFFIX, quantize_rows

    H, D, I, V = cfg.hidden, cfg.head_dim, cfg.intermediate, cfg.vocab
    nq, nkv = cfg.n_heads * D, cfg.n_kv_heads * D
    used = set()

    with Checkpoint(path) as ck:
        def need(name):
            if name not in ck:
                raise RocmError(f"checkpoint lacks '{name}'")
            used.add(name)
            return name

        def vec(name, n):
            inf = ck.info(need(name))
            if inf.shape != (n,):
                raise RocmError(f"{name}: shape {inf.shape}, expected ({n},)")
            t = Tensor([n], device=device)
            ck.load_into(name, t)
            return t

        def linear(blocks, k):
            """blocks: [(name, rows)] stacked in order -> (int8 [sum rows, k], fp32 scales).
            Each block lands in its row slice of the device tensors."""
            infos = [(n, ck.info(need(n)), r) for n, r in blocks]
            for n, inf, r in infos:
                if inf.shape != (r, k):
                    raise RocmError(f"{n}: shape {inf.shape}, expected ({r}, {k})")
            rows = sum(r for _, r in blocks)
            kinds = {inf.dtype in FLOAT_DTYPES for _, inf, _ in infos}
            if len(kinds) != 1:
                raise RocmError(f"{[n for n, _ in blocks]}: mixed int8 and fp storage")
            q = Tensor([rows, k], device=device, dtype="int8")
            s = Tensor([rows], device=device)
            if kinds == {True}:
                w = Tensor([rows, k], device=device)
                off = 0
                for n, _, r in infos:
                    ck.to_device_f32(n, w.data_ptr() + 4 * off * k, r * k)
                    off += r
                quantize_rows(w, q, s)
                return q, s
            off = 0
            for n, inf, r in infos:
                if inf.dtype != "I8":
                    raise RocmError(f"{n}: stored {inf.dtype}, expected I8 or fp")
                sn = need(n + SCALE_SUFFIX)
                if ck.info(sn).shape != (r,):
                    raise RocmError(f"{sn}: shape {ck.info(sn).shape}, expected ({r},)")
                ck.to_device(n, q.data_ptr() + off * k, r * k)
                ck.to_device_f32(sn, s.data_ptr() + 4 * off, r)
                off += r
            return q, s

        def fused_or_split(fused, split, k):
            if fused in ck:
                return linear([(fused, sum(r for _, r in split))], k)
            return linear(split, k)

        def bias(fused, split):
            if fused in ck:
                return vec(fused, sum(r for _, r in split))
            present = [n in ck for n, _ in split]
            if not any(present):
                return None
            if not all(present):
                raise RocmError(f"only some of {[n for n, _ in split]} are present")
            t = Tensor([sum(r for _, r in split)], device=device)
            off = 0
            for n, r in split:
                if ck.info(need(n)).shape != (r,):
                    raise RocmError(f"{n}: shape {ck.info(n).shape}, expected ({r},)")
                ck.to_device_f32(n, t.data_ptr() + 4 * off, r)
                off += r
            return t

        layers = []
        for i in range(cfg.n_layers):
            L = {}
            L["in_norm"] = vec(_hf(i, "input_layernorm.weight"), H)
            L["post_norm"] = vec(_hf(i, "post_attention_layernorm.weight"), H)
            qkv = [(_hf(i, f"self_attn.{p}_proj.weight"), r) for p, r in (("q", nq), ("k", nkv),
                                                                           ("v", nkv))]
            L["w_qkv"], L["s_qkv"] = fused_or_split(_hf(i, "self_attn.qkv_proj.weight"), qkv, H)
            L["b_qkv"] = bias(_hf(i, "self_attn.qkv_proj.bias"),
                              [(n[:-len("weight")] + "bias", r) for n, r in qkv])
            L["w_o"], L["s_o"] = linear([(_hf(i, "self_attn.o_proj.weight"), H)], nq)
            gu = [(_hf(i, "mlp.gate_proj.weight"), I), (_hf(i, "mlp.up_proj.weight"), I)]
            L["w_gu"], L["s_gu"] = fused_or_split(_hf(i, "mlp.gate_up_proj.weight"), gu, H)
            L["w_down"], L["s_down"] = linear([(_hf(i, "mlp.down_proj.weight"), H)], I)
            layers.append(L)
        emb_name = need("model.embed_tokens.weight")
        if ck.info(emb_name).shape != (V, H):
            raise RocmError(f"{emb_name}: shape {ck.info(emb_name).shape}, expected ({V}, {H})")
        embed = Tensor([V, H], device=device)
        ck.load_into(emb_name, embed)
        lm_name = "lm_head.weight" if "lm_head.weight" in ck else emb_name
        lm, s_lm = linear([(lm_name, V)], H)
        final = vec("model.norm.weight", H)
        if strict:
            extra = sorted(set(ck.names()) - used)
            if extra:
                raise RocmError(f"checkpoint tensors this decoder does not use: {extra[:8]}"
                                + (" ..." if len(extra) > 8 else ""))
    return {"embed": embed, "final_norm": final, "lm_head": lm, "s_lm_head": s_lm,
            "layers": layers}


MODES = {"eager": 0, "graph": 1, "persistent": 2}


def _mode(use_graph, mode) -> int:
    if mode is None:
        mode = "graph" if use_graph else "eager"
    if mode not in MODES:
        raise ValueError(f"unknown decode mode {mode!r}; one of {sorted(MODES)}")
    return MODES[mode]


class Qwen3Int8Decoder:
    """Native greedy decoder over library-owned device weights."""

    def __init__(self, cfg: Qwen3Config, weights: dict, device: str = "rocm:0",
                 stream: Optional[int] = None):
        self.cfg = cfg
        self._keep: List[Tensor] = []

        def up(a):
            if a is None:
                return None
            if isinstance(a, Tensor):   # already on the device (checkpoint loads)
                self._keep.append(a)
                return a.data_ptr()
            t = Tensor.from_numpy(np.ascontiguousarray(a), device)
            self._keep.append(t)
            return t.data_ptr()

        self._embed = up(weights["embed"])
        self._final = up(weights["final_norm"])
        self._lm = up(weights["lm_head"])
        self._slm = up(weights["s_lm_head"])
        layers = (_CLayer * cfg.n_layers)()
        for i, L in enumerate(weights["layers"]):
            for k in LAYER_KEYS:
                setattr(layers[i], k, up(L.get(k)))
        if cfg.kv_dtype not in _KV_CODES:
            raise ValueError(f"kv_dtype must be one of {sorted(_KV_CODES)}, not {cfg.kv_dtype!r}")
        fields = asdict(cfg)
        fields["kv_dtype"] = _KV_CODES[cfg.kv_dtype]
        c = _CConfig(**fields)
        self._cfg_c, self._layers_c = c, layers
        self._h = lib.pio_qwen3_create(ctypes.addressof(c), self._embed, self._final, self._lm,
                                       self._slm, ctypes.addressof(layers), stream)
        if not self._h:
            raise RocmError(f"pio_qwen3_create failed: {ops.last_error()}")
        self.prompt_len = 0

    def close(self):
        if getattr(self, "_h", None):
            lib.pio_qwen3_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def reset(self, ids) -> None:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib.pio_qwen3_reset(self._h, ids.ctypes.data, ids.size), "pio_qwen3_reset")
        self.prompt_len = int(ids.size)

    def persistent_supported(self) -> bool:
        """Whether the "persistent" mode runs this config on this device."""
        return bool(lib.pio_qwen3_persistent_supported(self._h))

    def prefill(self, n_steps: int, logits: bool = False) -> None:
        """The next n_steps prompt positions in one batched pass (the int8
        linears over all rows at once on the matrix cores); with logits, the
        last position's logits and next id as its step would give them."""
        check(lib.pio_qwen3_prefill(self._h, n_steps, int(logits)), "pio_qwen3_prefill")

    def trace_next(self, first_step: int) -> None:
        """The next persistent run is traced: phase stamps of its steps
        first_step and first_step + 1 (see phase_trace)."""
        check(lib.pio_qwen3_trace_next(self._h, first_step), "pio_qwen3_trace_next")

    def phase_trace(self) -> np.ndarray:
        """Stamps of the last traced run, in ns relative to the earliest
        one: float64 [2 steps][256 workgroups][n_layers + 1][16 slots], NaN
        where a slot was not reached (the slot meanings are in tensor_rocm.h)."""
        nb = int(lib.pio_qwen3_trace_bytes(self._h))
        raw = np.zeros(nb // 8, np.uint64)
        check(lib.pio_qwen3_trace_read(self._h, raw.ctypes.data, nb), "pio_qwen3_trace_read")
        raw = raw.reshape(2, 256, self.cfg.n_layers + 1, -1)
        t = raw.astype(np.float64)
        t[raw == 0] = np.nan
        return (t - np.nanmin(t)) * 10.0   # 100 MHz ticks -> ns

    def refresh_weights(self) -> None:
        """The persistent mode's copy of the int8 layer weights, taken again
        from the buffers this decoder was created with (after changing them
        in place)."""
        check(lib.pio_qwen3_refresh_weights(self._h), "pio_qwen3_refresh_weights")

    def persistent_replays(self) -> int:
        """Persistent launches re-run in graph mode because the device could
        not hold their whole grid at once (other work held CUs)."""
        return int(lib.pio_qwen3_persistent_replays(self._h))

    def run(self, n_steps: int, use_graph: bool = True, mode: Optional[str] = None) -> None:
        check(lib.pio_qwen3_run(self._h, n_steps, _mode(use_graph, mode)), "pio_qwen3_run")

    def read(self, n: int, with_logits: bool = False):
        ids = np.zeros(n, np.int32)
        logits = np.empty(self.cfg.vocab, np.float32) if with_logits else None
        check(lib.pio_qwen3_read(self._h, ids.ctypes.data, n,
                                 None if logits is None else logits.ctypes.data),
              "pio_qwen3_read")
        return (ids, logits) if with_logits else ids

    def generate(self, prompt, n_new: int, use_graph: bool = True,
                 mode: Optional[str] = None) -> np.ndarray:
        """Greedy decode: prompt (P ids) -> P + n_new ids. The prompt is consumed
        one position per step (P-1 steps), then n_new steps generate."""
        self.reset(prompt)
        P = len(prompt)
        self.run(P - 1 + n_new, use_graph, mode)
        return self.read(P + n_new)

    def teacher_forced_logits(self, ids, use_graph: bool = False,
                              mode: Optional[str] = None) -> np.ndarray:
        """Logits after each position of a fixed id sequence ([len-1, vocab])."""
        self.reset(ids)
        out = []
        for _ in range(len(ids) - 1):
            self.run(1, use_graph, mode)
            out.append(self.read(0, with_logits=True)[1].copy())
        return np.stack(out)


def _main(argv=None) -> int:
    """Runs the config-2 decode workload once and exits: random-init weights
    (seed 0), a random 128-token prompt (seed 1) as one batch, then `--steps`
    generated tokens in the fastest supported mode -- the same launches as
    bench.py's timed decode (a warmup generation of `--warmup` tokens, then the
    batched prompt and the generated steps), as a plain driver for profilers
    (rocprofv3 counter passes). In persistent mode the second decode launch
    is the one that runs the `--steps` tokens."""
    import argparse
    ap = argparse.ArgumentParser(prog="python -m mod_amd.qwen3")
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--mode", choices=sorted(MODES), default=None)
    args = ap.parse_args(argv)
    P = 128
    cfg = Qwen3Config(max_seq=max(384, P + args.steps))
    dec = Qwen3Int8Decoder(cfg, random_weights(cfg, seed=0))
    mode = args.mode or ("persistent" if dec.persistent_supported() else "graph")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=P).astype(np.int32)
    dec.reset(prompt)
    dec.prefill(P - 1)
    dec.run(min(max(args.warmup, 1), cfg.max_seq - P + 1), mode=mode)
    dec.reset(prompt)
    dec.prefill(P - 1)
    dec.run(args.steps, mode=mode)
    ids = dec.read(P + args.steps)
    print(f"decoded {args.steps} tokens ({mode}); first generated ids {ids[P:P + 4].tolist()}", flush=True)
    return 0


if __name__ == "__main__":
    import sys
    sys.exit(_main())
