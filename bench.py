#!/usr/bin/env python3
"""Benchmark of the MI355X int8 quantized-linear path (one JSON line on stdout).

Headline (BASELINE.json metric, config 2): greedy int8 decode tok/s of a
Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, 16/8 heads, head_dim 128,
SwiGLU 3072, vocab 151936, int8 lm_head), batch 1. A "step" is one whole
config-2 generation: reset to a 128-token random prompt, run the prompt's
first 127 positions as one batch (pio_qwen3_prefill: every int8 linear once
over all 127 rows on the W8 MFMA GEMM), then 256 greedy tokens (the first of
them consumes the last prompt position). `--steps K` times K generations after
`--warmup W` untimed ones, bracketed by device synchronization; HIP events on
the decoder's stream split each generation into prefill and decode, and
`value` = generated tokens / decode time (so every step decodes at the
config's mean context of 255.5 positions whatever K is). Random-init int8
weights (no checkpoint is available offline) and random prompt ids; every
input is resident in HBM before the timed region. The tokens run in the
persistent decode kernel (one launch per generation's 256 tokens)
when the config supports it; the captured-graph step path is timed on one
generation and reported next to it.

Also in the same line:
  roofline      the dominant kernel: the persistent decode kernel (algorithmic
                bytes of a generation's 256 tokens / its launch time, HIP
                events on the decoder's stream); on the graph path, the
                per-layer W8 GEMV replayed alone from a graph. `traffic` is the
                HBM bytes of that launch measured with rocprofv3 counters
                (FETCH_SIZE and WRITE_SIZE passes, each scaled by what the
                counter reads for a plain 1 GiB device copy, see
                --calibrate-copy), read from the profile summary
                profiles/decode_loop_kernel_traffic.txt.
  cpu_baseline  the reference CPU path (oracle/_ref/libtensor_ops_ref.so, built
                from the reference's own tensor_ops.c): its fp32 tensor_linear on
                per-channel-dequantized weights over every linear of one decode
                token, on the host cores.
  kernels       the other BASELINE configs' kernels: C1 GEMV, C3 W8A8 GEMMs +
                quantizer, C4 skinny-M sweep and lm_head, C5 MoE layer; each
                entry carries a `cpu` leg: the reference's tensor_matmul_int8
                (tensor_linear for C1's fp32 path, plus tensor_softmax /
                tensor_topk routing for C5) on a bounded sample, scaled.

Other modes (each prints its own line and exits):
  --weights             checkpoint loading: config-2 decoder weights as int8 and
                        BF16 safetensors, page cache -> HBM, with the reference
                        loader timed beside it.
  --gemm-launches S..   10 plain W8A8 GEMM launches per MxKxN shape (the command
                        the MFMA counter passes profile).
  --gemv-launches S..   10 plain W8 GEMV launches per MxKxN[:f16] shape (the
                        command the HBM traffic counter passes profile).
  --decode-timeline, --gemm-supply, --gemm-timeline: the decode's per-phase
                        timeline, the C3 GEMM's operand-supply probe and its
                        per-block timeline (the profiles' commands).
  --gemm-vendor         the C3 shapes through this library's GEMMs beside
                        hipBLASLt's int8 GEMM (torch._int_mm), int32 compared.
  --decode-only, --calibrate-copy: see --help.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, TOP/s
BF16_PEAK_TFLOPS = 2500.0       # MI355X dense bf16 / fp16 MFMA, TFLOP/s
METRIC = "int8 GEMV % HBM peak; W8A8 GEMM % int8 MFMA peak; Qwen3-0.6B decode tok/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ timing
class Timer:
    """Graph-captured repetitions timed with events on the capture stream."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.Stream()

    def graph(self, fn, reps):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            fn(self.stream.cuda_stream)           # warm (untimed, outside the graph)
            self.stream.synchronize()
            with torch.cuda.graph(g, stream=self.stream):
                for _ in range(reps):
                    fn(self.stream.cuda_stream)
        return g

    def time_graph(self, g, replays=3):
        torch = self.torch
        with torch.cuda.stream(self.stream):
            g.replay()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(self.stream)
            for _ in range(replays):
                g.replay()
            e1.record(self.stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / replays   # seconds per replay


# ------------------------------------------------------------------ decode
PROMPT_LEN = 128     # 128-token random-id prompt ...
GEN_LEN = 256        # ... then 256 greedy tokens


def bench_decode(torch, args):
    """BASELINE config 2, as stated: every step is one whole generation --
    reset to a 128-token prompt, the prompt's first 127 positions as one batch
    (prefill), then 256 greedy tokens -- so each timed step decodes at mean
    context 255.5 whatever --steps is.
    HIP events on the decoder's stream split each generation into prefill and
    decode; `value` is generated tokens / decode time."""
    import numpy as np
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights

    P, NG = PROMPT_LEN, GEN_LEN
    cfg = Qwen3Config(max_seq=P + NG)
    t0 = time.time()
    w = random_weights(cfg, seed=0)
    log(f"[decode] random weights built in {time.time() - t0:.1f}s")
    st = torch.cuda.Stream()
    dec = Qwen3Int8Decoder(cfg, w, stream=st.cuda_stream)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=P).astype(np.int32)
    modes = ["persistent", "graph"] if dec.persistent_supported() else ["graph"]
    if args.decode_only:
        modes = modes[:1]

    def generation(mode):
        dec.reset(prompt)                 # host-synchronous upload of the prompt
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(st)
        dec.prefill(P - 1)
        e[1].record(st)
        dec.run(NG, mode=mode)
        e[2].record(st)
        return e

    def run_mode(mode, steps, warmup):
        for _ in range(warmup):
            generation(mode)
        torch.cuda.synchronize()
        t_wall = time.perf_counter()
        evs = [generation(mode) for _ in range(steps)]
        torch.cuda.synchronize()
        t_wall = time.perf_counter() - t_wall
        ids = dec.read(P + NG)
        assert np.array_equal(ids[:P], prompt)
        pre = [e[0].elapsed_time(e[1]) * 1e-3 for e in evs]
        dcd = [e[1].elapsed_time(e[2]) * 1e-3 for e in evs]
        return t_wall, pre, dcd, ids

    wb = cfg.weight_bytes()
    mean_ctx = P + (NG - 1) / 2.0
    bytes_tok = wb["int8"] + wb["scales"] + wb["bias_norms"] + cfg.kv_bytes_per_pos() * mean_ctx
    res = {}
    for i, mode in enumerate(modes):
        # the first mode is the headline (all --steps); the other one is timed
        # on a single generation for comparison
        steps, warmup = (args.steps, args.warmup) if i == 0 else (1, 1)
        t_wall, pre, dcd, ids = run_mode(mode, steps, warmup)
        dsum = float(sum(dcd))
        res[mode] = {
            "generations": steps,
            "tok_s": NG * steps / dsum,
            "ms_per_token": dsum / (NG * steps) * 1e3,
            "decode_ms_per_generation": dsum / steps * 1e3,
            "prefill_ms_per_generation": float(sum(pre)) / steps * 1e3,
            "wall_ms_per_generation": t_wall / steps * 1e3,
            "decode_ms_min_max": [min(dcd) * 1e3, max(dcd) * 1e3],
            "bytes_per_token": bytes_tok,
            "hbm_frac": bytes_tok * NG * steps / dsum / (HBM_PEAK_GBS * 1e9),
            "ceiling_tok_s": HBM_PEAK_GBS * 1e9 / bytes_tok,
            "generated_head": ids[P:P + 8].tolist(),
        }
        log(f"[decode:{mode}] {res[mode]['tok_s']:.1f} tok/s over {steps} generation(s) of {NG} "
            f"tokens ({res[mode]['ms_per_token']:.3f} ms/token), prefill "
            f"{res[mode]['prefill_ms_per_generation']:.1f} ms")
        res[mode]["_ids"] = ids
    if len(modes) == 2:
        res["persistent"]["same_tokens_as_graph"] = bool(
            np.array_equal(res["persistent"]["_ids"], res["graph"]["_ids"]))
    if not args.decode_only:
        # the same generation with an fp16 KV cache (its own decoder), one
        # timed generation in the fastest mode
        from dataclasses import replace
        cfg16 = replace(cfg, kv_dtype="float16")
        dec16 = Qwen3Int8Decoder(cfg16, w, stream=st.cuda_stream)
        m16 = "persistent" if dec16.persistent_supported() else "graph"
        dec_main = dec
        dec = dec16
        try:
            t_wall, pre, dcd, ids = run_mode(m16, 1, 1)
        finally:
            dec = dec_main
        b16 = wb["int8"] + wb["scales"] + wb["bias_norms"] + cfg16.kv_bytes_per_pos() * mean_ctx
        res["kv_fp16"] = {
            "mode": m16, "tok_s": NG / dcd[0], "ms_per_token": dcd[0] / NG * 1e3,
            "bytes_per_token": b16, "hbm_frac": b16 * NG / dcd[0] / (HBM_PEAK_GBS * 1e9),
            "generated_head": ids[P:P + 8].tolist(),
        }
        log(f"[decode:kv fp16] {res['kv_fp16']['tok_s']:.1f} tok/s ({m16})")
        dec16.close()
        del dec16
    for m in modes:
        res[m].pop("_ids")
    res["mode"] = modes[0]
    return cfg, w, dec, st, res


def bench_decode_gemv(torch, timer, cfg, dec):
    """Dominant kernel: the 112 per-layer GEMVs of one token, replayed from a
    graph over the decoder's own weights (plus lm_head separately)."""
    from mod_amd import ops
    H, D, I = cfg.hidden, cfg.head_dim, cfg.intermediate
    nqkv = (cfg.n_heads + 2 * cfg.n_kv_heads) * D
    x = torch.randn(max(H, I, cfg.n_heads * D), device="cuda")
    y = torch.empty(max(nqkv, 2 * I, cfg.vocab), device="cuda")
    layers = dec._layers_c
    shapes = []
    for l in range(cfg.n_layers):
        L = layers[l]
        shapes += [(L.w_qkv, L.s_qkv, L.b_qkv, nqkv, H), (L.w_o, L.s_o, None, H, cfg.n_heads * D),
                   (L.w_gu, L.s_gu, None, 2 * I, H), (L.w_down, L.s_down, None, H, I)]

    def layer_gemvs(s):
        for (wp, sp, bp, n, k) in shapes:
            ops.gemv_w8(x, wp, sp, bp, y, 1, n, k, s)

    g = timer.graph(layer_gemvs, 1)
    t = timer.time_graph(g, replays=5)
    nbytes = sum(n * k + 4 * n + 4 * k + 4 * n + (4 * n if b else 0) for (_, _, b, n, k) in shapes)
    per_launch_bytes = nbytes / len(shapes)
    per_launch_s = t / len(shapes)

    def lm(s):
        ops.gemv_w8(x, dec._lm, dec._slm, None, y, 1, cfg.vocab, H, s)
    g2 = timer.graph(lm, 4)
    tl = timer.time_graph(g2, replays=5) / 4
    lm_bytes = cfg.vocab * H + 8 * cfg.vocab + 4 * H
    return {
        "layer_gemv_launches": len(shapes),
        "layer_gemv_us_per_launch": per_launch_s * 1e6,
        "layer_gemv_bytes_per_launch": per_launch_bytes,
        "layer_gemv_GBs": per_launch_bytes / per_launch_s / 1e9,
        "lm_head_us": tl * 1e6,
        "lm_head_GBs": lm_bytes / tl / 1e9,
    }


def gemm_supply(torch):
    """What bounds the C3 GEMM's K loop: the GEMM itself (fp16 out, graph of
    10 launches over 8 rotating operand sets) beside the probe that issues only
    its operand copies -- same 128 x 192 tiles, same XCD rectangles, two K steps
    in flight, one barrier per step -- with K steps of 128 B per row (the
    GEMM's), 256 B and 512 B. Per-CU supply = 320 rows x K bytes per block /
    the launch time (one block per CU)."""
    from mod_amd import ops
    timer = Timer(torch)
    out = {}
    for (M, N, K) in [(2048, 3072, 1024), (2048, 3072, 3072)]:
        sets = 8
        A = torch.randint(-127, 127, (sets, M, K), dtype=torch.int8, device="cuda")
        B = torch.randint(-127, 127, (sets, N, K), dtype=torch.int8, device="cuda")
        sa = torch.rand((M,), device="cuda") * 0.01
        sw = torch.rand((N,), device="cuda") * 0.01
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")

        def g(s):
            for i in range(sets):
                ops.gemm_w8a8(A[i], sa, B[i], sw, None, y, M, N, K, s)
        tg = timer.time_graph(timer.graph(g, 1), replays=5) / sets
        row = {"gemm_us": round(tg * 1e6, 2), "gemm_TOPS": round(2 * M * N * K / tg / 1e12, 1)}
        for step in (128, 256, 512):
            def f(s, step=step):
                for i in range(sets):
                    ops.check(ops.lib.pio_probe_gemm_supply(ops._ptr(A[i]), ops._ptr(B[i]), M, N, K, 128, 192,
                                                            step, 1, s), "pio_probe_gemm_supply")
            t = timer.time_graph(timer.graph(f, 1), replays=5) / sets
            row[f"copies_step{step}_us"] = round(t * 1e6, 2)
            row[f"copies_step{step}_GBs_per_CU"] = round(320 * K / t / 1e9, 1)
        out[f"M{M}_N{N}_K{K}"] = row
        log(f"[gemm-supply] {M}x{N}x{K}: {row}")
        del A, B
    return out


def gemm_vendor(torch):
    """The C3 shapes through this library's W8A8 GEMMs and through the vendor
    library (hipBLASLt, reached as torch._int_mm: int8 x int8 -> int32), timed
    the same way: a graph of 20 launches, HIP events around 5 replays. The
    vendor GEMM is also timed eagerly (50 back-to-back calls), in case its
    graph capture records extra nodes. The int32 products of the two libraries
    are compared element for element."""
    from mod_amd import ops
    timer = Timer(torch)
    out = {}
    reps = 20
    for (K, N) in [(1024, 3072), (3072, 1024), (1024, 2048)]:
        M = 2048
        A = torch.randint(-127, 127, (M, K), dtype=torch.int8, device="cuda")
        W = torch.randint(-127, 127, (N, K), dtype=torch.int8, device="cuda")   # [N, K] rows
        Bkn = W.t().contiguous()                                               # [K, N], the reference's b
        sa = torch.rand((M,), device="cuda") * 0.01
        sw = torch.rand((N,), device="cuda") * 0.01
        yh = torch.empty((M, N), dtype=torch.float16, device="cuda")
        c32 = torch.empty((M, N), dtype=torch.int32, device="cuda")
        ws = torch.empty(max(1, int(ops.lib.pio_matmul_int8_workspace(1, M, K, N))), dtype=torch.uint8,
                         device="cuda")
        row = {}
        t = timer.time_graph(timer.graph(lambda s: ops.gemm_w8a8(A, sa, W, sw, None, yh, M, N, K, s), reps),
                             replays=5) / reps
        row["ours_w8a8_f16_us"] = round(t * 1e6, 2)
        t = timer.time_graph(timer.graph(lambda s: ops.matmul_int8(A, Bkn, c32, 1, M, K, N, True, ws, s),
                                         reps), replays=5) / reps
        row["ours_matmul_int8_i32_us"] = round(t * 1e6, 2)
        # hipBLASLt wants the second operand column-major: W.t() is [K, N] in that layout
        ref = torch._int_mm(A, W.t())
        torch.cuda.synchronize()
        row["int32_equal"] = bool(torch.equal(ref, c32))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(timer.stream):
            torch._int_mm(A, W.t())
            timer.stream.synchronize()
            with torch.cuda.graph(g, stream=timer.stream):
                for _ in range(reps):
                    torch._int_mm(A, W.t())
        row["hipblaslt_i32_graph_us"] = round(timer.time_graph(g, replays=5) / reps * 1e6, 2)
        with torch.cuda.stream(timer.stream):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(timer.stream)
            for _ in range(50):
                torch._int_mm(A, W.t())
            e1.record(timer.stream)
        e1.synchronize()
        row["hipblaslt_i32_eager_us"] = round(e0.elapsed_time(e1) * 1e3 / 50, 2)
        for k in list(row):
            if k.endswith("_us"):
                row[k.replace("_us", "_TOPS")] = round(2 * M * N * K / (row[k] * 1e-6) / 1e12, 1)
        out[f"M{M}_K{K}_N{N}"] = row
        log(f"[gemm-vendor] M={M} K={K} N={N}: {row}")
        del A, W, Bkn, yh, c32, ws, ref, g
    return out


def gemm_timeline(torch):
    """Per-block timeline of the C3 GEMM (fp16 out) through its traced build
    (pio_probe_gemm_timeline): every block stamps its start, the end of its K
    loop, its stores issued and its stores complete. Times are relative to the
    first block's start; five eager launches on warm operands, medians."""
    import numpy as np
    from mod_amd import ops
    out = {}
    for (K, N) in [(1024, 3072), (3072, 1024), (1024, 2048)]:
        M = 2048
        A = torch.randint(-127, 127, (M, K), dtype=torch.int8, device="cuda")
        B = torch.randint(-127, 127, (N, K), dtype=torch.int8, device="cuda")
        sa = torch.rand((M,), device="cuda") * 0.01
        sw = torch.rand((N,), device="cuda") * 0.01
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        words = 4 * 2048
        tr = torch.zeros((words,), dtype=torch.int64, device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        rows = []
        for rep in range(6):
            n = ops.lib.pio_probe_gemm_timeline(ops._ptr(A), ops._ptr(sa), ops._ptr(B), ops._ptr(sw), ops._ptr(y),
                                                M, N, K, ops._ptr(tr), words, s)
            torch.cuda.synchronize()
            ops.check(n if n < 0 else 0, "pio_probe_gemm_timeline")
            t = tr[:4 * n].view(n, 4).cpu().numpy().astype(np.float64)
            t = t[t[:, 0] > 0]
            t0 = t[:, 0].min()
            if rep == 0:
                continue   # first touch of the operands
            rows.append({"blocks": int(t.shape[0]),
                         "first_to_last_start_us": (t[:, 0].max() - t0) / 100,
                         "k_loop_us_median": float(np.median(t[:, 1] - t[:, 0])) / 100,
                         "k_loop_us_max": float((t[:, 1] - t[:, 0]).max()) / 100,
                         "stores_issue_us_median": float(np.median(t[:, 2] - t[:, 1])) / 100,
                         "stores_drain_us_median": float(np.median(t[:, 3] - t[:, 2])) / 100,
                         "block_life_us_median": float(np.median(t[:, 3] - t[:, 0])) / 100,
                         "first_start_to_last_end_us": (t[:, 3].max() - t0) / 100})
        med = {k: round(float(np.median([r[k] for r in rows])), 2) for k in rows[0]}
        med["steps"] = K // 128
        med["per_launch"] = [{k: round(float(v), 2) for k, v in r.items()} for r in rows]
        out[f"M{M}_N{N}_K{K}"] = med
        log(f"[gemm-timeline] {M}x{N}x{K}: {dict((k, v) for k, v in med.items() if k != 'per_launch')}")
        for r in med["per_launch"]:
            log(f"[gemm-timeline]     {r}")
        del A, B, y
    return out


TL_SLOTS = ["layer start", "P1 cross-XCD reduction", "P2 gather", "q/k/v stored", "attention stored",
            "merged", "o_proj partial stored", "P5 cross-XCD reduction", "P6 gather", "act stored",
            "down partial stored"]


def decode_timeline(torch):
    """Per-phase timeline of the persistent decode at config 2: a generation
    (batched prompt, then 256 tokens in one traced launch) whose steps 124 and
    125 (context ~252, the generation's mean) are stamped at every phase
    boundary by every workgroup. Durations are medians over workgroups and
    layers 1 .. L-2 of step 124; a phase's time runs from the previous
    boundary, so it includes waiting for its input."""
    import numpy as np
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    P, NG, T0 = PROMPT_LEN, GEN_LEN, 124
    cfg = Qwen3Config(max_seq=P + NG)
    w = random_weights(cfg, seed=0)
    dec = Qwen3Int8Decoder(cfg, w)
    if not dec.persistent_supported():
        return {"error": "persistent decode unsupported here"}
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=P).astype(np.int32)
    for traced in (False, True):
        dec.reset(prompt)
        dec.prefill(P - 1)
        if traced:
            dec.trace_next(T0)
        dec.run(NG, mode="persistent")
    ids = dec.read(P + NG)
    A = dec.phase_trace()[0]                   # step T0: [256][L + 1][16], ns
    L = cfg.n_layers
    mid = A[:, 1:L - 1, :]
    att = (np.arange(256) // 8) < 8            # roles j * 8 + g with j < 8 run attention
    out = {"step": T0, "context": P - 1 + T0 + 1, "first_ids": ids[P:P + 4].tolist(), "phases_us": {}}

    def med(a):
        a = a[np.isfinite(a)]
        return round(float(np.median(a)) / 1e3, 3) if a.size else None

    prev = 0
    for k in range(1, 11):
        src = 3 if k == 5 else prev        # "merged" counts from the q/k/v store on every workgroup
        rows = att if k == 4 else slice(None)
        out["phases_us"][f"{TL_SLOTS[src]} -> {TL_SLOTS[k]}"] = med(mid[rows, :, k] - mid[rows, :, src])
        prev = k if k != 4 else 3
    out["phases_us"]["attention wgs: q/k/v stored -> merged"] = med(mid[att, :, 5] - mid[att, :, 3])
    out["subphases_us"] = {
        "P2 gather -> q/k/v weight lines landed": med(mid[:, :, 11] - mid[:, :, 2]),
        "weight lines landed -> q/k/v stored": med(mid[:, :, 3] - mid[:, :, 11]),
        "attention wgs: q/k/v stored -> q arrived": med(mid[att, :, 12] - mid[att, :, 3]),
        "attention wgs: q arrived -> computed": med(mid[att, :, 13] - mid[att, :, 12]),
        "attention wgs: computed -> stored (waves combined)": med(mid[att, :, 4] - mid[att, :, 13]),
        "attention wgs: stored -> merge inputs arrived": med(mid[att, :, 14] - mid[att, :, 4]),
        "other wgs: q/k/v stored -> merge inputs arrived": med(mid[~att, :, 14] - mid[~att, :, 3]),
        "merge inputs arrived -> merged": med(mid[:, :, 5] - mid[:, :, 14]),
    }
    starts = np.nanmedian(A[:, :L, 0], axis=0)
    out["layer_period_us"] = round(float(np.median(np.diff(starts[1:L - 1]))) / 1e3, 3)
    lm = A[:, L, :]
    out["lm_us"] = {"start -> reduced": med(lm[:, 1] - lm[:, 0]), "reduced -> gathered": med(lm[:, 2] - lm[:, 1]),
                    "gathered -> lm_head rows done": med(lm[:, 3] - lm[:, 2]),
                    "rows done -> key stored": med(lm[:, 4] - lm[:, 3])}
    B = dec.phase_trace()[1]
    out["token_period_us"] = round(float(np.nanmedian(B[:, 0, 0]) - np.nanmedian(A[:, 0, 0])) / 1e3, 3)
    out["layers_us"] = round(float(starts[L - 1] - starts[0]) / (L - 1) / 1e3, 3)
    # skew: spread of each boundary over the 256 workgroups (median over layers)
    out["boundary_spread_us"] = {TL_SLOTS[k]: med(np.nanmax(mid[:, :, k], axis=0) - np.nanmin(mid[:, :, k], axis=0))
                                 for k in range(11) if k != 4}
    # hand-offs: each consumer's stamp after the LAST producer it waits for
    # (the XCD's, or every workgroup's across XCDs), percentiles over
    # workgroups and layers: the wait that no producer skew explains
    g = np.arange(256) % 8
    hops = [("down partial stored (layer start) -> P1 reduced, across XCDs", 0, 1, True, None),
            ("o_proj partial stored -> P5 reduced, across XCDs", 6, 7, True, None),
            ("P1 reduced -> P2 gathered, in the XCD", 1, 2, False, None),
            ("P5 reduced -> P6 gathered, in the XCD", 7, 8, False, None),
            ("act stored -> down partial stored, in the XCD", 9, 10, False, None),
            ("q/k/v stored -> attention's q arrived, in the XCD", 3, 12, False, att),
            ("attention stored -> merge inputs arrived, in the XCD", 4, 14, False, None)]
    out["hop_after_last_producer_us"] = {}
    for name, src, dst, cross, rows in hops:
        d = []
        for x in range(8):
            prod = mid[att & (g == x)] if src == 4 else (mid if cross else mid[g == x])
            last = np.nanmax(prod[:, :, src], axis=0)
            cons = mid[(g == x) & (rows if rows is not None else True)][:, :, dst]
            d.append(cons - last[None, :])
        d = np.concatenate(d).ravel()
        d = d[np.isfinite(d)]
        q = np.percentile(d, [0, 10, 50, 90, 100]) / 1e3
        out["hop_after_last_producer_us"][name] = {k: round(float(v), 2) for k, v in
                                                     zip(("min", "p10", "p50", "p90", "max"), q)}
    for k, v in out["hop_after_last_producer_us"].items():
        log(f"[timeline] hop {k:55s} {v}")
    for k, v in list(out["phases_us"].items()) + list(out["subphases_us"].items()):
        log(f"[timeline] {k:55s} {v} us")
    log(f"[timeline] layer period {out['layer_period_us']} us, token period {out['token_period_us']} us, "
        f"lm {out['lm_us']}")
    dec.close()
    return out


# ----------------------------------------------------------------- kernels
def bench_kernels(torch, timer):
    from mod_amd import ops
    out = {}
    dev = "cuda"

    # C1: GEMV [1,1024] x int8 [3072,1024], rotating over 160 distinct weights
    # (> 256 MB Infinity Cache) so every launch streams from HBM.
    M, N, K = 1, 3072, 1024
    pool = 160
    Ws = torch.randint(-127, 127, (pool, N, K), dtype=torch.int8, device=dev)
    ss = torch.rand((pool, N), device=dev) * 0.019 + 0.001
    x = torch.randn((M, K), device=dev)
    y = torch.empty((M, N), device=dev)

    def c1(s):
        for i in range(pool):
            ops.gemv_w8(x, Ws[i], ss[i], None, y, M, N, K, s)
    t = timer.time_graph(timer.graph(c1, 1)) / pool
    b = N * K + 4 * N + 4 * K + 4 * N
    out["c1_gemv"] = {"us": t * 1e6, "GBs": b / t / 1e9, "hbm_frac": b / t / 1e9 / HBM_PEAK_GBS,
                      "bytes": b}
    del Ws, ss

    # The C1 linear over many fp32 rows (the prefill and large-M W8 path,
    # pio_gemv_w8 above 4 rows): the W8 MFMA GEMM, fp32 x as three exact bf16
    # parts. Algorithmic work 2MNK; the matrix cores run 3x that in bf16.
    many = {}
    for M in (128, 2048):
        N, K = 3072, 1024
        W = torch.randint(-127, 127, (N, K), dtype=torch.int8, device=dev)
        sw = torch.rand((N,), device=dev) * 0.019 + 0.001
        xm = torch.randn((M, K), device=dev)
        ym = torch.empty((M, N), device=dev)
        reps = 10
        t = timer.time_graph(timer.graph(lambda s: ops.gemv_w8(xm, W, sw, None, ym, M, N, K, s), reps)) / reps
        fl = 2.0 * M * N * K
        many[f"M{M}_N{N}_K{K}_f32"] = {
            "us": t * 1e6, "TFLOPs": fl / t / 1e12, "bf16_mfma_TFLOPs": 3 * fl / t / 1e12,
            "bf16_mfma_frac": 3 * fl / t / 1e12 / BF16_PEAK_TFLOPS,
            "weight_reads_GBs": (N * K + 4 * N) / t / 1e9}
        del W, xm, ym
    out["w8_linear_many_rows"] = many

    # C3: per-token quant + W8A8 GEMM, M=2048, fp16 in/out.
    c3 = {}
    for (K, N) in [(1024, 3072), (3072, 1024), (1024, 2048)]:
        M = 2048
        xh = torch.randn((M, K), device=dev).half()
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
        sa = torch.empty((M,), device=dev)
        W = torch.randint(-127, 127, (N, K), dtype=torch.int8, device=dev)
        sw = torch.rand((N,), device=dev) * 0.019 + 0.001
        yh = torch.empty((M, N), dtype=torch.float16, device=dev)
        reps = 20
        gam = torch.rand((K,), device=dev) + 0.5
        tq = timer.time_graph(timer.graph(lambda s: ops.quantize_per_token(xh, q, sa, M, K, s), reps)) / reps
        trq = timer.time_graph(timer.graph(
            lambda s: ops.rmsnorm_quant(xh, gam, q, sa, M, K, 1e-6, stream=s), reps)) / reps
        tg = timer.time_graph(timer.graph(lambda s: ops.gemm_w8a8(q, sa, W, sw, None, yh, M, N, K, s), reps)) / reps
        tops = 2 * M * N * K / tg / 1e12
        c3[f"K{K}_N{N}"] = {"gemm_us": tg * 1e6, "TOPS": tops, "mfma_frac": tops / INT8_PEAK_TOPS,
                            "quant_us": tq * 1e6, "quant_GBs": (3 * M * K + 4 * M) / tq / 1e9,
                            "with_quant_TOPS": 2 * M * N * K / (tg + tq) / 1e12,
                            "rmsnorm_quant_us": trq * 1e6,
                            "rmsnorm_quant_GBs": (3 * M * K + 4 * M + 4 * K) / trq / 1e9}
    out["c3_w8a8"] = c3

    # C4: Qwen3-8B linears, GEMV across M (skinny) + lm_head [151936, 4096].
    c4 = {}
    for (N, K) in [(12288, 4096), (4096, 12288)]:
        reps_w = 6   # 6 x 50 MB > Infinity Cache
        Wp = torch.randint(-127, 127, (reps_w, N, K), dtype=torch.int8, device=dev)
        sw = torch.rand((N,), device=dev) * 0.019 + 0.001
        for M in (1, 4, 16, 64):
            xh = torch.randn((M, K), device=dev).half()
            yh = torch.empty((M, N), dtype=torch.float16, device=dev)

            def f(s):
                for i in range(reps_w):
                    ops.gemv_w8(xh, Wp[i], sw, None, yh, M, N, K, s)
            t = timer.time_graph(timer.graph(f, 1)) / reps_w
            b = N * K + 4 * N + 2 * M * K + 2 * M * N
            c4[f"gemv_N{N}_K{K}_M{M}"] = {"us": t * 1e6, "GBs": b / t / 1e9,
                                          "hbm_frac": b / t / 1e9 / HBM_PEAK_GBS}
            # MFMA alternative at the same M: per-token quant + W8A8 GEMM.
            q = torch.empty((M, K), dtype=torch.int8, device=dev)
            sa = torch.empty((M,), device=dev)

            def f2(s):
                for i in range(reps_w):
                    ops.quantize_per_token(xh, q, sa, M, K, s)
                    ops.gemm_w8a8(q, sa, Wp[i], sw, None, yh, M, N, K, s)
            t2 = timer.time_graph(timer.graph(f2, 1)) / reps_w
            c4[f"w8a8_N{N}_K{K}_M{M}"] = {"us": t2 * 1e6, "GBs": b / t2 / 1e9}
        del Wp
    N, K = 151936, 4096
    Wl = torch.randint(-127, 127, (N, K), dtype=torch.int8, device=dev)
    sl = torch.rand((N,), device=dev) * 0.019 + 0.001
    xh = torch.randn((1, K), device=dev).half()
    yh = torch.empty((1, N), dtype=torch.float16, device=dev)
    t = timer.time_graph(timer.graph(lambda s: ops.gemv_w8(xh, Wl, sl, None, yh, 1, N, K, s), 4)) / 4
    b = N * K + 4 * N + 2 * K + 2 * N
    c4["lm_head_8b_M1"] = {"us": t * 1e6, "GBs": b / t / 1e9, "hbm_frac": b / t / 1e9 / HBM_PEAK_GBS}
    del Wl
    out["c4_skinny"] = c4

    # C5: MoE expert layer (128 experts, top-8, 512 tokens, H 2048, I 768).
    T, H, I, E, k = 512, 2048, 768, 128, 8
    xm = torch.randn((T, H), device=dev).half()
    lg = torch.randn((T, E), device=dev)
    wgu = torch.randint(-127, 127, (E, 2 * I, H), dtype=torch.int8, device=dev)
    sgu = torch.rand((E, 2 * I), device=dev) * 0.019 + 0.001
    wdn = torch.randint(-127, 127, (E, H, I), dtype=torch.int8, device=dev)
    sdn = torch.rand((E, H), device=dev) * 0.019 + 0.001
    om = torch.empty((T, H), dtype=torch.float16, device=dev)
    ws = torch.empty((ops.moe_workspace_bytes(T, H, I, E, k),), dtype=torch.uint8, device=dev)
    t = timer.time_graph(timer.graph(
        lambda s: ops.moe_w8a8(xm, lg, wgu, sgu, wdn, sdn, om, T, H, I, E, k, False, ws, s), 2)) / 2
    wbytes = E * (2 * I * H + H * I) + 4 * E * (2 * I + H)
    ops_ = T * k * (2 * H * 2 * I + 2 * I * H)
    out["c5_moe"] = {"us": t * 1e6, "weight_GBs": wbytes / t / 1e9,
                     "hbm_frac": wbytes / t / 1e9 / HBM_PEAK_GBS, "TOPS": ops_ / t / 1e12}
    return out


# ------------------------------------------------------------ CPU baseline
CPU_NOTE = ("reference CPU backend built from its own source (tensor_ops.c, Makefile:15 flags); "
            "it parallelizes over the batch dimension only (tensor_ops.c:225, 306), so a 2-D "
            "product runs on one core")


def _median_time(fn, reps=5, budget_s=5.0):
    """Median wall time of fn over up to `reps` calls within `budget_s`; the
    first call warms up, and counts as a sample when it is long (>= 0.2 s)."""
    import numpy as np
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    times = [first] if first >= 0.2 else []
    t_start = time.perf_counter()
    while len(times) < reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(cfg, w, budget_s=20.0):
    """Config 2 on the host: the reference's fp32 tensor_linear (tensor_ops.c:
    323-335) over one decode token's linears, weights dequantized per channel
    (what the reference model runs today)."""
    import numpy as np
    import oracle
    if not oracle.ref_available():
        return None
    L = oracle.ref_lib()
    H, D, I = cfg.hidden, cfg.head_dim, cfg.intermediate
    nqkv = (cfg.n_heads + 2 * cfg.n_kv_heads) * D
    x = {k: oracle.RefTensor((1, k), np.random.default_rng(k).standard_normal((1, k)).astype(np.float32))
         for k in {H, cfg.n_heads * D, I}}
    outs = {n: oracle.RefTensor((1, n)) for n in {nqkv, H, 2 * I, cfg.vocab}}
    mats = []
    t_build = time.time()
    for l, Lw in enumerate(w["layers"]):
        for (wk, sk, bk, n, k) in (("w_qkv", "s_qkv", "b_qkv", nqkv, H),
                                   ("w_o", "s_o", None, H, cfg.n_heads * D),
                                   ("w_gu", "s_gu", None, 2 * I, H),
                                   ("w_down", "s_down", None, H, I)):
            deq = Lw[wk].astype(np.float32) * Lw[sk][:, None]
            mats.append((oracle.RefTensor((n, k), deq),
                         oracle.RefTensor((n,), Lw[bk]) if bk and Lw.get(bk) is not None else None,
                         n, k))
    mats.append((oracle.RefTensor((cfg.vocab, H), w["lm_head"].astype(np.float32) * w["s_lm_head"][:, None]),
                 None, cfg.vocab, H))
    log(f"[cpu] dequantized reference weights in {time.time() - t_build:.1f}s")

    def one_token():
        for (tw, tb, n, k) in mats:
            L.tensor_linear(x[k].h, tw.h, tb.h if tb else None, outs[n].h)

    med, n = _median_time(one_token, reps=5, budget_s=budget_s)
    del mats
    return {
        "value": 1.0 / med,
        "unit": "tok/s",
        "cores": 1,
        "kind": "reference",
        "sample": (f"reference tensor_linear (fp32, tensor_ops.c:301-335) over one decode token's "
                   f"113 linears of the config-2 model (weights dequantized per channel), median "
                   f"of {n} tokens; attention/norm ops excluded. {CPU_NOTE} "
                   f"(OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'default')}, "
                   f"host cores={os.cpu_count()})."),
        "ms_per_token": med * 1e3,
    }


def cpu_kernel_baselines():
    """The other configs on the host, with the reference's own functions:
    tensor_matmul_int8 (tensor_ops.c:217-246, B given [K,N]) for every int8
    product plus the per-token / per-channel scale epilogue in numpy, and
    tensor_linear for C1's fp32 path; C5 adds the reference routing
    (tensor_softmax, tensor_topk). Each leg runs a bounded sample and is scaled
    to the full workload (rows and experts are independent work in these
    loops); the sample is stated per leg."""
    import numpy as np
    import oracle
    if not oracle.ref_available():
        return {}
    L = oracle.ref_lib()
    RT = oracle.RefTensor
    out = {}

    def mm_leg(q, WT, s_a, s_w, out_f16):
        """Reference int8 matmul q[M,K] x WT[K,N] then the scale epilogue."""
        M, K = q.shape
        N = WT.shape[1]
        ta, tb, to = RT((M, K), q), RT((K, N), WT), RT((M, N))

        def f():
            L.tensor_matmul_int8(ta.h, tb.h, to.h)
            y = to.f32() * s_a[:, None] * s_w[None, :]
            return y.astype(np.float16) if out_f16 else y
        return f

    rng = np.random.default_rng(5)

    # C1: (i) fp32 tensor_linear on per-channel dequantized W (what the model runs);
    #     (ii) tensor_matmul_int8 at M=1 on the per-token quantized x.
    N, K = 3072, 1024
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    x = rng.standard_normal((1, K), dtype=np.float32)
    tx, tw, ty = RT((1, K), x), RT((N, K), W.astype(np.float32) * s[:, None]), RT((1, N))
    t_lin, n1 = _median_time(lambda: L.tensor_linear(tx.h, tw.h, None, ty.h))
    q, sa = oracle.quant_per_token(x)
    t_i8, n2 = _median_time(mm_leg(q, np.ascontiguousarray(W.T), sa, s, False))
    out["c1_gemv"] = {"us": t_lin * 1e6, "kind": "reference", "cores": 1,
                      "int8_matmul_us": t_i8 * 1e6,
                      "sample": f"full C1: tensor_linear fp32 [1,1024]x[3072,1024]^T median of {n1}; "
                                f"int8 leg tensor_matmul_int8 [1,1024]x[1024,3072] + epilogue, median of {n2}"}
    # The same linear over many rows: tensor_linear parallelizes over rows
    # (tensor_ops.c:306), so here the host's OpenMP threads all work.
    Ms = 64
    txm, tym = RT((Ms, K), rng.standard_normal((Ms, K), dtype=np.float32)), RT((Ms, N))
    t_m, n3 = _median_time(lambda: L.tensor_linear(txm.h, tw.h, None, tym.h))
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    out["w8_linear_many_rows"] = {
        f"M{M}_N{N}_K{K}_f32": {"us": t_m * M / Ms * 1e6, "kind": "reference", "cores": min(Ms, threads),
                                "sample": f"tensor_linear fp32 [{Ms},1024]x[3072,1024]^T (median of {n3}), "
                                          f"scaled x{M / Ms:g}"}
        for M in (128, 2048)}
    del tw

    # C3: M=2048 rows; an 8-row sample of the int8 matmul (time is linear in M).
    c3 = {}
    for (K, N) in [(1024, 3072), (3072, 1024), (1024, 2048)]:
        Ms = 8
        xs = rng.standard_normal((Ms, K), dtype=np.float32).astype(np.float16)
        q, sa = oracle.quant_per_token(xs)
        W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
        sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
        t, n = _median_time(mm_leg(q, np.ascontiguousarray(W.T), sa, sw, True), reps=2)
        c3[f"K{K}_N{N}"] = {"gemm_us": t * 2048 / Ms * 1e6,
                            "TOPS": 2 * 2048 * N * K / (t * 2048 / Ms) / 1e12,
                            "kind": "reference", "cores": 1,
                            "sample": f"{Ms} of 2048 rows (median of {n}), scaled x{2048 // Ms}"}
    out["c3_w8a8"] = c3

    # C4: Qwen3-8B linears; M=1 measured, larger M from its time x M (the
    # reference loop redoes the whole B sweep per row).
    c4 = {}
    for (N, K) in [(12288, 4096), (4096, 12288)]:
        W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
        WT = np.ascontiguousarray(W.T)
        del W
        sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
        q, sa = oracle.quant_per_token(rng.standard_normal((1, K), dtype=np.float32).astype(np.float16))
        t, n = _median_time(mm_leg(q, WT, sa, sw, True), reps=2)
        for M in (1, 4, 16, 64):
            c4[f"N{N}_K{K}_M{M}"] = {
                "us": t * M * 1e6, "kind": "reference", "cores": 1,
                "sample": (f"full, median of {n}" if M == 1 else
                           f"the measured M=1 time x {M} (rows are independent passes over B)")}
        del WT
    N, K, Ns = 151936, 4096, 8192
    WT = rng.integers(-127, 127, size=(K, Ns), dtype=np.int8)
    sw = rng.uniform(0.001, 0.02, size=Ns).astype(np.float32)
    q, sa = oracle.quant_per_token(rng.standard_normal((1, K), dtype=np.float32).astype(np.float16))
    t, n = _median_time(mm_leg(q, WT, sa, sw, True), reps=3)
    c4["lm_head_8b_M1"] = {"us": t * N / Ns * 1e6, "kind": "reference", "cores": 1,
                           "sample": f"{Ns} of {N} output columns (median of {n}), scaled x{N / Ns:.2f}"}
    del WT
    out["c4_skinny"] = c4

    # C5: reference routing over all 512 tokens; then per expert gather, per-token
    # quant, tensor_matmul_int8 gate_up, SwiGLU, requant, tensor_matmul_int8 down
    # and the k-ordered combine, on a sample of 8 experts scaled by routed rows.
    T, H, I, E, k, Es = 512, 2048, 768, 128, 8, 4
    logits = rng.standard_normal((T, E), dtype=np.float32)
    xm = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    tl, tp = RT((T, E), logits), RT((T, E))
    tv, ti = RT((T, k)), RT((T, k))

    def route():
        L.tensor_softmax(tl.h, tp.h)
        L.tensor_topk(tp.h, k, tv.h, ti.h)
        return tv.f32(), ti.f32().astype(np.int32)
    t_route, _ = _median_time(route, reps=3)
    wts, ids = route()
    experts = []
    for e in range(Es):
        wgu = rng.integers(-127, 127, size=(2 * I, H), dtype=np.int8)
        wdn = rng.integers(-127, 127, size=(H, I), dtype=np.int8)
        experts.append((RT((H, 2 * I), np.ascontiguousarray(wgu.T)), RT((I, H), np.ascontiguousarray(wdn.T)),
                        rng.uniform(0.001, 0.02, size=2 * I).astype(np.float32),
                        rng.uniform(0.001, 0.02, size=H).astype(np.float32)))

    def experts_run():
        y = np.zeros((T, H), np.float32)
        for e in range(Es):
            tok, slot = np.nonzero(ids == e)
            n_e = tok.size
            if n_e == 0:
                continue
            tg, td, sgu, sdn = experts[e]
            q, sa = oracle.quant_per_token(xm[tok])
            tq, tgo = RT((n_e, H), q), RT((n_e, 2 * I))
            L.tensor_matmul_int8(tq.h, tg.h, tgo.h)
            gu = tgo.f32() * sa[:, None] * sgu[None, :]
            g, u = gu[:, :I], gu[:, I:]
            with np.errstate(over="ignore"):
                h = g / (1.0 + np.exp(-g)) * u
            qh, sh = oracle.quant_per_token(h.astype(np.float32))
            th, tdo = RT((n_e, I), qh), RT((n_e, H))
            L.tensor_matmul_int8(th.h, td.h, tdo.h)
            dn = tdo.f32() * sh[:, None] * sdn[None, :]
            y[tok] += wts[tok, slot][:, None] * dn
        return y
    t_exp, n = _median_time(experts_run, reps=2)
    rows_sample = int(np.isin(ids, np.arange(Es)).sum())
    t_total = t_route + t_exp * (T * k) / max(rows_sample, 1)
    ops_ = T * k * (2 * H * 2 * I + 2 * I * H)
    out["c5_moe"] = {"us": t_total * 1e6, "TOPS": ops_ / t_total / 1e12, "kind": "reference",
                     "cores": 1, "route_us": t_route * 1e6,
                     "sample": (f"reference tensor_softmax + tensor_topk over all {T} tokens; the "
                                f"expert pipeline on {Es} of {E} experts ({rows_sample} of {T * k} "
                                f"routed rows, median of {n}), scaled by routed rows")}
    return out


# ----------------------------------------------------------- checkpoint load
def _ckpt_tensors(cfg, w, fp: bool):
    """Config-2 decoder weights under Hugging Face names (fused qkv / gate_up,
    the reference layout): int8 + _scale pairs, or (fp) bf16 bits of the
    dequantized weights. Embedding stored bf16, norms and biases fp32."""
    import numpy as np

    def bf16(a):
        return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)

    t, dts = {}, {}

    def lin(name, q, s):
        if fp:
            t[name] = bf16(q.astype(np.float32) * s[:, None])
            dts[name] = "BF16"
        else:
            t[name], t[name + "_scale"] = q, s

    for i, L in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = L["in_norm"]
        t[p + "post_attention_layernorm.weight"] = L["post_norm"]
        lin(p + "self_attn.qkv_proj.weight", L["w_qkv"], L["s_qkv"])
        t[p + "self_attn.qkv_proj.bias"] = L["b_qkv"]
        lin(p + "self_attn.o_proj.weight", L["w_o"], L["s_o"])
        lin(p + "mlp.gate_up_proj.weight", L["w_gu"], L["s_gu"])
        lin(p + "mlp.down_proj.weight", L["w_down"], L["s_down"])
    t["model.embed_tokens.weight"] = bf16(w["embed"])
    dts["model.embed_tokens.weight"] = "BF16"
    t["model.norm.weight"] = w["final_norm"]
    lin("lm_head.weight", w["lm_head"], w["s_lm_head"])
    return t, dts


def bench_weights(torch):
    """Checkpoint -> HBM for the config-2 decoder, from the page cache (files
    just written): the int8 format loaded as stored, a BF16 checkpoint
    quantized on the GPU while loading, and the offline BF16 -> int8
    conversion; beside them a plain pinned host-to-device copy of the int8
    file's bytes, and the reference's loader (load_tensor_data into host fp32)
    over the BF16 file."""
    import shutil
    import tempfile
    import numpy as np
    from mod_amd import weights as W
    from mod_amd.qwen3 import Qwen3Config, random_weights, weights_from_checkpoint

    cfg = Qwen3Config()
    w = random_weights(cfg, seed=0)
    tmp = Path(tempfile.mkdtemp(prefix="pio_ckpt_", dir=os.environ.get("TMPDIR", "/tmp")))
    res = {}
    try:
        paths = {}
        for kind in ("int8", "bf16"):
            t, dts = _ckpt_tensors(cfg, w, fp=kind == "bf16")
            paths[kind] = tmp / f"{kind}.safetensors"
            t0 = time.perf_counter()
            W.save_safetensors(paths[kind], t, dtypes=dts)
            log(f"[weights] wrote {kind} checkpoint {paths[kind].stat().st_size / 1e6:.0f} MB "
                f"in {time.perf_counter() - t0:.1f}s")
            del t
        for kind in ("int8", "bf16"):
            times = []
            for _ in range(2):
                t0 = time.perf_counter()
                dw = weights_from_checkpoint(paths[kind], cfg)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                del dw
            nb = paths[kind].stat().st_size
            res[kind] = {"bytes": nb, "s": times[-1], "GBs": nb / times[-1] / 1e9,
                         "first_s": times[0]}
            log(f"[weights] {kind} checkpoint -> HBM: {times[-1]:.3f}s "
                f"({nb / times[-1] / 1e9:.2f} GB/s; first {times[0]:.3f}s)")
        t0 = time.perf_counter()
        W.quantize_checkpoint(paths["bf16"], tmp / "q.safetensors")
        res["quantize_checkpoint_s"] = time.perf_counter() - t0
        # plain pinned H2D copy of the same byte count
        nb = res["int8"]["bytes"]
        src = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(nb, dtype=torch.uint8, device="cuda")
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        res["h2d_pinned_GBs"] = nb / (time.perf_counter() - t0) / 1e9
        del src, dst
        # the reference loader over the BF16 file (its byte-count dispatch reads
        # the 2-byte tensors as F16: the same work, different values)
        res["cpu"] = _ref_loader_time(paths["bf16"])
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return res


def _ref_loader_time(path):
    import ctypes
    import numpy as np
    import oracle
    lib_path = oracle.HERE / "_ref" / "libsafetensors_ref.so"
    if not lib_path.exists():
        return None
    from oracle import safetensors_ref as stref
    L = ctypes.CDLL(str(lib_path))
    L.open_safetensors.restype = ctypes.c_void_p
    L.open_safetensors.argtypes = [ctypes.c_char_p]
    L.load_tensor_data.restype = ctypes.c_int
    L.load_tensor_data.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                   ctypes.POINTER(ctypes.c_float), ctypes.c_int]
    L.close_safetensors.argtypes = [ctypes.c_void_p]
    entries, _ = stref.read_header(path)
    t0 = time.perf_counter()
    ctx = L.open_safetensors(str(path).encode())
    ok = 0
    for name, (dt, shape, b, e) in entries.items():
        n = int(np.prod(shape))
        buf = np.empty(n, np.float32)
        ok += L.load_tensor_data(ctx, name.encode(), buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n)
    L.close_safetensors(ctx)
    dt_s = time.perf_counter() - t0
    nb = Path(path).stat().st_size
    return {"value": nb / dt_s / 1e9, "unit": "GB/s", "cores": int(os.environ.get("OMP_NUM_THREADS", 0))
            or os.cpu_count(), "kind": "reference",
            "sample": (f"reference load_tensor_data (safetensors_loader.c:147-243, built from its "
                       f"source) of all {len(entries)} tensors of the BF16 checkpoint into host "
                       f"fp32 buffers ({ok} loaded; its F16 conversion loop runs under OpenMP); "
                       f"the host-to-device copy the reference does next is not included"),
            "s": dt_s}


# ----------------------------------------------------------------- traffic
TRAFFIC_PROFILE = ROOT / "profiles" / "decode_loop_kernel_traffic.txt"


def measured_traffic(steps):
    """HBM bytes of one persistent-decode launch of `steps` tokens, from the
    committed counter summary (its `traffic_bytes_per_launch` and `steps`
    lines), or None when there is none for this step count."""
    try:
        kv = dict(l.split("=", 1) for l in TRAFFIC_PROFILE.read_text().splitlines()
                  if "=" in l and not l.startswith("#"))
        if int(kv["steps"]) == steps:
            return int(float(kv["traffic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        pass
    return None


# -------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3,
                    help="timed generations (each: 128-token prompt + 256 generated tokens)")
    ap.add_argument("--warmup", type=int, default=1, help="untimed generations before them")
    ap.add_argument("--no-kernels", action="store_true", help="skip the C1/C3/C4/C5 kernel suite")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the decode (its fastest supported mode; no graph-replayed "
                         "GEMVs, kernel suite or CPU baseline) -- the command the counter passes "
                         "of the traffic measurement profile")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (three times), for scaling "
                         "the FETCH_SIZE / WRITE_SIZE counters of the traffic measurement")
    ap.add_argument("--gemm-launches", nargs="+", metavar="MxKxN",
                    help="only run 10 plain (ungraphed) W8A8 GEMM launches per shape, fp16 out, "
                         "then exit -- the command the MFMA counter passes profile")
    ap.add_argument("--gemv-launches", nargs="+", metavar="MxKxN[:f16]",
                    help="only run 10 plain (ungraphed) W8 GEMV launches per shape (fp32 x and y, "
                         "or fp16 with ':f16'), each on its own weight copy, then exit -- the "
                         "command the GEMV traffic counter passes profile")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="only run the config-2 generation with one traced persistent launch and print "
                         "the per-phase timeline of two mid-generation tokens (the kernel's traced "
                         "build stamps every phase boundary of every workgroup)")
    ap.add_argument("--gemm-supply", action="store_true",
                    help="only time the C3 W8A8 GEMM beside its operand-supply probe (the K loop's "
                         "copies alone, in K steps of 128, 256 and 512 bytes per row) and print the "
                         "per-CU rates")
    ap.add_argument("--gemm-vendor", action="store_true",
                    help="only time the C3 shapes through this library's W8A8 GEMMs beside the "
                         "vendor library's int8 GEMM (hipBLASLt via torch._int_mm) and compare "
                         "their int32 products")
    ap.add_argument("--gemm-timeline", action="store_true",
                    help="only run the C3 W8A8 GEMM through its traced build and print the per-block "
                         "timeline (start, K loop, stores issued, stores complete)")
    ap.add_argument("--weights", action="store_true",
                    help="only time checkpoint loading (config-2 decoder weights, int8 and BF16 "
                         "safetensors from the page cache into HBM) and print its own JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the int8 path has no multi-GPU component in this "
              f"build (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": 1 << 30, "copies": 3}))
        return 0
    from mod_amd import ops
    log(f"[bench] {ops.version()}  lib={ops.LIB_FILE}")
    if args.gemm_launches:
        for shape in args.gemm_launches:
            M, K, N = (int(v) for v in shape.split("x"))
            A = torch.randint(-127, 127, (M, K), dtype=torch.int8, device="cuda")
            W = torch.randint(-127, 127, (N, K), dtype=torch.int8, device="cuda")
            sa = torch.rand(M, device="cuda")
            sw = torch.rand(N, device="cuda")
            y = torch.empty((M, N), dtype=torch.float16, device="cuda")
            for _ in range(10):
                ops.gemm_w8a8(A, sa, W, sw, None, y, M, N, K)
            torch.cuda.synchronize()
            print(f"done {shape}", flush=True)
        return 0
    if args.gemv_launches:
        for spec in args.gemv_launches:
            shape, _, kind = spec.partition(":")
            M, K, N = (int(v) for v in shape.split("x"))
            dt = torch.float16 if kind == "f16" else torch.float32
            Ws = [torch.randint(-127, 127, (N, K), dtype=torch.int8, device="cuda") for _ in range(2)]
            sw = torch.rand(N, device="cuda") * 0.019 + 0.001
            x = torch.randn((M, K), device="cuda").to(dt)
            y = torch.empty((M, N), dtype=dt, device="cuda")
            for i in range(10):   # alternate two weight copies so no launch reads a warm cache
                ops.gemv_w8(x, Ws[i % 2], sw, None, y, M, N, K)
            torch.cuda.synchronize()
            print(f"done {spec}", flush=True)
        return 0
    if args.decode_timeline:
        print(json.dumps(decode_timeline(torch)))
        return 0
    if args.gemm_supply:
        print(json.dumps(gemm_supply(torch)))
        return 0
    if args.gemm_timeline:
        print(json.dumps(gemm_timeline(torch)))
        return 0
    if args.gemm_vendor:
        print(json.dumps(gemm_vendor(torch)))
        return 0
    if args.weights:
        r = bench_weights(torch)
        cpu = r.pop("cpu")
        rnd = lambda d: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}  # noqa: E731
        print(json.dumps({
            "metric": "int8 checkpoint load, page cache -> HBM",
            "value": round(r["int8"]["GBs"], 3), "unit": "GB/s", "n_gpus": 1,
            "higher_is_better": True, "dtype": "int8 weights, fp32 scales, bf16 embedding",
            "data": "synthetic: random-init config-2 decoder weights written as safetensors",
            "config": {"workload": "Qwen3-0.6B-shaped decoder checkpoint (28 layers, vocab "
                                   "151936) loaded by qwen3.weights_from_checkpoint"},
            "int8": rnd(r["int8"]), "bf16_quantized_on_load": rnd(r["bf16"]),
            "quantize_checkpoint_s": round(r["quantize_checkpoint_s"], 3),
            "h2d_pinned_GBs": round(r["h2d_pinned_GBs"], 2),
            "frac_of_pinned_h2d": round(r["int8"]["GBs"] / r["h2d_pinned_GBs"], 4),
            "cpu_baseline": cpu and rnd(cpu),
        }), flush=True)
        return 0
    timer = Timer(torch)

    cfg, w, dec, st, dall = bench_decode(torch, args)
    dres = dall[dall["mode"]]
    if args.decode_only:
        args.no_kernels = args.no_cpu = True
        g = None
    else:
        g = bench_decode_gemv(torch, timer, cfg, dec)
        log(f"[gemv] layer GEMV {g['layer_gemv_us_per_launch']:.2f} us/launch "
            f"{g['layer_gemv_GBs']:.0f} GB/s; lm_head {g['lm_head_us']:.1f} us {g['lm_head_GBs']:.0f} GB/s")
    dec.close()
    kern = {}
    if not args.no_kernels:
        kern = bench_kernels(torch, timer)
        log("[kernels] " + json.dumps(kern))
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(cfg, w)
            if cpu:
                log(f"[cpu] config 2: {cpu['value']:.3f} tok/s ({cpu['ms_per_token']:.1f} ms/token)")
            t0 = time.time()
            legs = cpu_kernel_baselines()
            log(f"[cpu] kernel legs in {time.time() - t0:.1f}s: " + json.dumps(legs))
            for key, leg in legs.items():
                if key not in kern:
                    continue
                if key in ("c3_w8a8", "c4_skinny", "w8_linear_many_rows"):
                    for sub, v in leg.items():
                        for tgt in (sub, f"gemv_{sub}", f"w8a8_{sub}"):
                            if tgt in kern[key]:
                                kern[key][tgt]["cpu"] = v
                else:
                    kern[key]["cpu"] = leg
        except Exception as e:  # the GPU result stands without the baseline
            log(f"[cpu] baseline failed: {e!r}")

    NG = GEN_LEN
    if dall["mode"] == "persistent" or g is None:
        # Dominant kernel = the persistent decode kernel itself: one launch runs
        # a generation's 256 tokens, so bytes per launch = bytes per token x 256.
        roof = {
            "bound": "hbm",
            "kernel": ("decode_loop_kernel (persistent decode: one launch per generation's "
                       f"{NG} tokens)" if dall["mode"] == "persistent"
                       else "decode step graph (all generated tokens)"),
            "achieved": round(dres["bytes_per_token"] * dres["tok_s"] / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dres["hbm_frac"], 4),
            "traffic": measured_traffic(NG) if dall["mode"] == "persistent" else None,
            "bytes_per_launch": round(dres["bytes_per_token"] * NG),
            "us_per_launch": round(dres["decode_ms_per_generation"] * 1e3, 1),
        }
    else:
        achieved = g["layer_gemv_GBs"]
        roof = {
            "bound": "hbm",
            "kernel": "gemv_w8_stream_kernel (per-layer decode GEMVs: qkv, o, gate_up, down)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": round(g["layer_gemv_bytes_per_launch"]),
            "us_per_launch": round(g["layer_gemv_us_per_launch"], 3),
        }
    rnd = lambda d: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}  # noqa: E731
    line = {
        "metric": METRIC,
        "value": round(dres["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dres["wall_ms_per_generation"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights, fp32 activations/accumulate",
        "data": "synthetic: random-init int8 weights (seed 0), random 128-token prompt",
        "decode_mode": dall["mode"],
        "config": {
            "workload": (f"BASELINE config 2: Qwen3-0.6B-shaped int8 greedy decode, batch 1; one "
                         f"step = one generation: {PROMPT_LEN}-token prompt then {NG} generated "
                         f"tokens; value = generated tokens / decode time (prefill timed apart)"),
            "global_batch": 1, "prompt_len": PROMPT_LEN, "generated": NG,
            "seq_len": PROMPT_LEN + NG, "layers": cfg.n_layers,
            "hidden": cfg.hidden, "heads": f"{cfg.n_heads}q/{cfg.n_kv_heads}kv",
            "head_dim": cfg.head_dim, "intermediate": cfg.intermediate, "vocab": cfg.vocab,
            "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": cpu and rnd(cpu),
        "decode": {m: (rnd(r) if isinstance(r, dict) else r) for m, r in dall.items()},
        "decode_gemv": g and {k: (round(v, 3) if isinstance(v, float) else v) for k, v in g.items()},
        "kernels": kern,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
