"""Writes the small golden fixtures under tests/golden/.

Inputs come from numpy default_rng(seed). Expected outputs come from:
  * the reference CPU library itself (oracle/_ref/libtensor_ops_ref.so, compiled
    from /root/reference/.../tensor_ops.c by oracle/Makefile) for
    tensor_matmul_int8, tensor_softmax, tensor_topk and tensor_linear;
  * exact closed forms (integer arithmetic, float64) for the rest.
Run from the repo root: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent


def main():
    if not oracle.ref_available():
        raise SystemExit("build the reference library first: make -C oracle")

    # 1. tensor_matmul_int8 known answers (batch 2, odd K, extremes).
    rng = np.random.default_rng(0)
    a = rng.integers(-127, 127, size=(2, 5, 37), dtype=np.int8)
    b = rng.integers(-127, 127, size=(2, 37, 7), dtype=np.int8)
    a[0, 0, :] = 127
    b[0, :, 0] = 127
    a[1, 1, :] = -128
    b[1, :, 1] = -128
    c = oracle.ref_matmul_int8(a, b)
    np.savez_compressed(OUT / "mm_i8_small.npz", a=a, b=b, c=c)

    # 2. C1 GEMV golden (rows truncated to 64 for size), seeds 0..2.
    for seed in range(3):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((1, 1024), dtype=np.float32)
        W = rng.integers(-127, 127, size=(64, 1024), dtype=np.int8)
        s = rng.uniform(0.001, 0.02, size=64).astype(np.float32)
        y = (s.astype(np.float64) * (W.astype(np.float64) @ x[0].astype(np.float64)))[None]
        # The reference fp32 path on dequantized weights (tensor_linear).
        y_ref_lin = oracle.ref_linear(x, (W.astype(np.float32) * s[:, None]))
        np.savez_compressed(OUT / f"gemv_c1_seed{seed}.npz", x=x, W=W, s=s,
                            y_f64=y.astype(np.float64), y_ref_linear=y_ref_lin)

    # 3. Quantizer with exact half-way ties (s = 1 when amax = 127).
    x = np.array([
        [127.0, 2.5, 3.5, -0.5, -1.5, 0.5, 126.5, -126.5, 1.5, -2.5],
        [0.0] * 10,
        [-127.0, 0.49999997, 0.50000006, -64.5, 64.5, 100.5, -100.5, 7.0, -7.0, 0.0],
    ], dtype=np.float32)
    q = np.array([
        [127, 2, 4, 0, -2, 0, 126, -126, 2, -2],
        [0] * 10,
        [-127, 0, 1, -64, 64, 100, -100, 7, -7, 0],
    ], dtype=np.int8)
    s = np.array([1.0, 1.0, 1.0], dtype=np.float32)
    np.savez_compressed(OUT / "quant_tok.npz", x=x, q=q, s=s)

    # 4. Router: reference tensor_softmax + tensor_topk on 16 tokens x 8 experts,
    #    with a planted tie (tokens 0 and 1).
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((16, 8), dtype=np.float32)
    logits[0, 2] = logits[0, 5] = 3.0
    logits[1, :] = 0.25
    p = oracle.ref_softmax(logits)
    v, i = oracle.ref_topk(p, 2)
    np.savez_compressed(OUT / "route_tiny.npz", logits=logits, probs=p, topv=v, topi=i)

    # 5. MoE tiny (8 experts, top-2, 16 tokens, H=128, I=128): oracle output,
    #    fixed so later oracle edits are caught.
    rng = np.random.default_rng(4)
    T, H, I, E, K = 16, 128, 128, 8, 2
    xm = rng.standard_normal((T, H), dtype=np.float32)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    wgu = rng.integers(-127, 127, size=(E, 2 * I, H), dtype=np.int8)
    sgu = rng.uniform(0.001, 0.02, size=(E, 2 * I)).astype(np.float32)
    wd = rng.integers(-127, 127, size=(E, H, I), dtype=np.int8)
    sd = rng.uniform(0.001, 0.02, size=(E, H)).astype(np.float32)
    ym = oracle.moe_w8a8(xm, lg, wgu, sgu, wd, sd, K)
    np.savez_compressed(OUT / "moe_tiny.npz", x=xm, logits=lg, w_gu=wgu, s_gu=sgu, w_down=wd,
                        s_down=sd, y=ym)
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
