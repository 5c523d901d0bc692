"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Tolerances (from the path's correctness bar): int32 accumulators, quantized
bytes and scales are bit-exact; fp32 outputs within rel 1e-3, fp16 outputs
within rel 1e-2 (elementwise, floor 1e-2 * rms; see conftest.assert_rel).
Inputs: numpy default_rng(seed); weights randint(-127, 127) (exclusive upper
bound, so [-127, 126]), scales U(0.001, 0.02), activations N(0, 1).
"""
import sys

import numpy as np
import pytest

import oracle
from conftest import assert_rel

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def env(torch_dev):
    import torch
    from mod_amd import ops
    return torch, ops, torch_dev


def dev(torch, a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    return t.detach().cpu().numpy()


def sync(torch):
    torch.cuda.synchronize()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def _inputs(seed, M, N, K, x_dtype=np.float32):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(x_dtype)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    return x, W, s


# -------------------------------------------------------------------- GEMV
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gemv_c1_fp32(env, seed):
    torch, ops, d = env
    M, N, K = 1, 3072, 1024
    _say(f"gemv C1 seed={seed}")
    x, W, s = _inputs(seed, M, N, K)
    y = torch.empty((M, N), dtype=torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d), None, y, M, N, K, stream(torch))
    sync(torch)
    assert_rel(host(y), oracle.gemv_w8(x, W, s), 1e-3, "gemv C1")


@pytest.mark.parametrize("M,N,K,xdt,ydt,bias", [
    (1, 4096, 1024, np.float32, np.float32, True),     # qkv (bias=True in the reference)
    (1, 1024, 2048, np.float32, np.float32, False),    # o_proj
    (1, 1024, 3072, np.float32, np.float32, False),    # down
    (1, 4000, 1040, np.float32, np.float32, True),     # K tail (not a multiple of 1024)
    (2, 77, 64, np.float32, np.float16, False),        # tiny N, fp16 out
    (3, 12288, 4096, np.float16, np.float16, False),   # Qwen3-8B gate/up, fp16 act
    (4, 4096, 12288, np.float16, np.float16, False),   # Qwen3-8B down
    (16, 1000, 256, np.float16, np.float32, True),
    (64, 512, 512, np.float16, np.float16, False),
])
def test_gemv_shapes(env, M, N, K, xdt, ydt, bias):
    torch, ops, d = env
    _say(f"gemv M={M} N={N} K={K}")
    x, W, s = _inputs(M * 7 + N, M, N, K, xdt)
    b = np.random.default_rng(1).standard_normal(N, dtype=np.float32) if bias else None
    y = torch.empty((M, N), dtype=torch.float16 if ydt == np.float16 else torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d),
                None if b is None else dev(torch, b, d), y, M, N, K, stream(torch))
    sync(torch)
    ref = oracle.gemv_w8(x, W, s, b, out_dtype=ydt)
    assert_rel(host(y).astype(np.float64), ref.astype(np.float64),
               1e-2 if (ydt == np.float16 or xdt == np.float16) else 1e-3, "gemv")


@pytest.mark.parametrize("M,N,K,ydt,bias", [
    (2, 12288, 4096, np.float16, False),   # 1 row tile, 16 blocks, one pass
    (4, 4096, 12288, np.float32, True),    # 12-block K slices + fp32 partials reduce
    (16, 12288, 4096, np.float32, False),
    (16, 3072, 1024, np.float16, True),    # 4 blocks
    (7, 1000, 2048, np.float32, True),     # 8 blocks, ragged N
    (17, 4096, 4096, np.float32, False),   # 4 row tiles (rows 17..63 padded), K slices
    (64, 12288, 4096, np.float16, True),
    (64, 130, 1024, np.float32, True),
    (33, 2048, 12288, np.float16, False),
    (48, 5000, 6144, np.float32, True),    # streamed x, ragged N
    (20, 4096, 1024, np.float16, False),   # streamed x, 4 blocks, 20 live rows of 64
    (64, 1000, 16384, np.float32, False),  # streamed x, 16-block K slices
    (24, 3000, 8192, np.float16, True),    # streamed x, one 32-row tile, K slices, ragged N
])
def test_gemv_mfma_fp16(env, M, N, K, ydt, bias):
    """fp16 activations with 2 <= M <= 64 and K % 1024 == 0 take the MFMA GEMV
    (int8 weights widened exactly to fp16, fp32 accumulation; above 16 rows x
    streams through LDS with the weights). Every product
    is exact, so the fp32 output is held to rel 1e-3 against the oracle (the
    fp16-input bar is 1e-2); fp16 output to 1e-2. Two calls in a row."""
    torch, ops, d = env
    _say(f"gemv mfma M={M} N={N} K={K}")
    x, W, s = _inputs(M * 5 + N + K, M, N, K, np.float16)
    b = np.random.default_rng(2).standard_normal(N, dtype=np.float32) if bias else None
    ref = oracle.gemv_w8(x, W, s, b, out_dtype=ydt)
    xd, wd, sd = dev(torch, x, d), dev(torch, W, d), dev(torch, s, d)
    bd = None if b is None else dev(torch, b, d)
    for rep in range(2):
        y = torch.full((M, N), float("nan"), dtype=torch.float16 if ydt == np.float16 else torch.float32,
                       device=d)
        ops.gemv_w8(xd, wd, sd, bd, y, M, N, K, stream(torch))
        sync(torch)
        assert_rel(host(y).astype(np.float64), ref.astype(np.float64),
                   1e-2 if ydt == np.float16 else 1e-3, f"gemv mfma call {rep}")


@pytest.mark.parametrize("M,N,K,xdt,ydt,bias", [
    (128, 4096, 1024, np.float32, np.float32, True),     # C2 prefill qkv (128-token prompt)
    (128, 1024, 2048, np.float32, np.float32, False),    # prefill o_proj: K in 2 slices
    (128, 1024, 3072, np.float32, np.float32, False),    # prefill down: K in 4 slices
    (128, 6144, 1024, np.float32, np.float32, False),    # prefill gate_up
    (2048, 3072, 1024, np.float32, np.float32, False),   # C1's linear over 2048 rows
    (2048, 3072, 1024, np.float16, np.float16, True),
    (65, 1000, 1040, np.float32, np.float16, True),      # ragged M and N, K % 64 != 0
    (5, 4000, 1040, np.float32, np.float32, True),       # just past the FMA kernels' 4 rows
    (100, 130, 80, np.float16, np.float32, True),        # fp16 x, K % 1024 != 0, one partial step
    (300, 2048, 4096, np.float16, np.float32, False),    # fp16 x past the MFMA GEMVs' 64 rows
])
def test_gemv_many_rows_mfma_gemm(env, M, N, K, xdt, ydt, bias):
    """More than 4 rows (other than fp16 x at 2..64 rows with K % 1024 == 0)
    go to the W8 MFMA GEMM, which reads every weight once per launch: fp32 x
    as three exact bf16 parts, fp16 x as is, int8 weights exact, so only the
    fp32 accumulation rounds -- held to the fp32 bar (rel 1e-3) against the
    float64 oracle, fp16 outputs to 1e-2. Two calls in a row into a NaN-filled
    output (every element written)."""
    torch, ops, d = env
    _say(f"w8 mfma gemm M={M} N={N} K={K} x {np.dtype(xdt).name} y {np.dtype(ydt).name}")
    x, W, s = _inputs(M * 3 + N + K, M, N, K, xdt)
    b = np.random.default_rng(4).standard_normal(N, dtype=np.float32) if bias else None
    ref = oracle.gemv_w8(x, W, s, b, out_dtype=ydt)
    xd, wd, sd = dev(torch, x, d), dev(torch, W, d), dev(torch, s, d)
    bd = None if b is None else dev(torch, b, d)
    for rep in range(2):
        y = torch.full((M, N), float("nan"), dtype=torch.float16 if ydt == np.float16 else torch.float32,
                       device=d)
        ops.gemv_w8(xd, wd, sd, bd, y, M, N, K, stream(torch))
        sync(torch)
        got = host(y).astype(np.float64)
        assert np.isfinite(got).all(), "an output was never written"
        assert_rel(got, ref.astype(np.float64), 1e-2 if ydt == np.float16 else 1e-3, f"w8 mfma gemm call {rep}")


def test_gemv_many_rows_exact_parts(env):
    """The fp32-x MFMA GEMM splits x into bf16 parts exactly: with x values
    that need all 24 significand bits and weight rows +-e_j, every output is
    the selected x value times its (power-of-two) scale, bit for bit: any
    partial sum of the parts' products is then exact, so a part dropped,
    shifted or rounded would show; and scaling the scales by 4 scales y
    exactly."""
    torch, ops, d = env
    M, N, K = 96, 256, 1024
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-20, 20, (M, K)))).astype(np.float32)
    x.view(np.uint32)[:] |= 0x00000001            # the last significand bit set
    sel = rng.integers(0, K, N)
    W = np.zeros((N, K), np.int8)
    W[np.arange(N), sel] = rng.choice([-1, 1], N).astype(np.int8)
    s = np.exp2(rng.integers(-8, 0, N)).astype(np.float32)   # powers of two: exact products
    y = torch.empty((M, N), dtype=torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d), None, y, M, N, K, stream(torch))
    sync(torch)
    want = (x[:, sel].astype(np.float64) * W[np.arange(N), sel].astype(np.float64) * s).astype(np.float32)
    assert np.array_equal(host(y), want)
    y2 = torch.empty((M, N), dtype=torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s * 4, d), None, y2, M, N, K, stream(torch))
    sync(torch)
    assert np.array_equal(host(y2), host(y) * 4)


@pytest.mark.parametrize("M,N,K,xdt", [
    (1, 151936, 1024, np.float16),   # lm_head-sized N: many row groups per wave
    (5, 20000, 4096, np.float16),    # fp16 x at 2 <= M <= 64: the MFMA GEMV
    (1, 50001, 3072, np.float32),    # 4-row groups, ragged last group
    (5, 20000, 4096, np.float32),    # more than 4 fp32 rows: the MFMA GEMM
    (2, 4096, 12288, np.float32),    # stream kernel: one 2-x-row launch
    (9, 12288, 4096, np.float32),    # the MFMA GEMM, 9 live rows of a 64-row tile
])
def test_gemv_many_row_groups(env, M, N, K, xdt):
    """Large N: every persistent wave walks many row groups; every output must
    be written exactly once with the oracle's value (y starts as NaN)."""
    torch, ops, d = env
    _say(f"gemv many groups M={M} N={N} K={K}")
    x, W, s = _inputs(N + K, M, N, K, xdt)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d), None, y, M, N, K)
    sync(torch)
    got = host(y)
    assert np.isfinite(got).all(), "an output row was never written"
    assert_rel(got, oracle.gemv_w8(x, W, s), 1e-2 if xdt == np.float16 else 1e-3, "gemv many groups")


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288), (151936, 4096)])
def test_gemv_stream_fp16_in_out(env, N, K):
    """The fp16-in / fp16-out stream GEMV at M = 1 (the
    Qwen3-8B linears and lm_head), against the oracle at the fp16 bar. For the
    lm_head the oracle runs on a subset of rows (first, last and 4096 random
    ones): each output row depends only on its weight row."""
    torch, ops, d = env
    M = 1
    _say(f"gemv fp16 stream M=1 N={N} K={K}")
    x, W, s = _inputs(N + 3 * K, M, N, K, np.float16)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d), None, y, M, N, K)
    sync(torch)
    got = host(y).astype(np.float64)
    assert np.isfinite(got).all(), "an output row was never written"
    if N > 20000:
        rows = np.unique(np.concatenate([[0, 1, N - 1],
                                         np.random.default_rng(5).integers(0, N, 4096)]))
        W, s, got = W[rows], s[rows], got[:, rows]
    ref = oracle.gemv_w8(x, W, s, out_dtype=np.float16).astype(np.float64)
    assert_rel(got, ref, 1e-2, "gemv fp16 stream")


def test_gemv_repeated_launches_identical(env):
    """Back-to-back launches, interleaved with another shape, give
    bit-identical outputs (each output's sum has one fixed order)."""
    torch, ops, d = env
    M, N, K = 1, 40000, 2048
    x, W, s = _inputs(11, M, N, K)
    xd, wd, sd = dev(torch, x, d), dev(torch, W, d), dev(torch, s, d)
    x2, W2, s2 = _inputs(12, 2, 3000, 1024)
    outs = []
    for i in range(70):
        y = torch.empty((M, N), dtype=torch.float32, device=d)
        ops.gemv_w8(xd, wd, sd, None, y, M, N, K)
        if i % 7 == 0:
            y2 = torch.empty((2, 3000), dtype=torch.float32, device=d)
            ops.gemv_w8(dev(torch, x2, d), dev(torch, W2, d), dev(torch, s2, d), None, y2, 2, 3000, 1024)
        if i % 10 == 0:
            outs.append(y)
    sync(torch)
    first = host(outs[0])
    for o in outs[1:]:
        assert np.array_equal(host(o).view(np.uint32), first.view(np.uint32))
    assert_rel(first, oracle.gemv_w8(x, W, s), 1e-3, "gemv repeated")


def test_gemv_extreme_weights(env):
    torch, ops, d = env
    M, N, K = 1, 64, 2048
    rng = np.random.default_rng(3)
    x = rng.standard_normal((M, K), dtype=np.float32)
    W = np.full((N, K), 127, np.int8)
    W[1::2] = -128
    s = np.full(N, 0.01, np.float32)
    y = torch.empty((M, N), dtype=torch.float32, device=d)
    ops.gemv_w8(dev(torch, x, d), dev(torch, W, d), dev(torch, s, d), None, y, M, N, K)
    sync(torch)
    assert_rel(host(y), oracle.gemv_w8(x, W, s), 1e-3, "gemv extremes")


# --------------------------------------------------------------- quantizer
@pytest.mark.parametrize("M,K,xdt", [(2048, 1024, np.float16), (2048, 3072, np.float16),
                                     (17, 1000, np.float32), (5, 13, np.float32),
                                     (512, 2048, np.float16), (3, 12288, np.float32),
                                     (1, 12288, np.float16), (64, 4096, np.float16),
                                     (1030, 8200, np.float32), (1500, 520, np.float16)])
def test_quant_bitexact(env, M, K, xdt):
    torch, ops, d = env
    _say(f"quant M={M} K={K}")
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K), dtype=np.float32) * rng.uniform(0.1, 10, (M, 1)).astype(np.float32)).astype(xdt)
    x[0] = 0
    q = torch.empty((M, K), dtype=torch.int8, device=d)
    s = torch.empty((M,), dtype=torch.float32, device=d)
    ops.quantize_per_token(dev(torch, x, d), q, s, M, K, stream(torch))
    sync(torch)
    qr, sr = oracle.quant_per_token(x)
    assert np.array_equal(host(s).view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(host(q), qr)


def test_quant_golden_ties(env):
    torch, ops, d = env
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "quant_tok.npz")
    x = g["x"]
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=d)
    s = torch.empty((M,), dtype=torch.float32, device=d)
    ops.quantize_per_token(dev(torch, x, d), q, s, M, K)
    sync(torch)
    assert np.array_equal(host(q), g["q"]) and np.array_equal(host(s), g["s"])


# ------------------------------------------------- RMSNorm -> quantizer (f2)
@pytest.mark.parametrize("M,K,xdt,res", [(2048, 1024, np.float16, False), (2048, 1024, np.float16, True),
                                         (7, 3072, np.float32, False), (5, 3072, np.float32, True),
                                         (2048, 3072, np.float16, False), (2048, 3072, np.float16, True),
                                         (3, 8, np.float32, False), (9, 1000, np.float16, True),
                                         (4, 4096, np.float32, True), (2, 8192, np.float16, False),
                                         (3, 32768, np.float32, False), (130, 512, np.float16, False)])
def test_rmsnorm_quant_bitexact(env, M, K, xdt, res):
    """Fused RMSNorm (+ residual) -> per-token quantizer: q, s and the stored
    sum bit-exact against the oracle, which fixes the order of the sum of
    squares (every thread/LDS/butterfly tree level of the kernel's layouts:
    64, 128 and 256 threads per row, 1..16 chunks per thread, padded chunk
    counts such as K = 1000)."""
    torch, ops, d = env
    _say(f"rmsnorm_quant M={M} K={K} {np.dtype(xdt).name} residual={res}")
    rng = np.random.default_rng(M * 7 + K)
    x = (rng.standard_normal((M, K), dtype=np.float32) * rng.uniform(0.1, 10, (M, 1)).astype(np.float32)).astype(xdt)
    x[0] = 0
    r = rng.standard_normal((M, K), dtype=np.float32).astype(xdt) if res else None
    if res:
        r[0] = 0
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    eps = 1e-6
    xd = dev(torch, x, d)
    q = torch.empty((M, K), dtype=torch.int8, device=d)
    s = torch.empty((M,), dtype=torch.float32, device=d)
    rd = dev(torch, r, d) if res else None
    ops.rmsnorm_quant(xd, dev(torch, w, d), q, s, M, K, eps, residual=rd, x_sum=xd if res else None,
                      stream=stream(torch))
    sync(torch)
    qr, sr, _, xs = oracle.rmsnorm_quant(x, w, eps, residual=r)
    assert np.array_equal(host(s).view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(host(q), qr)
    if res:
        assert np.array_equal(host(xd).view(np.uint8), xs.view(np.uint8))
    assert np.all(host(q)[0] == 0) and host(s)[0] == 1.0


def test_rmsnorm_quant_rejects(env):
    torch, ops, d = env
    x = torch.zeros((2, 12), dtype=torch.float32, device=d)
    w = torch.ones((12,), dtype=torch.float32, device=d)
    q = torch.empty((2, 12), dtype=torch.int8, device=d)
    s = torch.empty((2,), dtype=torch.float32, device=d)
    with pytest.raises(ops.RocmError, match="multiple of 8"):
        ops.rmsnorm_quant(x, w, q, s, 2, 12)
    with pytest.raises(ops.RocmError, match="go together"):
        ops.rmsnorm_quant(x, w, q, s, 2, 8, residual=x)


# -------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(2048, 3072, 1024), (2048, 1024, 3072), (2048, 2048, 1024),
                                   (1, 64, 16), (130, 200, 80), (257, 129, 1040), (64, 4096, 4096)])
def test_gemm_int32_bitexact(env, M, N, K):
    torch, ops, d = env
    _say(f"gemm i32 M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    c = torch.empty((M, N), dtype=torch.int32, device=d)
    ops.gemm_w8a8(dev(torch, q, d), None, dev(torch, W, d), None, None, c, M, N, K, stream(torch))
    sync(torch)
    assert np.array_equal(host(c), oracle.matmul_nt_i32(q, W))


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 128), (4096, 4096, 256), (4096, 4096, 640),
                                   (4000, 4000, 640), (2048, 8192, 512)])
def test_gemm_big_tile_int32_bitexact(env, M, N, K):
    """Grids of >= 256 tiles of 256 x 256 take the 256 x 256 engine (half-step
    LDS ring): one and two K steps, a ring in steady state, ragged tile edges.
    Three launches each, every one bit-exact (a timing-dependent fault in the
    copy/read pipeline would show as a mismatch in some launch)."""
    torch, ops, d = env
    _say(f"gemm big tile M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K + 1)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    ref = oracle.matmul_nt_i32(q, W)
    qd, wd = dev(torch, q, d), dev(torch, W, d)
    for _ in range(3):
        c = torch.full((M, N), -1, dtype=torch.int32, device=d)
        ops.gemm_w8a8(qd, None, wd, None, None, c, M, N, K)
        sync(torch)
        assert np.array_equal(host(c), ref)


def test_gemm_big_tile_fp16_scaled(env):
    """The 256 x 256 engine's scaled fp16 epilogue, byte-equal to the oracle."""
    torch, ops, d = env
    M, N, K = 4096, 4096, 512
    rng = np.random.default_rng(77)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    y = torch.empty((M, N), dtype=torch.float16, device=d)
    ops.gemm_w8a8(dev(torch, q, d), dev(torch, sa, d), dev(torch, W, d), dev(torch, sw, d), dev(torch, b, d),
                  y, M, N, K)
    sync(torch)
    yr = oracle.w8a8(q, sa, W, sw, b, out="f16")
    assert np.array_equal(host(y).view(np.uint16), yr.view(np.uint16))


@pytest.mark.parametrize("M,N,K", [(1, 12288, 4096), (16, 12288, 4096), (64, 12288, 4096),
                                   (64, 4096, 12288), (100, 1000, 2048), (33, 1536, 2048),
                                   (256, 3072, 1024), (7, 130, 1536)])
def test_gemm_split_k(env, M, N, K):
    """Skinny M takes the split-K path (K slices as a batch into int32
    partials, summed in slice order): int32 bit-exact, and the scaled fp16 /
    fp32 outputs (with bias) byte-equal to the oracle, on two calls in a row
    (the partial workspace is reused)."""
    torch, ops, d = env
    _say(f"split-K M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 7 + N + K)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    qd, Wd, sad, swd, bd = (dev(torch, a, d) for a in (q, W, sa, sw, b))
    acc_ref = oracle.matmul_nt_i32(q, W)
    for rep in range(2):
        acc = torch.full((M, N), 7, dtype=torch.int32, device=d)
        y16 = torch.full((M, N), float("nan"), dtype=torch.float16, device=d)
        y32 = torch.full((M, N), float("nan"), dtype=torch.float32, device=d)
        ops.gemm_w8a8(qd, None, Wd, None, None, acc, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, bd, y16, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, None, y32, M, N, K)
        sync(torch)
        assert np.array_equal(host(acc), acc_ref), f"int32 call {rep}"
        yr16 = oracle.w8a8(q, sa, W, sw, b, out="f16")
        assert np.array_equal(host(y16).view(np.uint16), yr16.view(np.uint16)), f"f16 call {rep}"
        yr32 = oracle.w8a8(q, sa, W, sw, None, out="f32")
        assert np.array_equal(host(y32).view(np.uint32), yr32.view(np.uint32)), f"f32 call {rep}"


@pytest.mark.parametrize("seed", range(12))
def test_gemm_skinny_random_shapes(env, seed):
    """Seeded random skinny shapes (M 1..64, N 1..2048, K 1024..8192 in steps
    of 1024): every plan the skinny planners pick for them (one-pass or
    streamed, any slice count) is int32 bit-exact and fp16 byte-equal (with
    bias) to the oracle, on two calls in a row."""
    torch, ops, d = env
    rng = np.random.default_rng(7000 + seed)
    M, N, K = int(rng.integers(1, 65)), int(rng.integers(1, 2049)), 1024 * int(rng.integers(1, 9))
    _say(f"skinny random M={M} N={N} K={K}")
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    qd, Wd, sad, swd, bd = (dev(torch, a, d) for a in (q, W, sa, sw, b))
    acc_ref = oracle.matmul_nt_i32(q, W)
    yr16 = oracle.w8a8(q, sa, W, sw, b, out="f16")
    for rep in range(2):
        acc = torch.full((M, N), 7, dtype=torch.int32, device=d)
        y16 = torch.full((M, N), float("nan"), dtype=torch.float16, device=d)
        ops.gemm_w8a8(qd, None, Wd, None, None, acc, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, bd, y16, M, N, K)
        sync(torch)
        assert np.array_equal(host(acc), acc_ref), f"int32 call {rep}"
        assert np.array_equal(host(y16).view(np.uint16), yr16.view(np.uint16)), f"f16 call {rep}"


@pytest.mark.parametrize("seed", range(12))
def test_gemv_mfma_random_shapes(env, seed):
    """Seeded random fp16-x GEMV shapes (M 2..64, N 1..2048, K 1024..8192 in
    steps of 1024), so both MFMA GEMVs, every tile count and K slicing meet
    ragged N, with and without bias, fp32 or fp16 output: held to the oracle
    at rel 1e-3 (fp32 out) / 1e-2 (fp16 out)."""
    torch, ops, d = env
    rng = np.random.default_rng(8000 + seed)
    M, N, K = int(rng.integers(2, 65)), int(rng.integers(1, 2049)), 1024 * int(rng.integers(1, 9))
    ydt = np.float16 if seed % 2 else np.float32
    bias = seed % 3 != 0
    _say(f"gemv mfma random M={M} N={N} K={K} y={ydt.__name__} bias={bias}")
    x, W, s = _inputs(9000 + seed, M, N, K, np.float16)
    b = rng.standard_normal(N, dtype=np.float32) if bias else None
    ref = oracle.gemv_w8(x, W, s, b, out_dtype=ydt)
    xd, wd, sd = dev(torch, x, d), dev(torch, W, d), dev(torch, s, d)
    bd = None if b is None else dev(torch, b, d)
    for rep in range(2):
        y = torch.full((M, N), float("nan"), dtype=torch.float16 if ydt == np.float16 else torch.float32,
                       device=d)
        ops.gemv_w8(xd, wd, sd, bd, y, M, N, K, stream(torch))
        sync(torch)
        assert_rel(host(y).astype(np.float64), ref.astype(np.float64),
                   1e-2 if ydt == np.float16 else 1e-3, f"gemv mfma random call {rep}")


@pytest.mark.parametrize("M,N,K", [(1, 12288, 4096), (16, 12288, 4096), (64, 12288, 4096),
                                   (1, 4096, 12288), (16, 4096, 12288), (64, 4096, 12288),
                                   (16, 3072, 1024),
                                   (64, 3072, 1024), (1, 1024, 3072), (5, 1000, 2048),
                                   (17, 1000, 2048), (20, 200, 12288), (3, 48, 4096),
                                   (64, 130, 1024)])
def test_gemm_skinny(env, M, N, K):
    """M <= 64 with K % 1024 == 0 takes the skinny kernel (weights streamed
    into registers, the activation slice in LDS, 16x16x64 MFMAs; one pass or
    K slices into int32 partials). The shapes cover both row tilings (M <= 16
    and up to 64), both workgroup widths, 4/8/12/16 blocks per slice, one to
    twelve slices and ragged N. int32 bit-exact, fp16 / fp32 (with and
    without bias) byte-equal to the oracle, two calls in a row."""
    torch, ops, d = env
    _say(f"skinny M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 131 + N + 3 * K)
    q = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    qd, Wd, sad, swd, bd = (dev(torch, a, d) for a in (q, W, sa, sw, b))
    acc_ref = oracle.matmul_nt_i32(q, W)
    yr16 = oracle.w8a8(q, sa, W, sw, b, out="f16")
    yr32 = oracle.w8a8(q, sa, W, sw, None, out="f32")
    yr32b = oracle.w8a8(q, sa, W, sw, b, out="f32")
    for rep in range(2):
        acc = torch.full((M, N), 7, dtype=torch.int32, device=d)
        y16 = torch.full((M, N), float("nan"), dtype=torch.float16, device=d)
        y32 = torch.full((M, N), float("nan"), dtype=torch.float32, device=d)
        y32b = torch.full((M, N), float("nan"), dtype=torch.float32, device=d)
        ops.gemm_w8a8(qd, None, Wd, None, None, acc, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, bd, y16, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, None, y32, M, N, K)
        ops.gemm_w8a8(qd, sad, Wd, swd, bd, y32b, M, N, K)
        sync(torch)
        assert np.array_equal(host(acc), acc_ref), f"int32 call {rep}"
        assert np.array_equal(host(y16).view(np.uint16), yr16.view(np.uint16)), f"f16 call {rep}"
        assert np.array_equal(host(y32).view(np.uint32), yr32.view(np.uint32)), f"f32 call {rep}"
        assert np.array_equal(host(y32b).view(np.uint32), yr32b.view(np.uint32)), f"f32+bias call {rep}"


@pytest.mark.parametrize("K,N", [(1024, 3072), (3072, 1024), (1024, 2048)])
def test_gemm_c3_fp16_pipeline(env, K, N):
    """C3: x fp16 -> per-token quant -> W8A8 GEMM -> fp16, vs the oracle."""
    torch, ops, d = env
    M = 2048
    _say(f"C3 K={K} N={N}")
    rng = np.random.default_rng(K + N)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    q = torch.empty((M, K), dtype=torch.int8, device=d)
    sa = torch.empty((M,), dtype=torch.float32, device=d)
    y = torch.empty((M, N), dtype=torch.float16, device=d)
    acc = torch.empty((M, N), dtype=torch.int32, device=d)
    wd = dev(torch, W, d)
    swd = dev(torch, sw, d)
    ops.quantize_per_token(dev(torch, x, d), q, sa, M, K)
    ops.gemm_w8a8(q, sa, wd, swd, None, y, M, N, K)
    ops.gemm_w8a8(q, None, wd, None, None, acc, M, N, K)
    sync(torch)
    qr, sr = oracle.quant_per_token(x)
    assert np.array_equal(host(q), qr)
    assert np.array_equal(host(acc), oracle.matmul_nt_i32(qr, W))
    yr = oracle.w8a8(qr, sr, W, sw, out="f16")
    got = host(y)
    assert_rel(got.astype(np.float64), yr.astype(np.float64), 1e-2, "C3 fp16")
    # same formula and rounding on both sides: expect byte equality
    assert np.array_equal(got.view(np.uint16), yr.view(np.uint16))


def test_gemm_fp32_bias(env):
    torch, ops, d = env
    M, N, K = 100, 300, 512
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, N).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    y = torch.empty((M, N), dtype=torch.float32, device=d)
    ops.gemm_w8a8(dev(torch, q, d), dev(torch, sa, d), dev(torch, W, d), dev(torch, sw, d),
                  dev(torch, b, d), y, M, N, K)
    sync(torch)
    assert_rel(host(y), oracle.w8a8(q, sa, W, sw, b, out="f32"), 1e-5, "gemm f32 bias")


# ------------------------------------------------- tensor_matmul_int8 (a1)
@pytest.mark.parametrize("batch,M,K,N", [(1, 1, 1024, 3072), (2, 5, 37, 7), (3, 64, 1023, 65),
                                         (1, 128, 256, 128)])
def test_matmul_int8_matches_reference_semantics(env, batch, M, K, N):
    torch, ops, d = env
    _say(f"matmul_int8 b={batch} M={M} K={K} N={N}")
    rng = np.random.default_rng(batch * 1000 + K)
    a = rng.integers(-127, 127, size=(batch, M, K), dtype=np.int8)
    b = rng.integers(-127, 127, size=(batch, K, N), dtype=np.int8)
    c = torch.empty((batch, M, N), dtype=torch.float32, device=d)
    ci = torch.empty((batch, M, N), dtype=torch.int32, device=d)
    ad, bd = dev(torch, a, d), dev(torch, b, d)
    ops.matmul_int8(ad, bd, c, batch, M, K, N, out_i32=False)
    ops.matmul_int8(ad, bd, ci, batch, M, K, N, out_i32=True)
    sync(torch)
    ref = oracle.matmul_int8(a, b)
    assert np.array_equal(host(c).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(host(ci), oracle.matmul_int8(a, b, out_i32=True))
    if oracle.ref_available():
        assert np.array_equal(host(c), oracle.ref_matmul_int8(a, b).reshape(c.shape))


@pytest.mark.parametrize("batch,M,K,N,b_off,ws_off", [
    (1, 256, 1024, 3072, 0, 0),   # C3-sized b: whole 16-byte chunks in and out
    (2, 100, 200, 80, 0, 0),      # N % 16 == 0 with a partial tile on each edge, Kp = 208
    (2, 100, 200, 80, 1, 0),      # b one byte off alignment: byte reads
    (1, 70, 96, 48, 0, 3),        # caller workspace off alignment: refused
])
def test_matmul_int8_b_layouts(env, batch, M, K, N, b_off, ws_off):
    """The [K,N] -> [N,Kp] repack of b inside tensor_matmul_int8 on its
    16-byte and byte read paths, int32 results against the oracle; a caller
    workspace off 16-byte alignment is refused."""
    torch, ops, d = env
    _say(f"matmul_int8 layouts b={batch} M={M} K={K} N={N} b_off={b_off} ws_off={ws_off}")
    rng = np.random.default_rng(M * 7 + K)
    a = rng.integers(-128, 128, size=(batch, M, K), dtype=np.int8)
    b = rng.integers(-128, 128, size=(batch, K, N), dtype=np.int8)
    bbuf = torch.empty(b.size + 16, dtype=torch.int8, device=d)
    bd = bbuf[b_off:b_off + b.size]
    bd.copy_(torch.from_numpy(b.reshape(-1)).to(d))
    nws = int(ops.lib.pio_matmul_int8_workspace(batch, M, K, N))
    ws = torch.empty(nws + 16, dtype=torch.uint8, device=d)[ws_off:ws_off + nws]
    ci = torch.empty((batch, M, N), dtype=torch.int32, device=d)
    if ws_off % 16:
        with pytest.raises(RuntimeError, match="16-byte aligned"):
            ops.matmul_int8(dev(torch, a, d), bd, ci, batch, M, K, N, out_i32=True, workspace=ws)
        return
    ops.matmul_int8(dev(torch, a, d), bd, ci, batch, M, K, N, out_i32=True, workspace=ws)
    sync(torch)
    assert np.array_equal(host(ci), oracle.matmul_int8(a, b, out_i32=True))


# --------------------------------------------------------------------- MoE
def test_moe_route_matches_oracle(env):
    torch, ops, d = env
    T, E, k = 512, 128, 8
    rng = np.random.default_rng(21)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    lg[0, :] = 0.5          # all-equal row: ids 0..7
    lg[1, 3] = lg[1, 9] = 9.0
    for renorm in (False, True):
        w = torch.empty((T, k), dtype=torch.float32, device=d)
        i = torch.empty((T, k), dtype=torch.int32, device=d)
        ops.moe_route(dev(torch, lg, d), w, i, T, E, k, renorm)
        sync(torch)
        wr, ir = oracle.moe_route(lg, k, renorm)
        assert np.array_equal(host(i), ir)
        assert_rel(host(w), wr, 1e-5, "route weights")
    assert list(host(i)[0]) == list(range(8))


# (H, I) / 128 = the expert GEMMs' K steps: 1, 2, 3, 4 (= the prefetch depth),
# 5, 6, 9, 16 and 32 (the largest supported), around the engine's prologue and
# tail cases; T = 160 with 2 experts also takes the 64-row second tile pass;
# T = 4100 gives ~2050 rows per expert (33 row tiles); T = 2048 runs the
# grouping kernel's token walk in 4 rounds of 512.
@pytest.mark.parametrize("T,H,I,E,k,xdt", [(16, 128, 128, 8, 2, np.float32),
                                           (64, 256, 128, 16, 4, np.float16),
                                           (48, 384, 512, 8, 2, np.float32),
                                           (64, 512, 640, 16, 4, np.float16),
                                           (130, 1152, 128, 32, 8, np.float16),
                                           (160, 4096, 256, 2, 1, np.float32),
                                           (512, 2048, 768, 128, 8, np.float16),
                                           (2048, 256, 128, 8, 4, np.float16),
                                           (4100, 128, 128, 4, 2, np.float32)])
def test_moe_layer_matches_oracle(env, T, H, I, E, k, xdt):
    torch, ops, d = env
    _say(f"moe T={T} H={H} I={I} E={E} k={k}")
    rng = np.random.default_rng(T + E)
    x = rng.standard_normal((T, H), dtype=np.float32).astype(xdt)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    wgu = rng.integers(-127, 127, size=(E, 2 * I, H), dtype=np.int8)
    sgu = rng.uniform(0.001, 0.02, size=(E, 2 * I)).astype(np.float32)
    wd = rng.integers(-127, 127, size=(E, H, I), dtype=np.int8)
    sd = rng.uniform(0.001, 0.02, size=(E, H)).astype(np.float32)
    out = torch.empty((T, H), dtype=torch.float32, device=d)
    ops.moe_w8a8(dev(torch, x, d), dev(torch, lg, d), dev(torch, wgu, d), dev(torch, sgu, d),
                 dev(torch, wd, d), dev(torch, sd, d), out, T, H, I, E, k, False)
    sync(torch)
    ref = oracle.moe_w8a8(x, lg, wgu, sgu, wd, sd, k)
    # quantized x, the expert GEMMs' int32 sums, SwiGLU (deterministic exp)
    # and the requantized h are bit-identical to the oracle's (a flipped byte
    # would show as ~1e-3); what remains is the router's expf (libm vs device
    # library, last ulp of a routing weight), amplified where the k-sum
    # cancels (observed up to 1.7e-5 at the 1e-2 * rms floor)
    assert_rel(host(out), ref, 1e-4, "moe")


@pytest.mark.parametrize("bias_experts", [(5, 9), (0, 1, 2, 3)])
def test_moe_skewed_routing(env, bias_experts):
    """Routing concentrated on a few experts: most experts get no rows (their
    GEMM blocks find an empty range and write nothing), the chosen ones get
    every token (several 64-row tiles each); against the oracle."""
    torch, ops, d = env
    T, H, I, E, k = 300, 256, 128, 64, 2
    _say(f"moe skewed routing to experts {bias_experts}")
    rng = np.random.default_rng(77 + len(bias_experts))
    x = rng.standard_normal((T, H), dtype=np.float32)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    for j, e in enumerate(bias_experts):
        lg[:, e] += 20.0 - j
    wgu = rng.integers(-127, 127, size=(E, 2 * I, H), dtype=np.int8)
    sgu = rng.uniform(0.001, 0.02, size=(E, 2 * I)).astype(np.float32)
    wd = rng.integers(-127, 127, size=(E, H, I), dtype=np.int8)
    sd = rng.uniform(0.001, 0.02, size=(E, H)).astype(np.float32)
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device=d)
    ops.moe_w8a8(dev(torch, x, d), dev(torch, lg, d), dev(torch, wgu, d), dev(torch, sgu, d),
                 dev(torch, wd, d), dev(torch, sd, d), out, T, H, I, E, k, False)
    sync(torch)
    _, ids = oracle.moe_route(lg, k, False)
    assert set(np.unique(ids)) <= set(bias_experts)
    ref = oracle.moe_w8a8(x, lg, wgu, sgu, wd, sd, k)
    got = host(out)
    assert np.isfinite(got).all()
    assert_rel(got, ref, 1e-4, "moe skewed")


@pytest.mark.parametrize("renorm", [False, True])
def test_moe_c5_fp16_out_matches_oracle(env, renorm):
    """The full C5 layer (512 tokens, H 2048, I 768, 128 experts, top-8) with
    fp16 x and fp16 output -- the instantiation the benchmark times
    (moe_combine_kernel<_Float16>) -- with and without renormalized top-k
    weights. Held at the fp16 bar (rel 1e-2); the combine's fp32 sums agree
    with the oracle to the router's last ulp, so nearly every fp16 output is
    the same bytes (the count is asserted and reported). With renormalized
    weights a few outputs pass the fp16 range; they must be the oracle's
    infinities."""
    torch, ops, d = env
    T, H, I, E, k = 512, 2048, 768, 128, 8
    _say(f"moe C5 fp16 out renorm={renorm}")
    rng = np.random.default_rng(515 + int(renorm))
    x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    wgu = rng.integers(-127, 127, size=(E, 2 * I, H), dtype=np.int8)
    sgu = rng.uniform(0.001, 0.02, size=(E, 2 * I)).astype(np.float32)
    wd = rng.integers(-127, 127, size=(E, H, I), dtype=np.int8)
    sd = rng.uniform(0.001, 0.02, size=(E, H)).astype(np.float32)
    out = torch.empty((T, H), dtype=torch.float16, device=d)
    ops.moe_w8a8(dev(torch, x, d), dev(torch, lg, d), dev(torch, wgu, d), dev(torch, sgu, d),
                 dev(torch, wd, d), dev(torch, sd, d), out, T, H, I, E, k, renorm)
    sync(torch)
    ref = oracle.moe_w8a8(x, lg, wgu, sgu, wd, sd, k, renorm=renorm, out_dtype=np.float16)
    got = host(out)
    # renormalized weights sum to 1, so a few outputs pass 65504 and round to
    # +-inf in fp16 -- in the oracle too: they must be the same infinities
    inf = ~np.isfinite(ref)
    assert not np.isnan(got).any()
    assert np.array_equal(~np.isfinite(got), inf) and np.array_equal(got[inf], ref[inf])
    _say(f"  outputs past the fp16 range: {int(inf.sum())}")
    assert_rel(np.where(inf, 0, got).astype(np.float32), np.where(inf, 0, ref).astype(np.float32),
               1e-2, "moe fp16 out")
    same = float(np.mean(got.view(np.uint16) == ref.view(np.uint16)))
    _say(f"  byte-equal fp16 outputs: {same * 100:.3f}%")
    assert same >= 0.99


def test_moe_tiny_golden(env):
    torch, ops, d = env
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "moe_tiny.npz")
    T, H = g["x"].shape
    E, I2, _ = g["w_gu"].shape
    out = torch.empty((T, H), dtype=torch.float32, device=d)
    ops.moe_w8a8(dev(torch, g["x"], d), dev(torch, g["logits"], d), dev(torch, g["w_gu"], d),
                 dev(torch, g["s_gu"], d), dev(torch, g["w_down"], d), dev(torch, g["s_down"], d),
                 out, T, H, I2 // 2, E, 2, False)
    sync(torch)
    assert_rel(host(out), g["y"], 1e-4, "moe golden")


def test_skinny_paths_full_size_properties(env):
    """At the Qwen3-8B lm_head size (M = 16, N = 151936, K = 4096), where the
    oracle would take minutes, properties the arithmetic fixes:
    - MFMA GEMV (fp16 x, fp32 y): products are exact and the accumulation
      scales exactly by 2, so y(2x) == 2 y(x) bit for bit. Under a sign flip
      of W the result mirrors only to within a few ulp: the f16 MFMA's fp32
      accumulation does not round to nearest-even (measured: about 0.06% of
      outputs move by 1-4 ulp, the negative side larger, as rounding toward
      -inf does), so y(x; -W) == -y(x; W) is held to 8 ulp of max |y|;
    - skinny W8A8 (int32 out): acc(q; -W) == -acc(q; W) exactly, and a few
      rows equal the oracle's int32 dot products."""
    torch, ops, d = env
    M, N, K = 16, 151936, 4096
    _say(f"skinny full-size properties M={M} N={N} K={K}")
    rng = np.random.default_rng(99)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    Wd, Wn = dev(torch, W, d), dev(torch, -W, d)
    s = dev(torch, rng.uniform(0.001, 0.02, size=N).astype(np.float32), d)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    xd, x2d = dev(torch, x, d), dev(torch, (x.astype(np.float32) * 2).astype(np.float16), d)
    y, y2, yn = (torch.empty((M, N), dtype=torch.float32, device=d) for _ in range(3))
    ops.gemv_w8(xd, Wd, s, None, y, M, N, K)
    ops.gemv_w8(x2d, Wd, s, None, y2, M, N, K)
    ops.gemv_w8(xd, Wn, s, None, yn, M, N, K)
    sync(torch)
    hy = host(y)
    assert np.isfinite(hy).all()
    assert np.array_equal(host(y2), 2 * hy)
    # the accumulation error scales with the partial sums, not with outputs
    # that cancel to near zero: bound it by 8 ulp of the largest output
    assert np.abs(host(yn) + hy).max() <= 8 * np.spacing(np.float32(np.abs(hy).max()))
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    qd = dev(torch, q, d)
    acc, accn = (torch.empty((M, N), dtype=torch.int32, device=d) for _ in range(2))
    ops.gemm_w8a8(qd, None, Wd, None, None, acc, M, N, K)
    ops.gemm_w8a8(qd, None, Wn, None, None, accn, M, N, K)
    sync(torch)
    ha = host(acc)
    assert np.array_equal(host(accn), -ha)
    rows = [0, 1, 77, 4095, 100000, N - 1]
    assert np.array_equal(ha[:, rows], oracle.matmul_nt_i32(q, W[rows]))
