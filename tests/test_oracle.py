"""Pins the CPU oracle (oracle/int8_ref.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the reference library itself (compiled from the reference sources by
oracle/Makefile), exact integer / float64 closed forms, brute force on tiny
inputs, invariants, and the golden fixtures under tests/golden/.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLD = Path(__file__).resolve().parent / "golden"
needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


# ------------------------------------------------------------------- fp16
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, np.inf,
                         -np.inf, 6.1035156e-05, 6.1035152e-05, 5.9604645e-08, 2.9802322e-08,
                         2.9802326e-08, 8.940697e-08, 1e-10, 0.33333334, 2049.0, 2051.0, 2050.0,
                         1025.5, 1024.5], dtype=np.float32)
    r = np.concatenate([
        specials,
        rng.standard_normal(200000).astype(np.float32) * 100,
        (rng.standard_normal(100000) * 1e-5).astype(np.float32),
        rng.uniform(-70000, 70000, 50000).astype(np.float32),
    ])
    got = oracle.f32_to_f16_bits(r)
    exp = r.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)
    # exact half-way points between neighbouring halves round to even
    h = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float32)
    mid = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    assert np.array_equal(oracle.f32_to_f16_bits(mid), mid.astype(np.float16).view(np.uint16))


def test_f16_nan_stays_nan():
    got = oracle.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(got.view(np.float16)[0])


# ------------------------------------------------------------ int8 matmul
@needs_ref
@pytest.mark.parametrize("shape", [(1, 1, 64, 3072), (1, 7, 33, 5), (2, 4, 1023, 9),
                                   (3, 2, 1025, 17), (1, 16, 256, 64)])
def test_matmul_int8_bitwise_vs_reference(shape):
    batch, m, k, n = shape
    rng = np.random.default_rng(sum(shape))
    a = rng.integers(-127, 127, size=(batch, m, k), dtype=np.int8)
    b = rng.integers(-127, 127, size=(batch, k, n), dtype=np.int8)
    ours = oracle.matmul_int8(a, b)
    ref = oracle.ref_matmul_int8(a, b)
    assert ours.dtype == np.float32
    assert np.array_equal(ours.view(np.uint32), ref.reshape(ours.shape).view(np.uint32))


@needs_ref
def test_matmul_int8_both_reference_builds_agree():
    rng = np.random.default_rng(9)
    a = rng.integers(-127, 127, size=(2, 8, 100), dtype=np.int8)
    b = rng.integers(-127, 127, size=(2, 100, 12), dtype=np.int8)
    r1 = oracle.ref_matmul_int8(a, b)
    r2 = oracle.ref_matmul_int8(a, b, lib_=oracle.ref_lib(buildops_flags=True))
    assert np.array_equal(r1, r2)


def test_matmul_int8_closed_form_and_extremes():
    rng = np.random.default_rng(1)
    for (m, k, n) in [(1, 1024, 32), (5, 1041, 7), (3, 4096, 3)]:
        a = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        b = rng.integers(-128, 128, size=(k, n), dtype=np.int8)
        exact = a.astype(np.int64) @ b.astype(np.int64)
        assert np.array_equal(oracle.matmul_int8(a, b, out_i32=True)[0], exact)
        assert np.array_equal(oracle.matmul_int8(a, b)[0], exact.astype(np.float32))
    # all -127 (sum = 16129*K), mixed +-127, K tail 1025
    k = 1025
    a = np.full((2, k), -127, np.int8)
    b = np.full((k, 3), -127, np.int8)
    b[:, 1] = 127
    out = oracle.matmul_int8(a, b, out_i32=True)[0]
    assert out[0, 0] == 16129 * k and out[0, 1] == -16129 * k
    # zero operand
    assert not oracle.matmul_int8(np.zeros((3, 8), np.int8), b[:8], out_i32=True).any()


def test_matmul_nt_equals_transposed_reference_loop():
    rng = np.random.default_rng(2)
    a = rng.integers(-127, 127, size=(9, 77), dtype=np.int8)
    w = rng.integers(-127, 127, size=(13, 77), dtype=np.int8)
    nt = oracle.matmul_nt_i32(a, w)
    kn = oracle.matmul_int8(a, np.ascontiguousarray(w.T), out_i32=True)[0]
    assert np.array_equal(nt, kn)


def test_golden_mm_i8_small():
    g = np.load(GOLD / "mm_i8_small.npz")
    assert np.array_equal(oracle.matmul_int8(g["a"], g["b"]), g["c"])


# -------------------------------------------------------------------- GEMV
@needs_ref
def test_linear_f32_restatement_vs_reference():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 96), dtype=np.float32)
    W = rng.standard_normal((40, 96), dtype=np.float32)
    b = rng.standard_normal(40, dtype=np.float32)
    ours = oracle.linear_f32(x, W, b)
    ref = oracle.ref_linear(x, W, b)
    np.testing.assert_allclose(ours, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gemv_golden_c1_and_reference_linear(seed):
    """The W8 GEMV equals the reference fp32 tensor_linear on per-channel
    dequantized weights (what the model runs today) and the float64 closed form."""
    g = np.load(GOLD / f"gemv_c1_seed{seed}.npz")
    y = oracle.gemv_w8(g["x"], g["W"], g["s"])
    np.testing.assert_allclose(y, g["y_f64"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y, g["y_ref_linear"], rtol=2e-4, atol=2e-4)


def test_gemv_special_cases():
    rng = np.random.default_rng(6)
    k, n = 64, 16
    x = rng.standard_normal((2, k), dtype=np.float32)
    # e_j rows pick x[:, j] * s_w[j] exactly
    W = np.zeros((n, k), np.int8)
    W[np.arange(n), np.arange(n) * 3] = 1
    s = rng.uniform(0.001, 0.02, n).astype(np.float32)
    y = oracle.gemv_w8(x, W, s)
    exp = (x[:, np.arange(n) * 3].astype(np.float64) * s.astype(np.float64)).astype(np.float32)
    assert np.array_equal(y, exp)
    # bias adds, scaling s_w by 2^3 scales y exactly, linearity in x
    W = rng.integers(-127, 127, size=(n, k), dtype=np.int8)
    b = rng.standard_normal(n, dtype=np.float32)
    y0 = oracle.gemv_w8(x, W, s)
    yb = oracle.gemv_w8(x, W, s, b)
    np.testing.assert_allclose(yb - y0, np.broadcast_to(b, y0.shape), rtol=1e-5, atol=1e-5)
    assert np.array_equal(oracle.gemv_w8(x, W, s * 8), y0 * 8)
    x2 = rng.standard_normal((2, k), dtype=np.float32)
    np.testing.assert_allclose(oracle.gemv_w8(x + x2, W, s), y0 + oracle.gemv_w8(x2, W, s),
                               rtol=1e-4, atol=1e-4)
    # fp16 activations: identical to fp32 activations holding the same values
    xh = x.astype(np.float16)
    assert np.array_equal(oracle.gemv_w8(xh, W, s), oracle.gemv_w8(xh.astype(np.float32), W, s))
    yh = oracle.gemv_w8(x, W, s, out_dtype=np.float16)
    assert np.array_equal(yh, y0.astype(np.float16))


# --------------------------------------------------------------- quantizer
def test_quant_golden_ties():
    g = np.load(GOLD / "quant_tok.npz")
    q, s = oracle.quant_per_token(g["x"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(s, g["s"])


def _brute_quant_row(x):
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
    s = np.float32(1.0) if amax == 0 else np.float32(amax / np.float32(127.0))
    out = []
    for v in x:
        t = np.float32(v / s)  # IEEE fp32 division
        best = None
        for j in range(-127, 128):
            d = abs(float(t) - j)
            if best is None or d < best[0] - 1e-12 or (abs(d - best[0]) <= 1e-12 and j % 2 == 0):
                best = (d, j)
        out.append(best[1])
    return np.array(out, np.int8), s


def test_quant_brute_force_small():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 23), dtype=np.float32) * rng.uniform(0.01, 100, (6, 1)).astype(np.float32)
    q, s = oracle.quant_per_token(x)
    for i in range(x.shape[0]):
        qb, sb = _brute_quant_row(x[i])
        assert s[i] == sb
        assert np.array_equal(q[i], qb)


def test_quant_invariants():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((64, 1000), dtype=np.float32) * 3
    x[5] = 0
    q, s = oracle.quant_per_token(x)
    assert np.abs(q.astype(np.int32)).max() <= 127
    nz = np.abs(x).max(1) > 0
    assert np.all(np.abs(q[nz].astype(np.int32)).max(1) == 127)
    assert not q[5].any() and s[5] == 1.0
    err = np.abs(x - q.astype(np.float32) * s[:, None])
    assert np.all(err <= s[:, None] * (0.5 + 1e-5))
    assert np.all(np.sign(q[np.abs(x) > s[:, None]]) == np.sign(x[np.abs(x) > s[:, None]]))
    # fp16 input == fp32 input of the same values
    xh = x.astype(np.float16)
    q1, s1 = oracle.quant_per_token(xh)
    q2, s2 = oracle.quant_per_token(xh.astype(np.float32))
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


# -------------------------------------------------------------------- W8A8
@needs_ref
@pytest.mark.parametrize("K", [8, 1000, 1024, 4096])
def test_rmsnorm_quant_integer_rows_bitwise_vs_reference(K):
    """Rows of small integers have sums of squares that are exact in fp32 in
    any order, so the oracle's normalized y must equal the compiled reference
    tensor_rms_norm bit for bit (any slip in eps, the mean, the sqrt/division
    or the scale-then-weight order shows), and q, s must be the per-token
    quantizer of the reference's own output."""
    rng = np.random.default_rng(K)
    M = 6
    x = rng.integers(-16, 17, (M, K)).astype(np.float32)
    x[1] = 0.0                                    # zero row
    x[2, :] = 3.0                                 # constant row
    w = rng.uniform(0.5, 2.0, K).astype(np.float32)
    for eps in (1e-6, 1e-5, 0.25):
        q, s, y, _ = oracle.rmsnorm_quant(x, w, eps)
        y_ref = oracle.ref_rms_norm(x, w, eps)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), eps
        q_ref, s_ref = oracle.quant_per_token(y_ref)
        assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    assert np.all(q[1] == 0) and s[1] == 1.0


def test_rmsnorm_quant_random_rows_vs_float64():
    """Random fp32/fp16 rows: y within 4 ulp of the float64 RMSNorm, and every
    q within half a step (plus y's rounding) of y64 / s."""
    rng = np.random.default_rng(7)
    for dt in (np.float32, np.float16):
        for K in (64, 1024, 3072):
            x = (rng.standard_normal((5, K)) * rng.uniform(0.1, 30.0, (5, 1))).astype(dt)
            w = rng.uniform(0.2, 3.0, K).astype(np.float32)
            q, s, y, _ = oracle.rmsnorm_quant(x, w, 1e-6)
            x64 = x.astype(np.float64)
            y64 = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * w
            ulp = np.spacing(np.abs(y64).astype(np.float32)).astype(np.float64)
            assert np.all(np.abs(y - y64) <= 4 * ulp + 1e-30)
            s64 = np.abs(y64).max(axis=1) / 127.0
            assert np.allclose(s, s64, rtol=1e-6)
            assert np.all(np.abs(q - y64 / s[:, None]) <= 0.5 + 1e-4)
            assert np.abs(q).max() == 127


def test_rmsnorm_quant_fused_add():
    """With a residual the sum is stored in x's dtype (round to nearest even
    for fp16) and the result is that of the plain form on the stored sum."""
    rng = np.random.default_rng(8)
    for dt in (np.float32, np.float16):
        x = rng.standard_normal((4, 512)).astype(dt)
        r = rng.standard_normal((4, 512)).astype(dt)
        w = rng.uniform(0.5, 1.5, 512).astype(np.float32)
        q, s, y, xs = oracle.rmsnorm_quant(x, w, 1e-6, residual=r)
        assert np.array_equal(xs, (x.astype(np.float32) + r.astype(np.float32)).astype(dt))
        q2, s2, y2, _ = oracle.rmsnorm_quant(xs, w, 1e-6)
        assert np.array_equal(q, q2) and np.array_equal(s, s2) and np.array_equal(y, y2)


def test_w8a8_int_core_and_epilogue():
    rng = np.random.default_rng(10)
    m, n, k = 9, 21, 160
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    W = rng.integers(-127, 127, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, m).astype(np.float32)
    sw = rng.uniform(0.001, 0.02, n).astype(np.float32)
    acc = oracle.w8a8(q, sa, W, sw, out="i32")
    assert np.array_equal(acc, q.astype(np.int64) @ W.astype(np.int64).T)
    y32 = oracle.w8a8(q, sa, W, sw, out="f32")
    exact = acc.astype(np.float64) * sa[:, None].astype(np.float64) * sw[None].astype(np.float64)
    np.testing.assert_allclose(y32, exact, rtol=1e-6)
    y16 = oracle.w8a8(q, sa, W, sw, out="f16")
    assert np.array_equal(y16, y32.astype(np.float16))
    b = rng.standard_normal(n, dtype=np.float32)
    np.testing.assert_allclose(oracle.w8a8(q, sa, W, sw, b, out="f32"), y32 + b, rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------- MoE
@needs_ref
def test_softmax_topk_bitwise_vs_reference():
    g = np.load(GOLD / "route_tiny.npz")
    p = oracle.softmax(g["logits"])
    assert np.array_equal(p, g["probs"])
    v, i = oracle.topk(p, 2)
    assert np.array_equal(v, g["topv"]) and np.array_equal(i, g["topi"])
    # and live against the reference library on a larger case
    rng = np.random.default_rng(11)
    lg = rng.standard_normal((64, 128), dtype=np.float32)
    p = oracle.softmax(lg)
    assert np.array_equal(p, oracle.ref_softmax(lg))
    v, i = oracle.topk(p, 8)
    rv, ri = oracle.ref_topk(p, 8)
    assert np.array_equal(v, rv) and np.array_equal(i, ri)


def test_topk_ties_keep_lower_index_bruteforce():
    g = np.load(GOLD / "route_tiny.npz")
    p = g["probs"]
    for k in (1, 2, 5, 8):
        _, i = oracle.topk(p, k)
        exp = np.argsort(-p, axis=1, kind="stable")[:, :k]
        assert np.array_equal(i, exp)
    _, i = oracle.topk(p, 3)
    assert list(i[1]) == [0, 1, 2]  # all-equal row


def test_route_renorm():
    rng = np.random.default_rng(12)
    lg = rng.standard_normal((32, 16), dtype=np.float32)
    w, i = oracle.moe_route(lg, 4, renorm=False)
    p = oracle.softmax(lg)
    assert np.array_equal(w, np.take_along_axis(p, i, 1))
    wr, ir = oracle.moe_route(lg, 4, renorm=True)
    assert np.array_equal(i, ir)
    np.testing.assert_allclose(wr.sum(1), 1.0, rtol=1e-6)


def test_group_matches_reference_moe_dispatch_known_answer():
    """tests/test_moe_dispatch.py:10-86 of the reference: tokens [0,1,0,1] ->
    expert 0 gets tokens 0 and 2, expert 1 tokens 1 and 3; adding 10 and
    scatter-adding back gives [11,11,0,0,13,13,0,0] for expert 0."""
    ids = np.array([[0], [1], [0], [1]], np.int32)
    off, rows, pos = oracle.moe_group(ids, 2)
    assert list(off) == [0, 2, 4]
    assert list(rows[off[0]:off[1]]) == [0, 2]
    assert list(rows[off[1]:off[2]]) == [1, 3]
    data = np.array([[1, 1], [2, 2], [3, 3], [4, 4]], np.float32)
    out = np.zeros_like(data)
    for r in range(off[0], off[1]):
        out[rows[r]] += data[rows[r]] + 10
    assert out.ravel().tolist() == [11, 11, 0, 0, 13, 13, 0, 0]
    for t in range(4):
        assert rows[pos[t]] == t


def test_group_bruteforce():
    rng = np.random.default_rng(13)
    T, E, k = 50, 12, 3
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    off, rows, pos = oracle.moe_group(ids, E)
    for e in range(E):
        toks = sorted(t for t in range(T) if e in ids[t])
        assert list(rows[off[e]:off[e + 1]]) == toks
    for t in range(T):
        for kk in range(k):
            p = pos[t * k + kk]
            assert rows[p] == t and off[ids[t, kk]] <= p < off[ids[t, kk] + 1]


def test_exp_det_against_float64_exp():
    """The MoE SwiGLU's deterministic e^x: within 1 ulp of float64 exp over the
    whole finite range (dense sweep plus random points), and its special
    cases: exact 1 at 0, +inf past the overflow bound and for +inf, +0 below
    -103.98 and for -inf, NaN in, NaN out."""
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-103.9, 88.72, 2_000_001, dtype=np.float32),
                        (rng.standard_normal(1_000_000) * 20).astype(np.float32),
                        np.float32([-1e-8, 1e-8, -0.5, 0.5, 1.0, -1.0, 0.34657359, -0.34657359])])
    x = x[(x > -103.9) & (x < 88.72)]
    y = oracle.exp_det(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    normal = ref > np.finfo(np.float32).tiny
    ulp = np.abs(y[normal] - ref[normal]) / np.spacing(ref[normal].astype(np.float32))
    assert ulp.max() <= 1.0, ulp.max()
    sub = ~normal   # subnormal results: within one subnormal step
    assert np.all(np.abs(y[sub] - ref[sub]) <= np.float64(2.0 ** -149))
    sp = oracle.exp_det(np.float32([0.0, -0.0, 88.73, 1e30, np.inf, -104.0, -1e30, -np.inf, np.nan]))
    assert sp[0] == 1.0 and sp[1] == 1.0
    assert np.all(np.isposinf(sp[2:5]))
    assert np.all(sp[5:8] == 0.0) and not np.any(np.signbit(sp[5:8]))
    assert np.isnan(sp[8])


def _numpy_moe(x, logits, wgu, sgu, wd, sd, k, renorm=False):
    """Independent numpy composition of the MoE definition (float64 epilogues
    rounded to fp32 at the same points as the definition)."""
    T, H = x.shape
    E, I2, _ = wgu.shape
    I = I2 // 2
    w, ids = oracle.moe_route(logits, k, renorm)
    qx, sx = oracle.quant_per_token(x)
    out = np.zeros((T, H), np.float32)
    for t in range(T):
        acc_o = np.zeros(H, np.float32)
        for kk in range(k):
            e = ids[t, kk]
            acc = qx[t].astype(np.int64) @ wgu[e].astype(np.int64).T
            gu = (acc.astype(np.float32) * sx[t]) * sgu[e]
            g, u = gu[:I], gu[I:]
            h = (g * (np.float32(1) / (np.float32(1) + np.exp(-g)))) * u
            qh, sh = oracle.quant_per_token(h[None].astype(np.float32))
            acc2 = qh[0].astype(np.int64) @ wd[e].astype(np.int64).T
            d = (acc2.astype(np.float32) * sh[0]) * sd[e]
            acc_o = acc_o + w[t, kk] * d
        out[t] = acc_o
    return out


def test_moe_oracle_vs_numpy_composition_and_golden():
    g = np.load(GOLD / "moe_tiny.npz")
    y = oracle.moe_w8a8(g["x"], g["logits"], g["w_gu"], g["s_gu"], g["w_down"], g["s_down"], 2)
    assert np.array_equal(y, g["y"])
    yn = _numpy_moe(g["x"], g["logits"], g["w_gu"], g["s_gu"], g["w_down"], g["s_down"], 2)
    np.testing.assert_allclose(y, yn, rtol=2e-3, atol=2e-3 * np.abs(yn).max())


def test_moe_identical_experts_invariant():
    """With every expert identical and renormalized weights the layer equals
    one expert MLP, whatever the routing."""
    rng = np.random.default_rng(14)
    T, H, I, E, k = 8, 32, 16, 6, 3
    x = rng.standard_normal((T, H), dtype=np.float32)
    lg = rng.standard_normal((T, E), dtype=np.float32)
    wgu1 = rng.integers(-127, 127, size=(1, 2 * I, H), dtype=np.int8)
    sgu1 = rng.uniform(0.001, 0.02, (1, 2 * I)).astype(np.float32)
    wd1 = rng.integers(-127, 127, size=(1, H, I), dtype=np.int8)
    sd1 = rng.uniform(0.001, 0.02, (1, H)).astype(np.float32)
    rep = lambda a: np.repeat(a, E, axis=0)  # noqa: E731
    y = oracle.moe_w8a8(x, lg, rep(wgu1), rep(sgu1), rep(wd1), rep(sd1), k, renorm=True)
    single = oracle.moe_w8a8(x, np.zeros((T, 1), np.float32), wgu1, sgu1, wd1, sd1, 1, renorm=True)
    np.testing.assert_allclose(y, single, rtol=1e-5, atol=1e-5 * np.abs(single).max())


# ------------------------------------------------------------ decoder oracle
def _qwen2_logits_and_oracle(monkey_rope=None):
    """Teacher-forced logits of transformers' Qwen2ForCausalLM (float64) and of
    oracle/qwen3_ref.py stepping through the same 20 ids, same weights."""
    torch = pytest.importorskip("torch")
    tf = pytest.importorskip("transformers")
    import oracle.qwen3_ref as q3
    from mod_amd.qwen3 import random_weights

    cfg = q3.Qwen3Config(n_layers=2, hidden=128, n_heads=4, n_kv_heads=2, head_dim=64,
                         intermediate=256, vocab=300, max_seq=32)
    w = random_weights(cfg, seed=3)
    w["final_norm"] = (1.0 + 0.1 * np.random.default_rng(4).standard_normal(cfg.hidden)).astype(np.float32)
    hf_cfg = tf.Qwen2Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden,
                            intermediate_size=cfg.intermediate, num_hidden_layers=cfg.n_layers,
                            num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
                            head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_eps,
                            rope_theta=cfg.rope_theta, max_position_embeddings=cfg.max_seq,
                            tie_word_embeddings=False, attn_implementation="eager")
    model = tf.Qwen2ForCausalLM(hf_cfg).to(torch.float64).eval()
    deq = lambda W, s: torch.from_numpy(W.astype(np.float64) * s.astype(np.float64)[:, None])  # noqa: E731
    t64 = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    nq, D, I = cfg.n_heads * cfg.head_dim, cfg.head_dim, cfg.intermediate
    nk = cfg.n_kv_heads * D
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(t64(w["embed"]))
        model.model.norm.weight.copy_(t64(w["final_norm"]))
        model.lm_head.weight.copy_(deq(w["lm_head"], w["s_lm_head"]))
        for L, blk in zip(w["layers"], model.model.layers):
            Wqkv = deq(L["w_qkv"], L["s_qkv"])
            a = blk.self_attn
            a.q_proj.weight.copy_(Wqkv[:nq]); a.q_proj.bias.copy_(t64(L["b_qkv"][:nq]))
            a.k_proj.weight.copy_(Wqkv[nq:nq + nk]); a.k_proj.bias.copy_(t64(L["b_qkv"][nq:nq + nk]))
            a.v_proj.weight.copy_(Wqkv[nq + nk:]); a.v_proj.bias.copy_(t64(L["b_qkv"][nq + nk:]))
            a.o_proj.weight.copy_(deq(L["w_o"], L["s_o"]))
            Wgu = deq(L["w_gu"], L["s_gu"])
            blk.mlp.gate_proj.weight.copy_(Wgu[:I])
            blk.mlp.up_proj.weight.copy_(Wgu[I:])
            blk.mlp.down_proj.weight.copy_(deq(L["w_down"], L["s_down"]))
            blk.input_layernorm.weight.copy_(t64(L["in_norm"]))
            blk.post_attention_layernorm.weight.copy_(t64(L["post_norm"]))
        ids = np.random.default_rng(5).integers(0, cfg.vocab, 20)
        hf = model(torch.from_numpy(ids)[None]).logits[0].numpy()
    ref = q3.Qwen3Ref(cfg, w, np.float64)
    ours = np.stack([ref.step(int(t)) for t in ids])
    return ours, hf


def test_decoder_oracle_vs_transformers_qwen2():
    """oracle/qwen3_ref.py against an independent implementation: transformers'
    Qwen2 block has the reference architecture's structure (q/k/v projections
    with bias, no q/k norm, rotate-half RoPE, GQA, pre-norm, SwiGLU;
    ip/models/qwen3_0_6b/architecture.py:21-221). Loaded with the same
    dequantized int8 weights and run in float64, its teacher-forced logits
    must equal the oracle's step-by-step logits. transformers rounds its
    RMSNorm and RoPE tables through float32 (observed gap 1.1e-5 of the logit
    rms; with a float64 RMSNorm it falls below 1e-5), hence the 5e-5 bar."""
    ours, hf = _qwen2_logits_and_oracle()
    err = np.abs(ours - hf).max() / np.sqrt(np.mean(hf * hf))
    assert err < 5e-5, err


def test_decoder_oracle_pin_resolves_a_rope_slip(monkeypatch):
    """The comparison above resolves plausible mistakes: the oracle with RoPE
    pairs taken interleaved (2i, 2i+1) instead of rotate-half (i, i+D/2)
    misses transformers by orders of magnitude more than the bar."""
    import oracle.qwen3_ref as q3

    def rope_interleaved(v, c, s):
        r, im = v[..., 0::2], v[..., 1::2]
        out = np.empty_like(v)
        out[..., 0::2] = r * c - im * s
        out[..., 1::2] = r * s + im * c
        return out

    monkeypatch.setattr(q3, "_rope", rope_interleaved)
    ours, hf = _qwen2_logits_and_oracle()
    err = np.abs(ours - hf).max() / np.sqrt(np.mean(hf * hf))
    assert err > 1e-2, err


@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_decoder_oracle_batched_forward_equals_steps(kv_dtype):
    """qwen3_ref.forward_all (every position at once, causal mask) computes
    what Qwen3Ref.step computes position by position: float64 logits agree to
    1e-12 of their rms at every position, GQA (4 query heads on 2 KV heads)
    and the qkv bias included."""
    import oracle.qwen3_ref as q3
    from mod_amd.qwen3 import random_weights, Qwen3Config
    kw = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512,
              vocab=500, max_seq=64, kv_dtype=kv_dtype)
    w = random_weights(Qwen3Config(**kw), seed=9)
    cfg = q3.Qwen3Config(**kw)
    ids = np.random.default_rng(10).integers(0, cfg.vocab, 40)
    ref = q3.Qwen3Ref(cfg, w, np.float64)
    steps = np.stack([ref.step(int(t)) for t in ids])
    want = [0, 1, 17, 39]
    got = q3.forward_all(cfg, w, ids, want)
    err = np.abs(got - steps[want]).max() / np.sqrt(np.mean(steps * steps))
    assert err < 1e-12, err
