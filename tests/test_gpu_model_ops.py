"""GPU parity of the model-layer companion ops (mod_amd/csrc/model_ops.hip)
through the C-ABI and the Python mirror of the reference Tensor API, against
oracle/model_ops_ref.py (pinned in tests/test_oracle_model_ops.py).

Bars: index and data-movement ops (argmax, embed, slice, set_slice, cat,
reshape, the in-place residual sum) bit-exact; fp32 arithmetic within
RTOL = 2e-5 of the float64 oracle (conftest.assert_rel: relative, with a floor
of 1e-2 x the output rms; attention on the scale of max |v|, its outputs being
convex combinations of v rows), which covers fp32 summation order and the
device expf / sqrtf against float64."""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from oracle import model_ops_ref as mo
from tests.conftest import assert_rel

pytestmark = pytest.mark.gpu
RTOL = 2e-5


def _say(m):
    print(m, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def B(torch_dev):
    from mod_amd import backend
    return backend


def _t(B, a):
    return B.Tensor.from_numpy(np.ascontiguousarray(a, np.float32))


@pytest.mark.parametrize("rows,cols", [(1, 1024), (7, 3072), (3, 1000), (2, 70001)])
def test_rms_norm_and_fused_add(B, rows, cols):
    _say(f"rms_norm {rows}x{cols}")
    rng = np.random.default_rng(rows * 31 + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    r = rng.standard_normal((rows, cols)).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    tx, tr, tw = _t(B, x), _t(B, r), _t(B, w)
    assert_rel(tx.rms_norm(tw, 1e-6).numpy(), mo.rms_norm(x, w, 1e-6), RTOL, "rms_norm")
    y = tx.fused_add_rms_norm(tr, tw, 1e-5)
    s, ref = mo.fused_add_rms_norm(x, r, w, 1e-5)
    assert np.array_equal(tx.numpy(), x + r)          # fp32 sum stored in place, bit-exact
    assert_rel(y.numpy(), ref, RTOL, "fused_add_rms_norm")


@pytest.mark.parametrize("Bn,S,Hq,Hk,D", [(2, 5, 16, 8, 128), (1, 1, 16, 16, 128), (3, 4, 4, 1, 64)])
def test_rope(B, Bn, S, Hq, Hk, D):
    _say(f"rope B{Bn} S{S} Hq{Hq} Hk{Hk} D{D}")
    rng = np.random.default_rng(S * 100 + Hk)
    q = rng.standard_normal((Bn, S, Hq, D)).astype(np.float32)
    k = rng.standard_normal((Bn, S, Hk, D)).astype(np.float32)
    ang = rng.uniform(-40, 40, (S + 3, D // 2)).astype(np.float32)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    oq, ok = _t(B, q).rope(_t(B, k), _t(B, c), _t(B, s))
    rq, rk = mo.rope(q, k, c, s)
    assert_rel(oq.numpy(), rq, RTOL, "rope q")
    assert_rel(ok.numpy(), rk, RTOL, "rope k")


@pytest.mark.parametrize("n", [3 * 3072, 1000003])
def test_silu_swiglu_family(B, n):
    _say(f"silu family n={n}")
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 5).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    assert_rel(_t(B, g).silu().numpy(), mo.silu(g), RTOL, "silu")
    assert_rel(_t(B, g).swiglu(_t(B, u)).numpy(), mo.swiglu(g, u), RTOL, "swiglu")
    rows = 7
    gu = (rng.standard_normal((rows, 2 * 1536)) * 4).astype(np.float32)
    assert_rel(_t(B, gu).fused_swiglu().numpy(), mo.fused_gate_up_swiglu(gu), RTOL, "fused swiglu")


@pytest.mark.parametrize("rows,cols", [(3, 7), (5, 151936)])
def test_softmax_and_argmax(B, rows, cols):
    _say(f"softmax / argmax {rows}x{cols}")
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((rows, cols)) * 8).astype(np.float32)
    assert_rel(_t(B, x).softmax().numpy(), mo.softmax(x), RTOL, "softmax")
    x[0, cols // 2] = x[0, cols - 1] = 1e4             # tie: the first index
    if rows > 1:
        x[1, :] = -3e9                                 # nothing above -1e9: 0
    if rows > 2:
        x[2, 1] = np.nan                               # NaN never wins
    got = _t(B, x).argmax().numpy()
    assert np.array_equal(got, mo.argmax(x)), (got, mo.argmax(x))


def test_embed_exact(B):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((5000, 1024)).astype(np.float32)
    idx = np.array([[0, 17.9, 4999, 5000], [-3, 2.5, 1e12, 123]], np.float32)
    got = _t(B, w).embed(_t(B, idx))
    assert got.shape == (2, 4, 1024)
    assert np.array_equal(got.numpy(), mo.embed(w, idx))


@pytest.mark.parametrize("Bn,S,H,Hk,T,D", [(1, 1, 16, 8, 300, 128), (2, 7, 4, 4, 7, 64), (1, 2, 8, 2, 5000, 128),
                                           (1, 3, 2, 1, 1, 32)])
def test_scaled_dot_product_attention(B, Bn, S, H, Hk, T, D):
    _say(f"sdpa B{Bn} S{S} H{H} Hk{Hk} T{T} D{D}")
    rng = np.random.default_rng(T + H)
    q = rng.standard_normal((Bn, S, H, D)).astype(np.float32)
    k = rng.standard_normal((Bn, T, Hk, D)).astype(np.float32)
    v = rng.standard_normal((Bn, T, Hk, D)).astype(np.float32)
    got = B.scaled_dot_product_attention(_t(B, q), _t(B, k), _t(B, v)).numpy()
    # each output is a convex combination of v rows: its error is bounded on
    # the scale of max |v| (an output near zero has no relative accuracy of its own)
    err = float(np.abs(got - mo.sdpa(q, k, v, 1 / np.sqrt(D))).max() / np.abs(v).max())
    _say(f"  max err {err:.2e} x max|v|")
    assert err <= RTOL, err


def test_slice_set_slice_cat_reshape_exact(B):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 9, 4, 8)).astype(np.float32)
    tx = _t(B, x)
    for start, shape in [([0, 2, 1, 0], [3, 4, 2, 8]), ([1, 7, 3, 5], [2, 4, 2, 8])]:
        assert np.array_equal(tx.slice(start, shape).numpy(), mo.slice_from(x, shape, start, fill=0.0)), start
        src = rng.standard_normal(shape).astype(np.float32)
        td = _t(B, x)
        td.set_slice(_t(B, src), start)
        assert np.array_equal(td.numpy(), mo.set_slice(x, src, start)), start
    for axis in (1, 3):
        ps = [rng.standard_normal((2, n, 3, 5) if axis == 1 else (2, 3, 3, n)).astype(np.float32)
              for n in (1, 4, 2)]
        got = B.cat([_t(B, p) for p in ps], axis)
        assert np.array_equal(got.numpy(), mo.cat(ps, axis)), axis
    assert np.array_equal(tx.reshape([27, 32]).numpy(), x.reshape(27, 32))


def test_ops_reject_host_tensors_and_bad_shapes(B):
    from mod_amd.ops import RocmError
    x = _t(B, np.ones((2, 8), np.float32))
    with pytest.raises(RocmError, match="weight has"):
        x.rms_norm(_t(B, np.ones(4, np.float32)))
    h = B.Tensor([8], device="cpu")
    with pytest.raises(RocmError, match="host"):
        x.rms_norm(h)
    q = _t(B, np.ones((1, 1, 3, 8), np.float32))
    k = _t(B, np.ones((1, 4, 2, 8), np.float32))
    with pytest.raises(RocmError, match="Hk dividing"):
        B.scaled_dot_product_attention(q, k, k)


def test_in_place_forms_and_fused_overlap_refused(B):
    """silu, swiglu, softmax and RoPE with the output being an input (each
    element is read and written by one thread) equal their out-of-place
    results bit for bit; the fused gate_up SwiGLU refuses an output that
    overlaps gate_up, whose rows other threads still read."""
    from mod_amd import ops
    from mod_amd.ops import lib
    _say("in-place forms")
    rng = np.random.default_rng(11)
    g = (rng.standard_normal(5000) * 4).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    want = _t(B, g).silu().numpy()
    t = _t(B, g)
    assert lib.tensor_silu_status(t._handle, t._handle) == ops.OK
    assert np.array_equal(t.numpy(), want)
    want = _t(B, g).swiglu(_t(B, u)).numpy()
    t, tu = _t(B, g), _t(B, u)
    assert lib.tensor_swiglu_status(t._handle, tu._handle, t._handle) == ops.OK
    assert np.array_equal(t.numpy(), want)
    x = (rng.standard_normal((6, 777)) * 3).astype(np.float32)
    want = _t(B, x).softmax().numpy()
    t = _t(B, x)
    assert lib.tensor_softmax_status(t._handle, t._handle) == ops.OK
    assert np.array_equal(t.numpy(), want)
    q = rng.standard_normal((2, 3, 4, 64)).astype(np.float32)
    k = rng.standard_normal((2, 3, 2, 64)).astype(np.float32)
    ang = rng.uniform(-9, 9, (3, 32)).astype(np.float32)
    c, sn = _t(B, np.cos(ang)), _t(B, np.sin(ang))
    wq, wk = _t(B, q).rope(_t(B, k), c, sn)
    tq, tk = _t(B, q), _t(B, k)
    assert lib.tensor_rope_status(tq._handle, tk._handle, c._handle, sn._handle, tq._handle,
                                  tk._handle) == ops.OK
    assert np.array_equal(tq.numpy(), wq.numpy()) and np.array_equal(tk.numpy(), wk.numpy())
    gu = _t(B, rng.standard_normal((4, 256)).astype(np.float32))
    half = B.Tensor([4, 128])
    # a [4, 128] tensor over gate_up's first 512 floats (the struct is the
    # reference's plain Tensor, so a caller can build such a view)
    g0 = gu._handle.contents
    shp = (ctypes.c_int * 2)(4, 128)
    view = ops.CTensor(g0.data, ctypes.cast(shp, ctypes.POINTER(ctypes.c_int)), 2, 512, g0.device_id)
    assert lib.tensor_fused_gate_up_swiglu_status(gu._handle, ctypes.byref(view)) == ops.ERR_INVALID
    assert "overlaps" in ops.last_error()
    assert lib.tensor_fused_gate_up_swiglu_status(gu._handle, half._handle) == ops.OK


def test_reference_style_decoder_layer_with_kv_cache(B):
    """A Qwen3-style decoder layer written against the Tensor API as the
    reference writes it (qwen3_0_6b/architecture.py:68-135: fused qkv
    projection with bias, slice/reshape, RoPE, KV-cache set_slice / slice,
    attention, o_proj, fused add + RMSNorm, gate_up + fused SwiGLU, down),
    on rocm:0 with W8Linear projections, stepped one position at a time over
    6 positions; every step's output against the same composition of the
    oracle ops (linears: oracle.gemv_w8). GQA needs no repeat_kv copy here."""
    rng = np.random.default_rng(11)
    Hd, nh, nkv, D, I, P = 256, 4, 2, 64, 512, 6
    qs, kvs = nh * D, nkv * D

    def q8(n, k):
        w = rng.standard_normal((n, k)).astype(np.float32)
        s = (np.abs(w).max(1) / 127).astype(np.float32)
        return np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8), s

    wqkv, sqkv = q8(qs + 2 * kvs, Hd)
    bqkv = (rng.standard_normal(qs + 2 * kvs) * 0.1).astype(np.float32)
    wo, so = q8(Hd, qs)
    wgu, sgu = q8(2 * I, Hd)
    wd, sd = q8(Hd, I)
    g1 = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32)
    g2 = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32)
    ang = np.arange(P)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    def lin(n, k, w, s, b=None):
        m = B.W8Linear(k, n, bias=b is not None)
        m.load_quantized(w, s, b)
        return m

    qkv_p, o_p = lin(qs + 2 * kvs, Hd, wqkv, sqkv, bqkv), lin(Hd, qs, wo, so)
    gu_p, dn_p = lin(2 * I, Hd, wgu, sgu), lin(Hd, I, wd, sd)
    n1, n2 = B.RMSNorm(Hd), B.RMSNorm(Hd)
    n1.weight.load(g1)
    n2.weight.load(g2)
    tcos, tsin = _t(B, cos), _t(B, sin)
    k_cache = _t(B, np.zeros((1, P, nkv, D), np.float32))
    v_cache = _t(B, np.zeros((1, P, nkv, D), np.float32))
    ref_k = np.zeros((1, P, nkv, D))
    ref_v = np.zeros((1, P, nkv, D))
    xs = rng.standard_normal((P, Hd)).astype(np.float32)
    for pos in range(P):
        x = xs[pos][None, None, :]
        # ---- the layer on rocm:0 through the Tensor API
        hs = _t(B, x)
        h = n1(hs)
        qkv = qkv_p(h)
        q = qkv.slice([0, 0, 0], [1, 1, qs]).reshape([1, 1, nh, D])
        k = qkv.slice([0, 0, qs], [1, 1, kvs]).reshape([1, 1, nkv, D])
        v = qkv.slice([0, 0, qs + kvs], [1, 1, kvs]).reshape([1, 1, nkv, D])
        c = tcos.slice([pos, 0], [1, D // 2])
        s = tsin.slice([pos, 0], [1, D // 2])
        q, k = q.rope(k, c, s)
        k_cache.set_slice(k, [0, pos, 0, 0])
        v_cache.set_slice(v, [0, pos, 0, 0])
        kk = k_cache.slice([0, 0, 0, 0], [1, pos + 1, nkv, D])
        vv = v_cache.slice([0, 0, 0, 0], [1, pos + 1, nkv, D])
        att = B.scaled_dot_product_attention(q, kk, vv).reshape([1, 1, qs])
        a = o_p(att)
        hn = hs.fused_add_rms_norm(a, n2.weight, 1e-6)       # hs <- hs + a
        out = hs.add(dn_p(gu_p(hn).fused_swiglu())).numpy()[0, 0]
        # ---- the same layer composed from the oracle ops
        xr = x[0, 0].astype(np.float64)
        hr = mo.rms_norm(xr[None], g1, 1e-6)
        qkv_r = oracle.gemv_w8(hr.astype(np.float32), wqkv, sqkv, bqkv).astype(np.float64)[0]
        qr = qkv_r[:qs].reshape(1, 1, nh, D)
        kr = qkv_r[qs:qs + kvs].reshape(1, 1, nkv, D)
        vr = qkv_r[qs + kvs:].reshape(1, 1, nkv, D)
        qr, kr = mo.rope(qr, kr, cos[pos:pos + 1], sin[pos:pos + 1])
        ref_k[0, pos], ref_v[0, pos] = kr[0, 0], vr[0, 0]
        ar = mo.sdpa(qr, ref_k[:, :pos + 1], ref_v[:, :pos + 1], 1 / np.sqrt(D)).reshape(1, qs)
        a_r = oracle.gemv_w8(ar.astype(np.float32), wo, so).astype(np.float64)[0]
        s_r, hn_r = mo.fused_add_rms_norm(xr, a_r, g2, 1e-6)
        gu_r = oracle.gemv_w8(hn_r[None].astype(np.float32), wgu, sgu).astype(np.float64)
        d_r = oracle.gemv_w8(mo.fused_gate_up_swiglu(gu_r).astype(np.float32), wd, sd).astype(np.float64)[0]
        ref_out = s_r + d_r
        err = float(np.abs(out - ref_out).max() / np.sqrt(np.mean(ref_out ** 2)))
        _say(f"decoder layer position {pos}: max err {err:.2e} x rms")
        assert err <= 1e-4, (pos, err)
