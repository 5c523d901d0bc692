"""Pins oracle/model_ops_ref.py (the checker of the model-layer companion ops)
against the reference's own compiled functions (oracle/_ref, built from
plugins/cpu/c_src/tensor_ops.c), and against closed forms where the
restatement goes beyond what the reference loop defines."""
import ctypes

import numpy as np
import pytest

import oracle
from oracle import model_ops_ref as mo

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
RNG = np.random.default_rng(7)


def _close(a, b, tol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(1.0, float(np.abs(b).max()))
    assert np.abs(a - b).max() <= tol * scale, float(np.abs(a - b).max())


@needs_ref
def test_rms_norm_and_activations_match_reference():
    x = RNG.standard_normal((5, 1000)).astype(np.float32) * 3
    w = RNG.standard_normal(1000).astype(np.float32)
    _close(mo.rms_norm(x, w, 1e-6), oracle.ref_rms_norm(x, w, 1e-6), 2e-6)
    g = RNG.standard_normal((3, 700)).astype(np.float32) * 4
    u = RNG.standard_normal((3, 700)).astype(np.float32)
    _close(mo.silu(g), mo.ref("tensor_silu", g, g.shape), 2e-6)
    _close(mo.swiglu(g, u), mo.ref("tensor_swiglu", g, u, g.shape), 2e-6)
    gu = np.concatenate([g, u], axis=1)
    _close(mo.fused_gate_up_swiglu(gu), mo.ref("tensor_fused_gate_up_swiglu", gu, (3, 700)), 2e-6)
    s = RNG.standard_normal((4, 333)).astype(np.float32) * 10
    _close(mo.softmax(s), oracle.ref_softmax(s), 2e-6)
    assert np.allclose(mo.softmax(s).sum(-1), 1.0, atol=1e-12)


@needs_ref
def test_fused_add_rms_norm_is_add_then_norm():
    x = RNG.standard_normal((3, 512)).astype(np.float32)
    r = RNG.standard_normal((3, 512)).astype(np.float32)
    w = RNG.standard_normal(512).astype(np.float32)
    s, y = mo.fused_add_rms_norm(x, r, w, 1e-5)
    assert np.array_equal(s, x.astype(np.float64) + r)
    _close(y, oracle.ref_rms_norm((x + r).astype(np.float32), w, 1e-5), 2e-6)


@needs_ref
def test_rope_matches_reference_and_keeps_pair_norms():
    B, S, H, D = 2, 5, 3, 16
    q = RNG.standard_normal((B, S, H, D)).astype(np.float32)
    k = RNG.standard_normal((B, S, H, D)).astype(np.float32)
    ang = RNG.uniform(-3, 3, (S, D // 2)).astype(np.float32)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    oq, ok = mo.rope(q, k, c, s)
    rq, rk = mo.ref("tensor_rope", q, k, c, s, q.shape, k.shape)
    _close(oq, rq, 2e-6)
    _close(ok, rk, 2e-6)
    # grouped-query k (beyond the reference loop): a rotation keeps each pair's norm
    kg = RNG.standard_normal((B, S, 1, D)).astype(np.float32)
    _, okg = mo.rope(q, kg, c, s)
    h = D // 2
    n_in = kg[..., :h].astype(np.float64) ** 2 + kg[..., h:].astype(np.float64) ** 2
    n_out = okg[..., :h] ** 2 + okg[..., h:] ** 2
    _close(n_out, n_in, 1e-6)
    # and its single head rotates like a q head with the same values
    qs = np.repeat(kg, H, axis=2)
    oqs, _ = mo.rope(qs, qs, c, s)
    _close(okg[:, :, 0], oqs[:, :, 1], 1e-12)


@needs_ref
def test_argmax_and_embed_match_reference_exactly():
    x = RNG.standard_normal((6, 300)).astype(np.float32)
    x[1, 10] = x[1, 200] = 50.0        # tie: the first index wins
    x[2, :] = -2e9                     # nothing above -1e9: 0
    x[3, 5] = np.nan                   # NaN never wins
    x[4, :] = -1e9
    x[4, 7] = -9.9e8
    got = mo.argmax(x)
    ref = mo.ref("tensor_argmax", x, (6,))
    assert np.array_equal(got, ref), (got, ref)
    assert got[1] == 10 and got[2] == 0 and got[4] == 7
    w = RNG.standard_normal((50, 24)).astype(np.float32)
    idx = np.array([0, 3.7, 49, 50, -1, 12.2, 1e10, -0.5], np.float32)
    assert np.array_equal(mo.embed(w, idx), mo.ref("tensor_embed", w, idx, (idx.size, 24)))


@needs_ref
def test_sdpa_matches_reference_and_extends_it():
    B, S, H, D = 2, 6, 4, 32
    q = RNG.standard_normal((B, S, H, D)).astype(np.float32)
    k = RNG.standard_normal((B, S, H, D)).astype(np.float32)
    v = RNG.standard_normal((B, S, H, D)).astype(np.float32)
    sc = 1 / np.sqrt(D)
    ref = mo.ref("tensor_scaled_dot_product_attention", q, k, v, q.shape, scalars=(ctypes.c_float(sc),))
    _close(mo.sdpa(q, k, v, sc), ref, 2e-6)
    # grouped-query k / v: the reference on the repeat_kv expansion
    kg = RNG.standard_normal((B, S, 2, D)).astype(np.float32)
    vg = RNG.standard_normal((B, S, 2, D)).astype(np.float32)
    ref_g = mo.ref("tensor_scaled_dot_product_attention", q, np.repeat(kg, 2, 2), np.repeat(vg, 2, 2), q.shape,
                   scalars=(ctypes.c_float(sc),))
    _close(mo.sdpa(q, kg, vg, sc), ref_g, 2e-6)
    # more keys than queries: query rows are independent, so the reference on q
    # padded to T rows gives the first S rows
    T = 11
    kt = RNG.standard_normal((B, T, H, D)).astype(np.float32)
    vt = RNG.standard_normal((B, T, H, D)).astype(np.float32)
    qp = np.concatenate([q, RNG.standard_normal((B, T - S, H, D)).astype(np.float32)], axis=1)
    ref_t = mo.ref("tensor_scaled_dot_product_attention", qp, kt, vt, qp.shape, scalars=(ctypes.c_float(sc),))
    _close(mo.sdpa(q, kt, vt, sc), ref_t[:, :S], 2e-6)
    # one dominant key: the output is its value row
    kd = np.zeros((1, 4, 1, 8), np.float32)
    kd[0, 2, 0, :] = 100.0
    vd = RNG.standard_normal((1, 4, 1, 8)).astype(np.float32)
    qd = np.ones((1, 1, 1, 8), np.float32)
    _close(mo.sdpa(qd, kd, vd, 1.0)[0, 0, 0], vd[0, 2, 0], 1e-12)


@needs_ref
def test_slice_set_slice_cat_match_reference_exactly():
    L = mo._bind(oracle.ref_lib())
    x = RNG.standard_normal((3, 7, 5)).astype(np.float32)
    for start, shape in [([0, 2, 1], (3, 4, 3)), ([1, 5, 3], (2, 4, 3)), ([2, 0, 0], (3, 7, 5))]:
        ti = oracle.RefTensor(x.shape, x)
        fill = np.full(shape, 7.5, np.float32)
        to = oracle.RefTensor(shape, fill)
        c_start = (ctypes.c_int * 3)(*start)
        c_shape = (ctypes.c_int * 3)(*shape)
        L.tensor_slice(ti.h, to.h, c_start, c_shape)
        assert np.array_equal(mo.slice_from(x, shape, start, fill=7.5), to.f32()), start
        # set_slice of a block into a copy of x
        src = RNG.standard_normal(shape).astype(np.float32)
        td = oracle.RefTensor(x.shape, x)
        ts = oracle.RefTensor(shape, src)
        L.tensor_set_slice(td.h, ts.h, c_start)
        assert np.array_equal(mo.set_slice(x, src, start), td.f32()), start
    parts = [RNG.standard_normal((2, n, 3)).astype(np.float32) for n in (1, 4, 2)]
    ts = [oracle.RefTensor(p.shape, p) for p in parts]
    arr = (ctypes.POINTER(oracle.RefCTensor) * 3)(*[t.h for t in ts])
    to = oracle.RefTensor((2, 7, 3))
    L.tensor_cat(arr, 3, 1, to.h)
    assert np.array_equal(mo.cat(parts, 1), to.f32())
