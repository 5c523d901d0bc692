"""Oracle of the model-layer companion ops -- TEST INFRASTRUCTURE ONLY.

numpy restatements of the reference CPU backend's ops that a decoder layer
calls around its linears (plugins/cpu/c_src/tensor_ops.c, cited per
function), the checker of mod_amd/csrc/model_ops.hip. Floating-point ops are
evaluated in float64 (the GPU result is held to a stated fp32 tolerance
against them); index and data-movement ops are exact.

Pinning: tests/test_oracle_model_ops.py runs each restatement against the
reference's own compiled functions (oracle/_ref/libtensor_ops_ref.so, built
from tensor_ops.c) on the inputs where the reference loop is defined, and
against closed forms (softmax sums, rotation norms, one-hot attention) where
this restatement goes past it (grouped-query k in rope and attention, more
keys than queries).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import RefCTensor, RefTensor, ref_lib

NEG = -1e9   # the reference's starting maximum (tensor_ops.c:358, 543-567, 654)


def rms_norm(x, w, eps):
    """tensor_ops.c:369-383: x * (1 / sqrt(sum(x^2) / cols + eps)) * w per row."""
    x = np.asarray(x, np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x * (1.0 / np.sqrt(ms + eps)) * np.asarray(w, np.float64)


def fused_add_rms_norm(x, residual, w, eps):
    """tensor_ops_cuda.cu:220-240 (bound at backend.py:157, 515): returns
    (x + residual, rms_norm(x + residual)); the op stores the sum into x."""
    s = np.asarray(x, np.float64) + np.asarray(residual, np.float64)
    return s, rms_norm(s, w, eps)


def rope(q, k, cos, sin):
    """tensor_ops.c:384-413 (rotate-half): q [.., S, Hq, D], k [.., S, Hk, D],
    cos / sin rows s of [>= S, D/2]. k with its own head count (the reference
    loop assumes Hk == Hq)."""
    def rot(x):
        x = np.asarray(x, np.float64)
        S, D = x.shape[-3], x.shape[-1]
        h = D // 2
        c = np.asarray(cos, np.float64).reshape(-1, h)[:S][:, None, :]
        s = np.asarray(sin, np.float64).reshape(-1, h)[:S][:, None, :]
        re, im = x[..., :h], x[..., h:]
        return np.concatenate([re * c - im * s, re * s + im * c], axis=-1)
    return rot(q), rot(k)


def silu(x):
    """tensor_ops.c:336-342."""
    x = np.asarray(x, np.float64)
    return x * (1.0 / (1.0 + np.exp(-x)))


def swiglu(gate, up):
    """tensor_ops.c:579-587."""
    return silu(gate) * np.asarray(up, np.float64)


def fused_gate_up_swiglu(gate_up):
    """tensor_ops.c:588-604: rows [gate | up] of 2h columns -> h columns."""
    gu = np.asarray(gate_up, np.float64)
    h = gu.shape[-1] // 2
    return silu(gu[..., :h]) * gu[..., h:]


def softmax(x):
    """tensor_ops.c:351-367: max from -1e9, exp(x - max), times 1 / sum."""
    x = np.asarray(x, np.float64)
    m = np.maximum(np.max(x, axis=-1, keepdims=True), NEG)
    e = np.exp(x - m)
    return e * (1.0 / np.sum(e, axis=-1, keepdims=True))


def argmax(x):
    """tensor_ops.c:649-661: per row the first index of the largest value
    strictly above -1e9 (the scan's start), 0 when there is none (NaN never
    wins a strict comparison). Exact."""
    x = np.asarray(x, np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros(rows.shape[0], np.float32)
    for r, row in enumerate(rows):
        ok = row > np.float32(NEG)   # False for NaN
        if ok.any():
            m = row[ok].max()
            out[r] = float(np.flatnonzero(ok & (row == m))[0])
    return out.reshape(x.shape[:-1])


def embed(weight, indices):
    """tensor_ops.c:663-671: rows weight[(int)idx] (C truncation), rows
    outside [0, vocab) -> row 0. Exact."""
    w = np.asarray(weight, np.float32)
    f = np.asarray(indices, np.float32).ravel()
    idx = np.zeros(f.size, np.int64)
    fin = np.isfinite(f) & (f > -2147483648.0) & (f < 2147483648.0)
    idx[fin] = np.trunc(f[fin]).astype(np.int64)
    idx[(idx < 0) | (idx >= w.shape[0])] = 0
    return w[idx].reshape(tuple(np.shape(indices)) + (w.shape[1],))


def sdpa(q, k, v, scale):
    """tensor_ops.c:536-578: q [B, S, H, D], k / v [B, T, Hk, D]; scores over
    all T keys (no mask), softmax with max from -1e9, normalised weights
    times v. Query head h reads kv head h // (H // Hk) (the copy repeat_kv,
    qwen3_0_6b/architecture.py:57-66, puts there); the reference loop itself
    has T == S and Hk == H."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    H, Hk = q.shape[2], k.shape[2]
    rep = H // Hk
    k = np.repeat(k, rep, axis=2)
    v = np.repeat(v, rep, axis=2)
    sc = np.einsum("bshd,bthd->bhst", q, k) * scale
    p = softmax(sc)
    return np.einsum("bhst,bthd->bshd", p, v)


def _strides(shape):
    st = [1] * len(shape)
    for d in range(len(shape) - 2, -1, -1):
        st[d] = st[d + 1] * shape[d + 1]
    return st


def slice_from(inp, out_shape, start, fill=0.0):
    """tensor_ops.c:605-637: out[i] = inp[sum((start[d] + coord_out[d]) *
    stride_in[d])]; where that offset falls outside inp, out keeps its value
    (here `fill`). Exact."""
    inp = np.asarray(inp, np.float32)
    out = np.full(out_shape, fill, np.float32)
    return _walk(inp.ravel(), out.ravel(), list(out_shape), list(inp.shape), start, gather=True).reshape(out_shape)


def set_slice(dst, src, start):
    """tensor_ops.c:504-535: dst[sum((start[d] + coord_src[d]) *
    stride_dst[d])] = src[i], skipped when the offset falls outside dst.
    Exact; returns the new dst."""
    dst = np.array(dst, np.float32, copy=True)
    src = np.asarray(src, np.float32)
    return _walk(src.ravel(), dst.ravel(), list(src.shape), list(dst.shape), start, gather=False).reshape(dst.shape)


def _walk(a, b, walk_shape, other_shape, start, gather):
    sw = _strides(walk_shape)
    so = _strides(other_shape)
    n_other = int(np.prod(other_shape))
    n = int(np.prod(walk_shape))
    b = b.copy()
    for i in range(n):
        rem, off = i, 0
        for d in range(len(walk_shape)):
            if sw[d] == 0:
                continue
            c = rem // sw[d]
            rem -= c * sw[d]
            off += (start[d] + c) * so[d]
        if 0 <= off < n_other:
            if gather:
                b[i] = a[off]
            else:
                b[off] = a[i]
    return b


def cat(inputs, axis):
    """tensor_ops.c:702-718 (the inputs in order along axis). Exact."""
    return np.concatenate([np.asarray(t, np.float32) for t in inputs], axis=axis)


# ------------------------------------------------ the reference's own functions
def _bind(L):
    T = ctypes.POINTER(RefCTensor)
    L.tensor_rope.argtypes = [T, T, T, T, T, T]
    L.tensor_silu.argtypes = [T, T]
    L.tensor_swiglu.argtypes = [T, T, T]
    L.tensor_scaled_dot_product_attention.argtypes = [T, T, T, T, ctypes.c_float]
    L.tensor_embed.argtypes = [T, T, T]
    L.tensor_slice.argtypes = [T, T, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    L.tensor_set_slice.argtypes = [T, T, ctypes.POINTER(ctypes.c_int)]
    L.tensor_cat.argtypes = [ctypes.POINTER(T), ctypes.c_int, ctypes.c_int, T]
    L.tensor_reshape.argtypes = [T, T]
    return L


def ref(name, *arrays_and_shapes, scalars=()):
    """Runs reference function `name` on fp32 host tensors: each argument is
    an array (loaded) or a shape tuple (an output, returned in order)."""
    L = _bind(ref_lib())
    ts, outs = [], []
    for a in arrays_and_shapes:
        if isinstance(a, tuple):
            t = RefTensor(a)
            outs.append(t)
        else:
            a = np.ascontiguousarray(a, np.float32)
            t = RefTensor(a.shape, a)
        ts.append(t)
    getattr(L, name)(*[t.h for t in ts], *scalars)
    res = [t.f32() for t in outs]
    return res[0] if len(res) == 1 else res
