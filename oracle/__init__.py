"""CPU oracle for the int8 quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker; the product
(``mod_amd``) never imports it and fails loudly when its HIP library is missing.

Two native libraries back it:

* ``liboracle_int8.so`` -- ``int8_ref.c``, the restatement of the path (each C
  function cites the reference file:line it follows);
* ``_ref/libtensor_ops_ref.so`` -- the reference's own CPU backend
  (``plugins/cpu/c_src/tensor_ops.c``) compiled from its source by
  ``oracle/Makefile``; used to pin the restatement and as the CPU baseline.

Parity status of each function (how it is pinned) is listed in the docstrings.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle_int8.so"
REF_LIB = HERE / "_ref" / "libtensor_ops_ref.so"
REF_LIB_BUILDOPS = HERE / "_ref" / "libtensor_ops_ref_buildops.so"
REFERENCE_SRC = Path("/root/reference/src/inference_pio/plugins")

_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_u16p = ctypes.POINTER(ctypes.c_uint16)
_vp = ctypes.c_void_p


def build(with_reference: bool | None = None) -> None:
    """Compile the restatement and, when the reference tree is present, the
    reference CPU library (``make -C oracle``)."""
    if with_reference is None:
        with_reference = REFERENCE_SRC.exists()
    target = "all" if with_reference else "oracle"
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), target], check=True)


def _load(path: Path) -> ctypes.CDLL:
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built (run `make -C {HERE}`)")
    return ctypes.CDLL(str(path))


_lib = None
_ref = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load(ORACLE_LIB)
        L = _lib
        L.ref_f32_to_f16.restype = ctypes.c_uint16
        L.ref_f32_to_f16.argtypes = [ctypes.c_float]
        L.ref_f16_to_f32.restype = ctypes.c_float
        L.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ref_f32_to_f16_array.argtypes = [_c_f32p, _c_u16p, ctypes.c_int64]
        L.ref_matmul_int8.argtypes = [_c_i8p, _c_i8p, _c_f32p] + [ctypes.c_int] * 4
        L.ref_matmul_int8_i32.argtypes = [_c_i8p, _c_i8p, _c_i32p] + [ctypes.c_int] * 4
        L.ref_matmul_nt_i32.argtypes = [_c_i8p, _c_i8p, _c_i32p] + [ctypes.c_int] * 3
        L.ref_linear_f32.argtypes = [_c_f32p, _c_f32p, _c_f32p, _c_f32p] + [ctypes.c_int] * 3
        L.ref_gemv_w8.argtypes = [_vp, ctypes.c_int, _c_i8p, _c_f32p, _c_f32p, _vp,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.ref_quant_per_token.argtypes = [_vp, ctypes.c_int, _c_i8p, _c_f32p, ctypes.c_int,
                                          ctypes.c_int]
        L.ref_w8a8.argtypes = [_c_i8p, _c_f32p, _c_i8p, _c_f32p, _c_f32p, _vp, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.ref_softmax.argtypes = [_c_f32p, _c_f32p, ctypes.c_int, ctypes.c_int]
        L.ref_topk.argtypes = [_c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_f32p,
                               _c_i32p]
        L.ref_moe_route.argtypes = [_c_f32p] + [ctypes.c_int] * 4 + [_c_f32p, _c_i32p]
        L.ref_moe_w8a8.argtypes = [_vp, ctypes.c_int, _c_f32p, _c_i8p, _c_f32p, _c_i8p, _c_f32p,
                                   _vp, ctypes.c_int] + [ctypes.c_int] * 6
        L.ref_moe_group.argtypes = [_c_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_i32p,
                                    _c_i32p, _c_i32p]
        L.ref_rmsnorm_quant.argtypes = [_vp, ctypes.c_int, _vp, _vp, _c_f32p, ctypes.c_float,
                                        _c_i8p, _c_f32p, _c_f32p, ctypes.c_int, ctypes.c_int]
        L.ref_num_threads.restype = ctypes.c_int
        L.ref_exp_det.restype = ctypes.c_float
        L.ref_exp_det.argtypes = [ctypes.c_float]
        L.ref_exp_det_array.argtypes = [_c_f32p, _c_f32p, ctypes.c_int64]
    return _lib


def _p(a: np.ndarray, ct):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ct)


def _vpp(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


# --------------------------------------------------------------------- fp16
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """RNE float->half bits (pinned against numpy's astype(float16))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ref_f32_to_f16_array(_p(x, _c_f32p), _p(out, _c_u16p), x.size)
    return out


def exp_det(x: np.ndarray) -> np.ndarray:
    """The deterministic fp32 e^x of the MoE SwiGLU (int8_ref.c ref_exp_det).
    Pinned against float64 exp (<= 2 ulp) and special values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().ref_exp_det_array(_p(x, _c_f32p), _p(out, _c_f32p), x.size)
    return out


# --------------------------------------------------------------- int8 matmul
def matmul_int8(a: np.ndarray, b: np.ndarray, out_i32: bool = False) -> np.ndarray:
    """tensor_ops.c:217-246 restated. a [batch,m,k] int8, b [batch,k,n] int8.
    Pinned: bitwise vs the reference library and numpy int64 matmul."""
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    if a.ndim == 2:
        a, b = a[None], b[None]
    batch, m, k = a.shape
    n = b.shape[-1]
    if out_i32:
        c = np.empty((batch, m, n), np.int32)
        lib().ref_matmul_int8_i32(_p(a, _c_i8p), _p(b, _c_i8p), _p(c, _c_i32p), batch, m, k, n)
    else:
        c = np.empty((batch, m, n), np.float32)
        lib().ref_matmul_int8(_p(a, _c_i8p), _p(b, _c_i8p), _p(c, _c_f32p), batch, m, k, n)
    return c


def matmul_nt_i32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """int32 a @ w.T with w in the Linear layout [n,k]."""
    a = np.ascontiguousarray(a, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    m, k = a.shape
    n = w.shape[0]
    c = np.empty((m, n), np.int32)
    lib().ref_matmul_nt_i32(_p(a, _c_i8p), _p(w, _c_i8p), _p(c, _c_i32p), m, n, k)
    return c


def linear_f32(x, W, bias=None):
    """tensor_ops.c:301-335 restated (fp32 Linear)."""
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    m, k = x.shape
    n = W.shape[0]
    y = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().ref_linear_f32(_p(x, _c_f32p), _p(W, _c_f32p), None if b is None else _p(b, _c_f32p),
                         _p(y, _c_f32p), m, n, k)
    return y


# ---------------------------------------------------------------------- GEMV
def gemv_w8(x, W, s_w, bias=None, out_dtype=np.float32):
    """y = s_w * (x @ W.T) + bias; x fp32|fp16 [m,k], W int8 [n,k]."""
    x = np.ascontiguousarray(x)
    x_f16 = int(x.dtype == np.float16)
    if not x_f16:
        x = x.astype(np.float32, copy=False)
    W = np.ascontiguousarray(W, np.int8)
    s_w = np.ascontiguousarray(s_w, np.float32)
    m, k = x.shape
    n = W.shape[0]
    y = np.empty((m, n), np.float16 if out_dtype == np.float16 else np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().ref_gemv_w8(_vpp(x), x_f16, _p(W, _c_i8p), _p(s_w, _c_f32p),
                      None if b is None else _p(b, _c_f32p), _vpp(y),
                      int(y.dtype == np.float16), m, n, k)
    return y


# ----------------------------------------------------------------- quantizer
def quant_per_token(x):
    """Per-token symmetric int8 quantization; returns (q int8 [m,k], s fp32 [m])."""
    x = np.ascontiguousarray(x)
    x_f16 = int(x.dtype == np.float16)
    if not x_f16:
        x = x.astype(np.float32, copy=False)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    lib().ref_quant_per_token(_vpp(x), x_f16, _p(q, _c_i8p), _p(s, _c_f32p), m, k)
    return q, s


# ---------------------------------------------------------------------- W8A8
def rmsnorm_quant(x, w, eps=1e-6, residual=None):
    """RMSNorm (optionally after a residual add) then the per-token quantizer
    (int8_ref.c ref_rmsnorm_quant). x, residual: [M, K] fp32 or fp16 (same
    dtype), w: [K]. Returns (q, s, y, x_sum): y the normalized fp32 values the
    quantizer saw, x_sum = x + residual in x's dtype (None without residual)."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    x_f16 = int(x.dtype == np.float16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    y = np.empty((m, k), np.float32)
    r = None if residual is None else np.ascontiguousarray(residual, dtype=x.dtype)
    xs = None if residual is None else np.empty_like(x)
    lib().ref_rmsnorm_quant(_vpp(x), x_f16, _vpp(r), _vpp(xs), _p(w, _c_f32p), eps,
                            _p(q, _c_i8p), _p(s, _c_f32p), _p(y, _c_f32p), m, k)
    return q, s, y, xs


def ref_rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Runs the reference tensor_rms_norm (fp32) itself."""
    tx = RefTensor(x.shape, x.astype(np.float32))
    tw = RefTensor(w.shape, w.astype(np.float32))
    to = RefTensor(x.shape)
    tx.L.tensor_rms_norm(tx.h, tw.h, to.h, ctypes.c_float(eps))
    return to.f32()


def w8a8(q, s_a, W, s_w, bias=None, out="f16"):
    """acc = q @ W.T (int32); y = float(acc)*s_a*s_w (+bias). out in f32|f16|i32."""
    q = np.ascontiguousarray(q, np.int8)
    W = np.ascontiguousarray(W, np.int8)
    s_a = np.ascontiguousarray(s_a, np.float32)
    s_w = np.ascontiguousarray(s_w, np.float32)
    m, k = q.shape
    n = W.shape[0]
    kind = {"f32": 0, "f16": 1, "i32": 3}[out]
    y = np.empty((m, n), {"f32": np.float32, "f16": np.float16, "i32": np.int32}[out])
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().ref_w8a8(_p(q, _c_i8p), _p(s_a, _c_f32p), _p(W, _c_i8p), _p(s_w, _c_f32p),
                   None if b is None else _p(b, _c_f32p), _vpp(y), kind, m, n, k)
    return y


# ----------------------------------------------------------------------- MoE
def softmax(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().ref_softmax(_p(x, _c_f32p), _p(out, _c_f32p), x.shape[0], x.shape[1])
    return out


def topk(x, k):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    v = np.empty((rows, k), np.float32)
    i = np.empty((rows, k), np.int32)
    lib().ref_topk(_p(x, _c_f32p), rows, cols, k, _p(v, _c_f32p), _p(i, _c_i32p))
    return v, i


def moe_route(logits, k, renorm=False):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    w = np.empty((T, k), np.float32)
    i = np.empty((T, k), np.int32)
    lib().ref_moe_route(_p(logits, _c_f32p), T, E, k, int(renorm), _p(w, _c_f32p), _p(i, _c_i32p))
    return w, i


def moe_group(ids, E):
    ids = np.ascontiguousarray(ids, np.int32)
    T, k = ids.shape
    off = np.empty(E + 1, np.int32)
    rows = np.empty(T * k, np.int32)
    pos = np.empty(T * k, np.int32)
    lib().ref_moe_group(_p(ids, _c_i32p), T, E, k, _p(off, _c_i32p), _p(rows, _c_i32p),
                        _p(pos, _c_i32p))
    return off, rows, pos


def moe_w8a8(x, logits, w_gu, s_gu, w_down, s_down, k, renorm=False, out_dtype=np.float32):
    x = np.ascontiguousarray(x)
    x_f16 = int(x.dtype == np.float16)
    if not x_f16:
        x = x.astype(np.float32, copy=False)
    logits = np.ascontiguousarray(logits, np.float32)
    w_gu = np.ascontiguousarray(w_gu, np.int8)
    w_down = np.ascontiguousarray(w_down, np.int8)
    s_gu = np.ascontiguousarray(s_gu, np.float32)
    s_down = np.ascontiguousarray(s_down, np.float32)
    T, H = x.shape
    E, I2, _ = w_gu.shape
    out = np.empty((T, H), np.float16 if out_dtype == np.float16 else np.float32)
    lib().ref_moe_w8a8(_vpp(x), x_f16, _p(logits, _c_f32p), _p(w_gu, _c_i8p), _p(s_gu, _c_f32p),
                       _p(w_down, _c_i8p), _p(s_down, _c_f32p), _vpp(out),
                       int(out.dtype == np.float16), T, H, I2 // 2, E, k, int(renorm))
    return out


# ------------------------------------------------------- reference library
class RefCTensor(ctypes.Structure):
    """The reference Tensor struct (plugins/common/tensor.h:19-25)."""
    _fields_ = [("data", ctypes.POINTER(ctypes.c_float)), ("shape", ctypes.POINTER(ctypes.c_int)),
                ("ndim", ctypes.c_int), ("size", ctypes.c_int), ("device_id", ctypes.c_int)]


def ref_available() -> bool:
    return REF_LIB.exists()


def ref_lib(buildops_flags: bool = False) -> ctypes.CDLL:
    """The reference CPU backend compiled from /root/reference sources."""
    global _ref
    if buildops_flags:
        L = _load(REF_LIB_BUILDOPS)
    else:
        if _ref is not None:
            return _ref
        L = _ref = _load(REF_LIB)
    T = ctypes.POINTER(RefCTensor)
    L.create_tensor.restype = T
    L.create_tensor.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
    L.free_tensor.argtypes = [T]
    L.tensor_load_data.argtypes = [T, _c_f32p, ctypes.c_int]
    L.tensor_get_data.argtypes = [T, _c_f32p, ctypes.c_int]
    for nm in ("tensor_matmul_int8", "tensor_matmul", "tensor_matmul_transposed"):
        getattr(L, nm).argtypes = [T, T, T]
    L.tensor_linear.argtypes = [T, T, T, T]
    L.tensor_softmax.argtypes = [T, T]
    L.tensor_topk.argtypes = [T, ctypes.c_int, T, T]
    L.tensor_fused_gate_up_swiglu.argtypes = [T, T]
    L.tensor_count_value.argtypes = [T, ctypes.c_float, ctypes.POINTER(ctypes.c_int)]
    L.tensor_gather_by_value.argtypes = [T, T, ctypes.c_float, T, T]
    L.tensor_scatter_add_by_index.argtypes = [T, T, T]
    L.tensor_rms_norm.argtypes = [T, T, T, ctypes.c_float]
    L.tensor_argmax.argtypes = [T, T]
    L.tensor_fill.argtypes = [T, ctypes.c_float]
    return L


class RefTensor:
    """Owns one reference Tensor*; payload loaded as raw bytes, the way the
    reference carries int8 inside its float buffer (tensor_ops.c:227-228)."""

    def __init__(self, shape, data: np.ndarray | None = None, lib_=None):
        self.L = lib_ or ref_lib()
        shp = (ctypes.c_int * len(shape))(*shape)
        self.h = self.L.create_tensor(shp, len(shape), -1)
        self.shape = tuple(shape)
        self.size = int(np.prod(shape)) if shape else 1
        if data is not None:
            self.load(data)

    def load(self, data: np.ndarray) -> None:
        raw = np.ascontiguousarray(data).view(np.uint8).ravel()
        words = (raw.size + 3) // 4
        buf = np.zeros(words * 4, np.uint8)
        buf[: raw.size] = raw
        self.L.tensor_load_data(self.h, buf.ctypes.data_as(_c_f32p), words)

    def f32(self) -> np.ndarray:
        out = np.empty(self.size, np.float32)
        self.L.tensor_get_data(self.h, out.ctypes.data_as(_c_f32p), self.size)
        return out.reshape(self.shape)

    def __del__(self):
        try:
            self.L.free_tensor(self.h)
        except Exception:
            pass


def ref_matmul_int8(a: np.ndarray, b: np.ndarray, lib_=None) -> np.ndarray:
    """Runs the reference tensor_matmul_int8 itself (a [..,m,k], b [..,k,n])."""
    m, k = a.shape[-2:]
    n = b.shape[-1]
    ta = RefTensor(a.shape, a.astype(np.int8), lib_)
    tb = RefTensor(b.shape, b.astype(np.int8), lib_)
    to = RefTensor(a.shape[:-2] + (m, n), None, lib_)
    ta.L.tensor_matmul_int8(ta.h, tb.h, to.h)
    return to.f32()


def ref_linear(x: np.ndarray, W: np.ndarray, bias=None, lib_=None) -> np.ndarray:
    """Runs the reference tensor_linear (fp32) itself."""
    tx = RefTensor(x.shape, x.astype(np.float32), lib_)
    tw = RefTensor(W.shape, W.astype(np.float32), lib_)
    tb = None if bias is None else RefTensor(bias.shape, bias.astype(np.float32), lib_)
    to = RefTensor(x.shape[:-1] + (W.shape[0],), None, lib_)
    tx.L.tensor_linear(tx.h, tw.h, None if tb is None else tb.h, to.h)
    return to.f32()


def ref_softmax(x: np.ndarray) -> np.ndarray:
    tx = RefTensor(x.shape, x.astype(np.float32))
    to = RefTensor(x.shape)
    tx.L.tensor_softmax(tx.h, to.h)
    return to.f32()


def ref_topk(x: np.ndarray, k: int):
    tx = RefTensor(x.shape, x.astype(np.float32))
    tv = RefTensor(x.shape[:-1] + (k,))
    ti = RefTensor(x.shape[:-1] + (k,))
    tx.L.tensor_topk(tx.h, k, tv.h, ti.h)
    return tv.f32(), ti.f32().astype(np.int32)


def threads() -> int:
    return int(lib().ref_num_threads())


__all__ = [n for n in dir() if not n.startswith("_")]
