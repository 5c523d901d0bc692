"""Python mirror of the reference Tensor/Module/Linear API for ``rocm:N`` devices.

The reference engine's Python front end (ip/core/engine/backend.py:201-702) is
torch-free: a ``Tensor`` owns a C ``Tensor*`` created by a backend library and
every op allocates its output and calls one C entry point. This module keeps
that contract on top of libtensor_ops_rocm.so, so model code written against
``Tensor``/``Linear`` runs unchanged, and adds the int8 layers of this path:

* ``W8Linear``   -- weight-only int8 (per-output-channel scales), decode GEMV;
* ``W8A8Linear`` -- per-token int8 activations x int8 weights on MFMA;
* ``MoEW8A8``    -- routed int8 expert layer (replaces Qwen3Coder30BMoE).

The layer ops around the linears (rms_norm, fused_add_rms_norm, rope,
swiglu / fused_swiglu, softmax, argmax, embed, slice / set_slice / reshape,
``cat``, ``scaled_dot_product_attention``, ``RMSNorm``, ``Embedding``) run on
the device too (model_ops.hip), so a reference-style decoder layer with a KV
cache runs on ``rocm:N`` end to end.

Differences from the reference, on purpose:
* tensors free through the library that created them (the reference frees
  every tensor through ``_lib_cpu``, backend.py:266-272);
* failed C calls raise ``RocmError`` instead of being ignored;
* tensors carry a dtype (float32 / float16 / int8 / int32);
* ``reshape`` copies the data into the new tensor (the reference returns a
  fresh tensor of the new shape, backend.py:416-421); ``slice`` zero-fills
  what falls outside the source;
* attention takes grouped-query k / v directly (no repeat_kv copy needed).
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

from . import ops
from .ops import CTensor, RocmError, check, lib

_NP = {"float32": np.float32, "float16": np.float16, "int8": np.int8, "int32": np.int32}
_CODE = {"float32": ops.F32, "float16": ops.F16, "int8": ops.I8, "int32": ops.I32}


def _device_id(device: str) -> int:
    if device == "cpu":
        return -1
    if not device.startswith("rocm"):
        raise ValueError(f"libtensor_ops_rocm serves 'rocm:N' and 'cpu' devices, not {device!r}")
    return int(device.split(":")[1]) if ":" in device else 0


class Tensor:
    """A library-owned tensor. ``data`` may be a list or a numpy array."""

    __slots__ = ("device", "dtype", "_handle", "_src", "__weakref__")

    def __init__(self, shape: Sequence[int], data=None, device: str = "rocm:0",
                 dtype: str = "float32", _handle=None):
        self.device = device
        self.dtype = dtype
        self._src = None
        if _handle is not None:
            self._handle = _handle
        else:
            if dtype not in _CODE:
                raise ValueError(f"unsupported dtype {dtype}")
            c_shape = (ctypes.c_int * len(shape))(*[int(s) for s in shape])
            h = lib.create_tensor_typed(c_shape, len(shape), _device_id(device), _CODE[dtype])
            if not h:
                raise RocmError(f"create_tensor failed: {ops.last_error()}")
            self._handle = h
        if data is not None:
            self.load(data)

    # ------------------------------------------------------------ lifetime
    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None:
            try:
                lib.free_tensor(h)
            except Exception:
                pass
            self._handle = None

    # ---------------------------------------------------------- properties
    @property
    def shape(self) -> Tuple[int, ...]:
        c = self._handle.contents
        return tuple(c.shape[i] for i in range(c.ndim))

    @property
    def ndim(self) -> int:
        return self._handle.contents.ndim

    @property
    def size(self) -> int:
        return self._handle.contents.size

    def data_ptr(self) -> int:
        return ctypes.cast(self._handle.contents.data, ctypes.c_void_p).value or 0

    @property
    def nbytes(self) -> int:
        return self.size * np.dtype(_NP[self.dtype]).itemsize

    # ------------------------------------------------------- data movement
    def load(self, data) -> None:
        arr = np.ascontiguousarray(np.asarray(data, dtype=_NP[self.dtype]))
        if arr.size != self.size:
            raise ValueError(f"load: {arr.size} elements for a tensor of {self.size}")
        check(lib.tensor_load_bytes_status(self._handle, arr.ctypes.data, arr.nbytes),
              "tensor_load_bytes")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=_NP[self.dtype])
        check(lib.tensor_get_bytes_status(self._handle, out.ctypes.data, out.nbytes),
              "tensor_get_bytes")
        return out

    def to_list(self) -> List[float]:
        return self.numpy().ravel().tolist()

    @classmethod
    def from_numpy(cls, arr: np.ndarray, device: str = "rocm:0") -> "Tensor":
        name = str(arr.dtype)
        if name not in _CODE:
            raise ValueError(f"unsupported dtype {arr.dtype}")
        return cls(arr.shape, arr, device=device, dtype=name)

    @classmethod
    def pinned(cls, shape: Sequence[int], dtype: str = "float32") -> "Tensor":
        """A host tensor ("cpu") in pinned memory: copies to and from the GPU
        run as DMA on a stream, overlapping kernels."""
        c_shape = (ctypes.c_int * len(shape))(*[int(x) for x in shape])
        h = lib.create_tensor_pinned(c_shape, len(shape), _CODE[dtype])
        if not h:
            raise RocmError(f"create_tensor_pinned failed: {ops.last_error()}")
        return cls(shape, device="cpu", dtype=dtype, _handle=h)

    def to(self, device: str, non_blocking: bool = False, stream=None) -> "Tensor":
        """Reference Tensor.to (backend.py:302-315): a copy on `device`
        ("cpu" or "rocm:N"). The copy runs on `stream` (a HIPStream or raw
        handle; default the current stream). A host destination is pinned.
        With non_blocking the call returns at once and the result keeps the
        source alive; the caller orders later work after the copy (an event,
        or synchronizing the stream).

        On a stream other than the current one, the copy first waits for the
        work already queued on the current stream (which may still be
        writing this tensor), and a device destination is allocated with that
        stream current, so the allocator's per-stream cache hands its block
        out again only behind the copy that writes it."""
        if device == self.device:
            return self
        sh = _stream_handle(stream)
        cur = lib.get_current_stream()
        side = sh is not None and (sh or None) != (cur or None)
        if side:
            ev = HIPEvent()
            ev.record(None)
            check(lib.stream_wait_event(sh, ev._handle), "stream_wait_event")
            lib.set_current_stream(sh)
        try:
            out = Tensor.pinned(self.shape, self.dtype) if device == "cpu" else \
                Tensor(self.shape, device=device, dtype=self.dtype)
        finally:
            if side:
                lib.set_current_stream(cur)
        check(lib.tensor_copy_async(out._handle, self._handle, sh), "tensor_copy_async")
        if non_blocking:
            out._src = self
        else:
            lib.stream_synchronize(sh)
        return out

    # ----------------------------------------------------------------- ops
    def _new(self, shape, dtype=None) -> "Tensor":
        return Tensor(shape, device=self.device, dtype=dtype or self.dtype)

    def fill(self, value: float) -> None:
        lib.tensor_clear_error()
        lib.tensor_fill(self._handle, ctypes.c_float(value))
        _raise_if_error("tensor_fill")

    def add(self, other: "Tensor") -> "Tensor":
        out = self._new(self.shape)
        lib.tensor_clear_error()
        lib.tensor_add(self._handle, other._handle, out._handle)
        _raise_if_error("tensor_add")
        return out

    def mul(self, other: "Tensor") -> "Tensor":
        out = self._new(self.shape)
        lib.tensor_clear_error()
        lib.tensor_mul(self._handle, other._handle, out._handle)
        _raise_if_error("tensor_mul")
        return out

    __add__ = add
    __mul__ = mul

    def matmul_int8(self, other: "Tensor", out_dtype: str = "float32") -> "Tensor":
        """tensor_matmul_int8 semantics (tensor_ops.c:217-246): self [..,M,K],
        other [..,K,N], both int8."""
        m, k = self.shape[-2:]
        n = other.shape[-1]
        out = self._new(list(self.shape[:-2]) + [m, n], out_dtype)
        fn = lib.tensor_matmul_int8_i32_status if out_dtype == "int32" else lib.tensor_matmul_int8_status
        check(fn(self._handle, other._handle, out._handle), "tensor_matmul_int8")
        return out

    def dequantize(self, scale: "Tensor") -> "Tensor":
        out = self._new(self.shape, "float32")
        check(lib.tensor_dequantize_status(self._handle, scale._handle, out._handle),
              "tensor_dequantize")
        return out

    def quantize_per_token(self) -> Tuple["Tensor", "Tensor"]:
        q = self._new(self.shape, "int8")
        s = self._new(list(self.shape[:-1]) or [1], "float32")
        check(lib.tensor_quantize_per_token_status(self._handle, q._handle, s._handle),
              "tensor_quantize_per_token")
        return q, s

    def rms_norm_quantize(self, weight: "Tensor", eps: float = 1e-6) -> Tuple["Tensor", "Tensor"]:
        """RMSNorm (reference Tensor.rms_norm, backend.py:502-506) and the
        per-token quantizer in one pass: returns (q int8, s fp32)."""
        q = self._new(self.shape, "int8")
        s = self._new(list(self.shape[:-1]) or [1], "float32")
        check(lib.tensor_rms_norm_quantize_status(self._handle, weight._handle, q._handle,
                                                  s._handle, ctypes.c_float(eps)),
              "tensor_rms_norm_quantize")
        return q, s

    def fused_add_rms_norm_quantize(self, residual: "Tensor", weight: "Tensor",
                                    eps: float = 1e-6) -> Tuple["Tensor", "Tensor"]:
        """self <- self + residual in place (as the reference's
        fused_add_rms_norm, backend.py:515-523), then rms_norm_quantize of the
        sum: returns (q, s)."""
        q = self._new(self.shape, "int8")
        s = self._new(list(self.shape[:-1]) or [1], "float32")
        check(lib.tensor_fused_add_rms_norm_quantize_status(self._handle, residual._handle,
                                                            weight._handle, q._handle, s._handle,
                                                            ctypes.c_float(eps)),
              "tensor_fused_add_rms_norm_quantize")
        return q, s

    def linear_w8(self, weight: "Tensor", scale: "Tensor", bias: Optional["Tensor"] = None,
                  out_dtype: Optional[str] = None) -> "Tensor":
        n = weight.shape[0]
        out = self._new(list(self.shape[:-1]) + [n], out_dtype or self.dtype)
        check(lib.tensor_linear_w8_status(self._handle, weight._handle, scale._handle,
                                          bias._handle if bias is not None else None,
                                          out._handle), "tensor_linear_w8")
        return out

    def linear_w8a8(self, s_a: "Tensor", weight: "Tensor", scale: "Tensor",
                    bias: Optional["Tensor"] = None, out_dtype: str = "float16") -> "Tensor":
        n = weight.shape[0]
        out = self._new(list(self.shape[:-1]) + [n], out_dtype)
        check(lib.tensor_linear_w8a8_status(self._handle, s_a._handle, weight._handle,
                                            scale._handle,
                                            bias._handle if bias is not None else None,
                                            out._handle), "tensor_linear_w8a8")
        return out


    # ------------------------- companion ops of the model layers (model_ops.hip)
    def rms_norm(self, weight: "Tensor", eps: float = 1e-6) -> "Tensor":
        """backend.py:502-506 (tensor_ops.c:369-383)."""
        out = self._new(self.shape)
        check(lib.tensor_rms_norm_status(self._handle, weight._handle, out._handle, ctypes.c_float(eps)),
              "tensor_rms_norm")
        return out

    def fused_add_rms_norm(self, residual: "Tensor", weight: "Tensor", eps: float) -> "Tensor":
        """backend.py:515-523: self <- self + residual (in place); returns the
        RMSNorm of the sum."""
        out = self._new(self.shape)
        check(lib.tensor_fused_add_rms_norm_status(self._handle, residual._handle, weight._handle,
                                                   out._handle, ctypes.c_float(eps)),
              "tensor_fused_add_rms_norm")
        return out

    def rope(self, k: "Tensor", cos: "Tensor", sin: "Tensor") -> Tuple["Tensor", "Tensor"]:
        """backend.py:508-513 (tensor_ops.c:384-413); k may have fewer heads."""
        out_q, out_k = self._new(self.shape), k._new(k.shape)
        check(lib.tensor_rope_status(self._handle, k._handle, cos._handle, sin._handle, out_q._handle,
                                     out_k._handle), "tensor_rope")
        return out_q, out_k

    def silu(self) -> "Tensor":
        """backend.py:490-495 (tensor_ops.c:336-342)."""
        out = self._new(self.shape)
        check(lib.tensor_silu_status(self._handle, out._handle), "tensor_silu")
        return out

    def swiglu(self, up_proj_out: "Tensor") -> "Tensor":
        """backend.py:385-393 (tensor_ops.c:579-587): silu(self) * up."""
        out = self._new(self.shape)
        check(lib.tensor_swiglu_status(self._handle, up_proj_out._handle, out._handle), "tensor_swiglu")
        return out

    def fused_swiglu(self) -> "Tensor":
        """backend.py:395-401 (tensor_ops.c:588-604): rows [gate | up]."""
        out = self._new(list(self.shape[:-1]) + [self.shape[-1] // 2])
        check(lib.tensor_fused_gate_up_swiglu_status(self._handle, out._handle),
              "tensor_fused_gate_up_swiglu")
        return out

    def softmax(self, dim: int = -1) -> "Tensor":
        """backend.py:484-488 (tensor_ops.c:351-367), over the last dimension."""
        out = self._new(self.shape)
        check(lib.tensor_softmax_status(self._handle, out._handle), "tensor_softmax")
        return out

    def argmax(self, dim: int = -1) -> "Tensor":
        """backend.py:552-557 (tensor_ops.c:649-661): indices as floats."""
        out = self._new(list(self.shape[:-1]) or [1], "float32")
        check(lib.tensor_argmax_status(self._handle, out._handle), "tensor_argmax")
        return out

    def embed(self, indices: "Tensor") -> "Tensor":
        """backend.py:559-564 (tensor_ops.c:663-671): self is [vocab, dim]."""
        out = self._new(list(indices.shape) + [self.shape[1]])
        check(lib.tensor_embed_status(self._handle, indices._handle, out._handle), "tensor_embed")
        return out

    def slice(self, start_indices: Sequence[int], slice_shapes: Sequence[int]) -> "Tensor":
        """backend.py:566-592 (tensor_ops.c:605-637) with host start indices.
        Elements whose source falls outside self are 0 (the reference leaves
        them as the fresh tensor holds them)."""
        if len(start_indices) != self.ndim or len(slice_shapes) != self.ndim:
            raise ValueError("slice: start and shape need one entry per dimension")
        out = self._new(slice_shapes)
        out.fill(0.0)
        c_start = (ctypes.c_int * self.ndim)(*[int(v) for v in start_indices])
        c_shape = (ctypes.c_int * self.ndim)(*[int(v) for v in slice_shapes])
        check(lib.tensor_slice_status(self._handle, out._handle, c_start, c_shape), "tensor_slice")
        return out

    def set_slice(self, src: "Tensor", start_indices: Sequence[int]) -> None:
        """backend.py:594-611 (tensor_ops.c:504-535): src into self at start."""
        if len(start_indices) != self.ndim:
            raise ValueError("set_slice: start needs one entry per dimension")
        c_start = (ctypes.c_int * self.ndim)(*[int(v) for v in start_indices])
        check(lib.tensor_set_slice_status(self._handle, src._handle, c_start), "tensor_set_slice")

    def reshape(self, new_shape: Sequence[int]) -> "Tensor":
        """backend.py:416-421, with the data: the reference returns a fresh
        tensor of the new shape without copying into it; this one copies
        (tensor_reshape, tensor_ops.c:672)."""
        if int(np.prod(new_shape)) != self.size:
            raise ValueError("Reshape size mismatch")
        out = self._new(new_shape)
        check(lib.tensor_reshape_status(self._handle, out._handle), "tensor_reshape")
        return out

def _stream_handle(stream):
    """Raw handle of a HIPStream (or a raw handle / None: the current stream)."""
    if stream is None:
        return None
    return getattr(stream, "_handle", stream)


def _raise_if_error(what: str) -> None:
    msg = ops.last_error()
    if msg:
        raise RocmError(f"{what} failed: {msg}")


# ---------------------------------------------------------------- modules
class Module:
    """Same surface as the reference Module (backend.py:656-693)."""

    def __init__(self):
        self._parameters = {}
        self._modules = {}
        self.training = False

    def __call__(self, *a, **k):
        return self.forward(*a, **k)

    def forward(self, *a, **k):
        raise NotImplementedError

    def register_parameter(self, name: str, p):
        self._parameters[name] = p

    def parameters(self):
        for p in self._parameters.values():
            if p is not None:
                yield p
        for m in self._modules.values():
            yield from m.parameters()

    def named_parameters(self, prefix: str = ""):
        for n, p in self._parameters.items():
            if p is not None:
                yield prefix + n, p
        for n, m in self._modules.items():
            yield from m.named_parameters(prefix + n + ".")

    def _set_parameter(self, name: str, value) -> None:
        """Replaces a parameter (dotted names reach submodules), keeping the
        attribute of the same name in step, as the reference's Module.to does."""
        if "." in name:
            head, rest = name.split(".", 1)
            self._modules[head]._set_parameter(rest, value)
            return
        self._parameters[name] = value
        if hasattr(self, name):
            setattr(self, name, value)

    def to(self, device: str, non_blocking: bool = False, stream=None):
        """Reference Module.to (backend.py:665-674): every parameter moved."""
        for name, p in list(self.named_parameters()):
            self._set_parameter(name, p.to(device, non_blocking=non_blocking, stream=stream))
        return self

    def state_dict(self, prefix: str = "", destination=None):
        destination = {} if destination is None else destination
        for n, p in self._parameters.items():
            if p is not None:
                destination[prefix + n] = p
        for n, m in self._modules.items():
            m.state_dict(prefix + n + ".", destination)
        return destination


class W8Linear(Module):
    """Drop-in for the reference Linear (backend.py:695-702) with int8 weights
    [out, in] and per-output-channel fp32 scales; forward(x) = x.linear_w8(...)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device: str = "rocm:0"):
        super().__init__()
        self.weight = Tensor([out_features, in_features], device=device, dtype="int8")
        self.weight_scale = Tensor([out_features], device=device)
        self.bias = Tensor([out_features], device=device) if bias else None
        self.register_parameter("weight", self.weight)
        self.register_parameter("weight_scale", self.weight_scale)
        if bias:
            self.register_parameter("bias", self.bias)

    def load_quantized(self, q: np.ndarray, s: np.ndarray, b: Optional[np.ndarray] = None):
        self.weight.load(q)
        self.weight_scale.load(s)
        if b is not None:
            if self.bias is None:
                raise ValueError("layer was created without bias")
            self.bias.load(b)

    def load_float(self, w: np.ndarray, b: Optional[np.ndarray] = None):
        """Quantize an fp weight [out, in] per output channel on the GPU
        (s = amax_row / 127, q = rint(w / s)) and load it."""
        from .weights import quantize_array
        q, s = quantize_array(w, self.weight.device)
        self.load_quantized(q, s, b)

    def forward(self, x: Tensor) -> Tensor:
        return x.linear_w8(self.weight, self.weight_scale, self.bias)


class W8A8Linear(W8Linear):
    """Prefill / expert linear: per-token int8 activations on int8 MFMA."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device: str = "rocm:0", out_dtype: str = "float16"):
        super().__init__(in_features, out_features, bias, device)
        self.out_dtype = out_dtype

    def forward(self, x: Tensor) -> Tensor:
        q, s = x.quantize_per_token()
        return self.forward_quantized(q, s)

    def forward_quantized(self, q: Tensor, s: Tensor) -> Tensor:
        """The linear on activations already quantized per token, e.g. by
        Tensor.rms_norm_quantize, which folds the quantizer into the RMSNorm
        that produces a prefill layer's qkv and gate_up inputs."""
        return q.linear_w8a8(s, self.weight, self.weight_scale, self.bias, self.out_dtype)


class MoEW8A8(Module):
    """Routed int8 expert layer: forward(x [T,H], router_logits [T,E]) -> [T,H]."""

    def __init__(self, hidden: int, intermediate: int, num_experts: int, top_k: int,
                 renormalize: bool = False, device: str = "rocm:0", out_dtype: str = "float32"):
        super().__init__()
        self.top_k, self.renormalize, self.out_dtype = top_k, renormalize, out_dtype
        E, H, I = num_experts, hidden, intermediate
        self.w_gate_up = Tensor([E, 2 * I, H], device=device, dtype="int8")
        self.s_gate_up = Tensor([E, 2 * I], device=device)
        self.w_down = Tensor([E, H, I], device=device, dtype="int8")
        self.s_down = Tensor([E, H], device=device)
        for n in ("w_gate_up", "s_gate_up", "w_down", "s_down"):
            self.register_parameter(n, getattr(self, n))

    def forward(self, x: Tensor, router_logits: Tensor) -> Tensor:
        out = Tensor(list(x.shape), device=x.device, dtype=self.out_dtype)
        check(lib.tensor_moe_w8a8_status(x._handle, router_logits._handle, self.w_gate_up._handle,
                                         self.s_gate_up._handle, self.w_down._handle,
                                         self.s_down._handle, self.top_k,
                                         int(self.renormalize), out._handle), "tensor_moe_w8a8")
        return out


# ------------------------------------- model-layer functions and modules
def cat(tensors: List[Tensor], axis: int = 0) -> Tensor:
    """backend.py:740-754 (tensor_ops.c:702-718)."""
    if not tensors:
        return None
    shape = list(tensors[0].shape)
    shape[axis] = sum(t.shape[axis] for t in tensors)
    out = tensors[0]._new(shape)
    arr = (ctypes.POINTER(CTensor) * len(tensors))(*[t._handle for t in tensors])
    check(lib.tensor_cat_status(arr, len(tensors), axis, out._handle), "tensor_cat")
    return out


def scaled_dot_product_attention(q: Tensor, k: Tensor, v: Tensor, scale: Optional[float] = None) -> Tensor:
    """backend.py:771-790 (tensor_ops.c:536-578): q [B, S, H, D], k / v
    [B, T, Hk, D] (Hk dividing H: no repeat_kv copy needed), no mask."""
    if scale is None:
        scale = 1.0 / (q.shape[-1] ** 0.5)
    out = q._new(q.shape)
    check(lib.tensor_scaled_dot_product_attention_status(q._handle, k._handle, v._handle, out._handle,
                                                         ctypes.c_float(scale)),
          "tensor_scaled_dot_product_attention")
    return out


class RMSNorm(Module):
    """backend.py:726-731."""

    def __init__(self, normalized_shape: int, eps: float = 1e-6, device: str = "rocm:0"):
        super().__init__()
        self.eps = eps
        self.weight = Tensor([normalized_shape], device=device)
        self.register_parameter("weight", self.weight)

    def forward(self, input: Tensor) -> Tensor:
        return input.rms_norm(self.weight, self.eps)


class Embedding(Module):
    """backend.py:719-724."""

    def __init__(self, num_embeddings: int, embedding_dim: int, device: str = "rocm:0"):
        super().__init__()
        self.weight = Tensor([num_embeddings, embedding_dim], device=device)
        self.register_parameter("weight", self.weight)

    def forward(self, input: Tensor) -> Tensor:
        return self.weight.embed(input)


# ------------------------------------------------- allocator and streams
def init_memory_pool(size_mb: int = 1024) -> None:
    """Reserve the HBM arena (reference: backend.py:792-799, CPU arena)."""
    lib.init_memory_pool(size_mb * 1024 * 1024)


def reset_memory_pool() -> None:
    lib.reset_memory_pool()


def allocate_pinned(size_bytes: int):
    return lib.allocate_pinned_memory(size_bytes)


def free_pinned(ptr) -> None:
    lib.free_pinned_memory(ptr)


def synchronize() -> None:
    lib.stream_synchronize(None)


class HIPStream:
    """Mirror of the reference CUDAStream (backend.py:165-189): an in-order
    stream of the library; ``with stream:`` makes it the current stream for
    every op (and restores the previous one on exit)."""

    def __init__(self):
        self._handle = lib.create_stream()
        if not self._handle:
            raise RocmError(f"create_stream failed: {ops.last_error()}")
        self._prev = None

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h:
            try:
                lib.destroy_stream(h)
            except Exception:
                pass
            self._handle = None

    def synchronize(self):
        lib.stream_synchronize(self._handle)

    def __enter__(self):
        self._prev = lib.get_current_stream()
        lib.set_current_stream(self._handle)
        return self

    def __exit__(self, exc_type, exc_val, exc_tb):
        lib.set_current_stream(self._prev)
        self._prev = None

    def record_event(self) -> "HIPEvent":
        ev = HIPEvent()
        ev.record(self)
        return ev

    def wait_event(self, ev: "HIPEvent") -> None:
        check(lib.stream_wait_event(self._handle, ev._handle), "stream_wait_event")


class HIPEvent:
    """Orders one stream's later work after what another stream queued before
    the event (no reference counterpart; hybrid_scheduler.py:51-53 notes it
    would need one)."""

    def __init__(self):
        self._handle = lib.create_event()
        if not self._handle:
            raise RocmError(f"create_event failed: {ops.last_error()}")

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h:
            try:
                lib.destroy_event(h)
            except Exception:
                pass
            self._handle = None

    def record(self, stream=None) -> None:
        check(lib.record_event(self._handle, _stream_handle(stream)), "record_event")

    @classmethod
    def on_current_stream(cls) -> "HIPEvent":
        """An event recorded on the current stream now."""
        ev = cls()
        ev.record(None)
        return ev

    def synchronize(self) -> None:
        check(lib.event_synchronize(self._handle), "event_synchronize")

    def query(self) -> bool:
        r = lib.event_query(self._handle)
        if r < 0:
            raise RocmError(f"event_query failed: {ops.last_error()}")
        return r == 1


class HIPGraph:
    """Mirror of the reference CUDAGraph wrapper (backend.py:801-810)."""

    def capture_begin(self):
        lib.begin_capture()

    def capture_end(self):
        lib.end_capture()

    def replay(self):
        lib.replay_graph()
