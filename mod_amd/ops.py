"""ctypes binding of libtensor_ops_rocm.so (raw-pointer layer + signatures).

The library is the product: there is no CPU or PyTorch fallback. Importing this
module without the built library raises ``ImportError`` so a missing build is
never mistaken for a working GPU path.

Raw entry points take device pointers (ints) -- from the library's own
allocator (``mod_amd.backend.Tensor``) or from any other owner of HBM such as
``torch.Tensor.data_ptr()`` -- and a ``hipStream_t`` (int or None = the
library's current stream).

In a process that also uses torch on the GPU, import torch first: torch's
wheel carries its own HIP and HSA runtimes, and the library's libamdhip64.so.7
then resolves to the one torch loaded. Loaded before torch, the process ends up
with two HIP runtimes, and once torch has initialised the device the library's
runtime reports no device.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

from .build_ops import LIB_PATH

F32, F16, I8, I32 = 0, 1, 2, 3
OK, ERR_INVALID, ERR_HIP, ERR_OOM, ERR_UNSUPPORTED = 0, -1, -2, -3, -4

_DTYPE_CODES = {"float32": F32, "float16": F16, "int8": I8, "int32": I32}


class CTensor(ctypes.Structure):
    """Field-for-field mirror of the reference Tensor struct
    (plugins/common/tensor.h:19-25; backend.py:37-44)."""
    _fields_ = [
        ("data", ctypes.POINTER(ctypes.c_float)),
        ("shape", ctypes.POINTER(ctypes.c_int)),
        ("ndim", ctypes.c_int),
        ("size", ctypes.c_int),
        ("device_id", ctypes.c_int),
    ]


TP = ctypes.POINTER(CTensor)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

# Every symbol declared in include/tensor_rocm.h: name -> (restype, argtypes).
SIGNATURES: dict[str, tuple] = {
    "create_tensor": (TP, [ctypes.POINTER(ctypes.c_int), _i, _i]),
    "create_tensor_typed": (TP, [ctypes.POINTER(ctypes.c_int), _i, _i, _i]),
    "free_tensor": (None, [TP]),
    "tensor_dtype": (_i, [TP]),
    "tensor_fill": (None, [TP, ctypes.c_float]),
    "tensor_load_data": (None, [TP, ctypes.POINTER(ctypes.c_float), _i]),
    "tensor_get_data": (None, [TP, ctypes.POINTER(ctypes.c_float), _i]),
    "tensor_add": (None, [TP, TP, TP]),
    "tensor_mul": (None, [TP, TP, TP]),
    "tensor_load_bytes": (None, [TP, _vp, _sz]),
    "tensor_get_bytes": (None, [TP, _vp, _sz]),
    "tensor_load_bytes_status": (_i, [TP, _vp, _sz]),
    "tensor_get_bytes_status": (_i, [TP, _vp, _sz]),
    "init_memory_pool": (None, [_sz]),
    "reset_memory_pool": (None, []),
    "allocate_pinned_memory": (_vp, [_sz]),
    "free_pinned_memory": (None, [_vp]),
    "tensor_pool_stats": (None, [ctypes.POINTER(ctypes.c_size_t)]),
    "tensor_empty_cache": (None, []),
    "tensor_pool_graph_bytes": (_sz, []),
    "create_stream": (_vp, []),
    "destroy_stream": (None, [_vp]),
    "stream_synchronize": (None, [_vp]),
    "set_current_stream": (None, [_vp]),
    "get_current_stream": (_vp, []),
    "device_synchronize": (None, []),
    "begin_capture": (None, []),
    "end_capture": (None, []),
    "replay_graph": (None, []),
    # companion ops of the reference model layers (model_ops.hip)
    "tensor_rms_norm": (None, [TP, TP, TP, ctypes.c_float]),
    "tensor_rms_norm_status": (_i, [TP, TP, TP, ctypes.c_float]),
    "tensor_fused_add_rms_norm": (None, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_fused_add_rms_norm_status": (_i, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_rope": (None, [TP, TP, TP, TP, TP, TP]),
    "tensor_rope_status": (_i, [TP, TP, TP, TP, TP, TP]),
    "tensor_silu": (None, [TP, TP]),
    "tensor_silu_status": (_i, [TP, TP]),
    "tensor_swiglu": (None, [TP, TP, TP]),
    "tensor_swiglu_status": (_i, [TP, TP, TP]),
    "tensor_fused_gate_up_swiglu": (None, [TP, TP]),
    "tensor_fused_gate_up_swiglu_status": (_i, [TP, TP]),
    "tensor_softmax": (None, [TP, TP]),
    "tensor_softmax_status": (_i, [TP, TP]),
    "tensor_argmax": (None, [TP, TP]),
    "tensor_argmax_status": (_i, [TP, TP]),
    "tensor_embed": (None, [TP, TP, TP]),
    "tensor_embed_status": (_i, [TP, TP, TP]),
    "tensor_scaled_dot_product_attention": (None, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_scaled_dot_product_attention_status": (_i, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_slice": (None, [TP, TP, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "tensor_slice_status": (_i, [TP, TP, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "tensor_set_slice": (None, [TP, TP, ctypes.POINTER(ctypes.c_int)]),
    "tensor_set_slice_status": (_i, [TP, TP, ctypes.POINTER(ctypes.c_int)]),
    "tensor_reshape": (None, [TP, TP]),
    "tensor_reshape_status": (_i, [TP, TP]),
    "tensor_cat": (None, [ctypes.POINTER(TP), _i, _i, TP]),
    "tensor_cat_status": (_i, [ctypes.POINTER(TP), _i, _i, TP]),
    "create_tensor_pinned": (TP, [ctypes.POINTER(ctypes.c_int), _i, _i]),
    "tensor_is_pinned": (_i, [TP]),
    "tensor_copy_async": (_i, [TP, TP, _vp]),
    "create_event": (_vp, []),
    "destroy_event": (None, [_vp]),
    "record_event": (_i, [_vp, _vp]),
    "stream_wait_event": (_i, [_vp, _vp]),
    "event_synchronize": (_i, [_vp]),
    "event_query": (_i, [_vp]),
    "tensor_last_error": (ctypes.c_char_p, []),
    "tensor_clear_error": (None, []),
    "tensor_matmul_int8": (None, [TP, TP, TP]),
    "tensor_matmul_int8_status": (_i, [TP, TP, TP]),
    "tensor_matmul_int8_i32": (None, [TP, TP, TP]),
    "tensor_matmul_int8_i32_status": (_i, [TP, TP, TP]),
    "tensor_dequantize": (None, [TP, TP, TP]),
    "tensor_dequantize_status": (_i, [TP, TP, TP]),
    "tensor_linear_w8": (None, [TP, TP, TP, TP, TP]),
    "tensor_linear_w8_status": (_i, [TP, TP, TP, TP, TP]),
    "tensor_quantize_per_token": (None, [TP, TP, TP]),
    "tensor_quantize_per_token_status": (_i, [TP, TP, TP]),
    "tensor_linear_w8a8": (None, [TP, TP, TP, TP, TP, TP]),
    "tensor_linear_w8a8_status": (_i, [TP, TP, TP, TP, TP, TP]),
    "tensor_moe_w8a8": (None, [TP, TP, TP, TP, TP, TP, _i, _i, TP]),
    "tensor_moe_w8a8_status": (_i, [TP, TP, TP, TP, TP, TP, _i, _i, TP]),
    "pio_gemv_w8": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pio_quantize_per_token": (_i, [_vp, _i, _vp, _vp, _i, _i, _vp]),
    "pio_rmsnorm_quant": (_i, [_vp, _i, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i, _i, _vp]),
    "tensor_rms_norm_quantize": (None, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_rms_norm_quantize_status": (_i, [TP, TP, TP, TP, ctypes.c_float]),
    "tensor_fused_add_rms_norm_quantize": (None, [TP, TP, TP, TP, TP, ctypes.c_float]),
    "tensor_fused_add_rms_norm_quantize_status": (_i, [TP, TP, TP, TP, TP, ctypes.c_float]),
    "pio_gemm_w8a8": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pio_gemm_w8a8_static": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pio_matmul_int8_workspace": (_sz, [_i, _i, _i, _i]),
    "pio_matmul_int8": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "pio_moe_route": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pio_moe_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "pio_moe_w8a8": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                          _vp, _vp]),
    "pio_qwen3_create": (_vp, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "pio_qwen3_destroy": (None, [_vp]),
    "pio_qwen3_reset": (_i, [_vp, _vp, _i]),
    "pio_qwen3_run": (_i, [_vp, _i, _i]),
    "pio_qwen3_persistent_supported": (_i, [_vp]),
    "pio_qwen3_refresh_weights": (_i, [_vp]),
    "pio_qwen3_persistent_replays": (_i, [_vp]),
    "pio_qwen3_prefill": (_i, [_vp, _i, _i]),
    "pio_probe_gemm_supply": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "pio_probe_gemm_timeline": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "pio_qwen3_trace_next": (_i, [_vp, _i]),
    "pio_qwen3_trace_bytes": (_sz, [_vp]),
    "pio_qwen3_trace_read": (_i, [_vp, _vp, _sz]),
    "pio_qwen3_read": (_i, [_vp, _vp, _i, _vp]),
    "pio_qwen3_logits": (_vp, [_vp]),
    "open_safetensors": (_vp, [ctypes.c_char_p]),
    "load_tensor_data": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), _i]),
    "close_safetensors": (None, [_vp]),
    "pio_safetensors_count": (_i, [_vp]),
    "pio_safetensors_name": (ctypes.c_char_p, [_vp, _i]),
    "pio_safetensors_info": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_i),
                                  ctypes.POINTER(ctypes.c_int64), _i, ctypes.POINTER(_i),
                                  ctypes.POINTER(ctypes.c_int64)]),
    "pio_safetensors_read": (_i, [_vp, ctypes.c_char_p, _vp, ctypes.c_int64]),
    "pio_safetensors_to_device": (_i, [_vp, ctypes.c_char_p, _vp, ctypes.c_int64, _vp]),
    "pio_safetensors_to_device_f32": (_i, [_vp, ctypes.c_char_p, _vp, ctypes.c_int64, _vp]),
    "tensor_load_safetensors": (None, [_vp, ctypes.c_char_p, TP]),
    "tensor_load_safetensors_status": (_i, [_vp, ctypes.c_char_p, TP]),
    "pio_version": (ctypes.c_char_p, []),
}


class RocmError(RuntimeError):
    """A libtensor_ops_rocm call returned an error status."""


def _load() -> ctypes.CDLL:
    path = Path(os.environ.get("PIO_ROCM_LIB", LIB_PATH))
    if not path.exists():
        raise ImportError(
            f"{path} is not built: run `python -m mod_amd.build_ops` (hipcc, gfx950). "
            "The ROCm int8 path has no fallback.")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()
LIB_FILE = Path(os.environ.get("PIO_ROCM_LIB", LIB_PATH))


def last_error() -> str:
    return (lib.tensor_last_error() or b"").decode(errors="replace")


def check(status: int, what: str = "") -> None:
    if status != OK:
        raise RocmError(f"{what or 'libtensor_ops_rocm'} failed ({status}): {last_error()}")


def _ptr(x) -> int | None:
    """Device pointer of a torch tensor / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return int(x.data_ptr())
    raise TypeError(f"cannot take a device pointer of {type(x)}")


def _dt(x, default=F32) -> int:
    """Element-type code of a torch tensor (or the default for raw pointers)."""
    if hasattr(x, "dtype"):
        name = str(x.dtype).replace("torch.", "")
        if name in _DTYPE_CODES:
            return _DTYPE_CODES[name]
        raise TypeError(f"unsupported dtype {x.dtype}")
    return default


def _stream(s) -> int | None:
    if s is None:
        return None
    if isinstance(s, int):
        return s
    if hasattr(s, "cuda_stream"):
        return int(s.cuda_stream)
    raise TypeError(f"bad stream {s!r}")


# --------------------------------------------------------------- raw layer
def gemv_w8(x, w, s_w, bias, y, M: int, N: int, K: int, stream=None) -> None:
    """y[M,N] = s_w * (x[M,K] @ w[N,K]^T) + bias."""
    check(lib.pio_gemv_w8(_ptr(x), _dt(x), _ptr(w), _ptr(s_w), _ptr(bias), _ptr(y), _dt(y), M, N,
                          K, _stream(stream)), "pio_gemv_w8")


def quantize_per_token(x, q, s, M: int, K: int, stream=None) -> None:
    check(lib.pio_quantize_per_token(_ptr(x), _dt(x), _ptr(q), _ptr(s), M, K, _stream(stream)),
          "pio_quantize_per_token")


def rmsnorm_quant(x, gamma, q, s, M: int, K: int, eps: float = 1e-6, residual=None,
                  x_sum=None, stream=None) -> None:
    check(lib.pio_rmsnorm_quant(_ptr(x), _dt(x), _ptr(residual), _ptr(x_sum), _ptr(gamma), eps,
                                _ptr(q), _ptr(s), M, K, _stream(stream)), "pio_rmsnorm_quant")


def gemm_w8a8(q, s_a, w, s_w, bias, y, M: int, N: int, K: int, stream=None) -> None:
    check(lib.pio_gemm_w8a8(_ptr(q), _ptr(s_a), _ptr(w), _ptr(s_w), _ptr(bias), _ptr(y), _dt(y),
                            M, N, K, _stream(stream)), "pio_gemm_w8a8")


def matmul_int8(a, b, c, batch: int, M: int, K: int, N: int, out_i32: bool, workspace=None,
                stream=None) -> None:
    check(lib.pio_matmul_int8(_ptr(a), _ptr(b), _ptr(c), int(out_i32), batch, M, K, N,
                              _ptr(workspace), _stream(stream)), "pio_matmul_int8")


def moe_route(logits, topk_w, topk_id, T: int, E: int, k: int, renorm: bool, stream=None) -> None:
    check(lib.pio_moe_route(_ptr(logits), _ptr(topk_w), _ptr(topk_id), T, E, k, int(renorm),
                            _stream(stream)), "pio_moe_route")


def moe_workspace_bytes(T: int, H: int, I: int, E: int, k: int) -> int:
    return int(lib.pio_moe_workspace(T, H, I, E, k))


def moe_w8a8(x, logits, w_gu, s_gu, w_down, s_down, out, T: int, H: int, I: int, E: int, k: int,
             renorm: bool, workspace=None, stream=None) -> None:
    check(lib.pio_moe_w8a8(_ptr(x), _dt(x), _ptr(logits), _ptr(w_gu), _ptr(s_gu), _ptr(w_down),
                           _ptr(s_down), _ptr(out), _dt(out), T, H, I, E, k, int(renorm),
                           _ptr(workspace), _stream(stream)), "pio_moe_w8a8")


def pool_stats() -> dict:
    arr = (ctypes.c_size_t * 7)()
    lib.tensor_pool_stats(arr)
    keys = ["reserved", "in_use", "cached", "peak", "n_malloc", "arena_size", "arena_used"]
    return dict(zip(keys, list(arr)))


def version() -> str:
    return lib.pio_version().decode()
