"""ROCm hardware plugin: the L3 side of the boundary.

``GPUHardwareInterface`` restates the reference ABC field for field
(ip/plugins/base/gpu_interface.py:4-55) so the plugin can be checked here
without the reference package; in the reference tree the plugin subclasses the
original. ``ROCmPlugin`` mirrors the shape of the vendor plugins
(cuda/base.py:9-96, amd/base.py:8-84): it loads its library through
``load_backend_lib``'s path convention (common/utils/lib_loader.py:13-37,
``plugins/rocm/c_src/libtensor_ops_rocm.so``) and exposes allocate / free /
memcpy / synchronize / matmul over the library's Tensor* exports.

``register_rocm_backends`` is what PluginManager.load_hardware_backends
(ip/plugins/manager.py:36-88) does for AMD GPUs instead of mapping them to the
OpenCL plugin (manager.py:70-73): one ROCmPlugin per device under "rocm:{i}".
"""
from __future__ import annotations

import ctypes
import logging
from abc import ABC, abstractmethod
from typing import Any, Dict

import numpy as np

logger = logging.getLogger(__name__)


class GPUHardwareInterface(ABC):
    """Contract of the reference's GPU plugins (gpu_interface.py:4-55)."""

    @abstractmethod
    def initialize(self, **kwargs) -> bool: ...

    @abstractmethod
    def get_device_info(self) -> Dict[str, Any]: ...

    @abstractmethod
    def allocate(self, size_bytes: int) -> Any: ...

    @abstractmethod
    def free(self, ptr: Any) -> None: ...

    @abstractmethod
    def memcpy_h2d(self, dst_ptr: Any, src_data: Any, size_bytes: int) -> None: ...

    @abstractmethod
    def memcpy_d2h(self, dst_data: Any, src_ptr: Any, size_bytes: int) -> None: ...

    @abstractmethod
    def synchronize(self) -> None: ...

    @abstractmethod
    def matmul(self, a_ptr: Any, b_ptr: Any, c_ptr: Any, M: int, N: int, K: int) -> None: ...

    @abstractmethod
    def cleanup(self) -> None: ...


class ROCmPlugin(GPUHardwareInterface):
    """MI355X (gfx950) backend over libtensor_ops_rocm.so.

    Handles are ``Tensor*`` (ops.CTensor pointers) of fp32-sized buffers, the
    same convention as the CUDA/AMD plugins' ``allocate`` (a 1-D tensor of
    ceil(bytes/4) floats on device ``device_id``)."""

    def __init__(self, device_id: int = 0):
        self.device_id = device_id
        self.lib = None
        self._ready = False
        try:
            from . import ops
            self.ops = ops
            self.lib = ops.lib
        except ImportError as e:
            logger.warning("ROCm backend library unavailable: %s", e)

    # -------------------------------------------------------------- setup
    def initialize(self, **kwargs) -> bool:
        """True when the library is loaded and device `device_id` accepts an
        allocation (no GPU -> False, as the reference plugins report)."""
        if self.lib is None:
            return False
        h = self._create(1)
        if not h:
            logger.info("ROCm device %d unavailable: %s", self.device_id, self.ops.last_error())
            self.lib.tensor_clear_error()
            return False
        self.lib.free_tensor(h)
        self._ready = True
        return True

    def get_device_info(self) -> Dict[str, Any]:
        info = {"vendor": "AMD", "backend": "ROCm", "arch": "gfx950", "device": self.device_id}
        if self.lib is not None:
            info["library"] = self.ops.version()
            info["pool"] = self.ops.pool_stats() if self._ready else None
        return info

    # ------------------------------------------------------------- memory
    def _create(self, elements: int):
        shape = (ctypes.c_int * 1)(max(1, elements))
        return self.lib.create_tensor(shape, 1, self.device_id)

    def allocate(self, size_bytes: int):
        if self.lib is None:
            return None
        h = self._create((size_bytes + 3) // 4)
        if not h:
            raise MemoryError(f"ROCm allocate({size_bytes}) failed: {self.ops.last_error()}")
        return h

    def free(self, ptr) -> None:
        if self.lib is not None and ptr:
            self.lib.free_tensor(ptr)

    def memcpy_h2d(self, dst_ptr, src_data, size_bytes: int) -> None:
        arr = np.ascontiguousarray(src_data)
        if arr.nbytes < size_bytes:
            raise ValueError("memcpy_h2d: source smaller than size_bytes")
        self.ops.check(self.lib.tensor_load_bytes_status(dst_ptr, arr.ctypes.data, size_bytes),
                       "memcpy_h2d")

    def memcpy_d2h(self, dst_data, src_ptr, size_bytes: int) -> None:
        arr = dst_data
        if not isinstance(arr, np.ndarray) or not arr.flags["C_CONTIGUOUS"] or arr.nbytes < size_bytes:
            raise ValueError("memcpy_d2h: destination must be a C-contiguous numpy array")
        self.ops.check(self.lib.tensor_get_bytes_status(src_ptr, arr.ctypes.data, size_bytes),
                       "memcpy_d2h")

    def synchronize(self) -> None:
        if self.lib is not None:
            self.lib.stream_synchronize(None)

    # -------------------------------------------------------------- compute
    def matmul(self, a_ptr, b_ptr, c_ptr, M: int, N: int, K: int) -> None:
        """C[M,N] = A[M,K] x B[K,N] for int8 operands with int32 sums cast to
        fp32 (tensor_matmul_int8 semantics, tensor_ops.c:217-246). The fp32
        matmul of the other plugins is not part of the int8 path: a and b are
        int8 Tensor* handles (create_tensor_typed), c an fp32 or int32 one."""
        a, b, c = a_ptr.contents, b_ptr.contents, c_ptr.contents
        got = (a.shape[a.ndim - 2], b.shape[b.ndim - 1], a.shape[a.ndim - 1])
        if a.ndim < 2 or b.ndim < 2 or c.ndim < 2 or got != (M, N, K):
            raise ValueError(f"matmul: tensors hold (M,N,K)={got}, caller passed {(M, N, K)}")
        fn = (self.lib.tensor_matmul_int8_i32_status
              if self.lib.tensor_dtype(c_ptr) == self.ops.I32 else self.lib.tensor_matmul_int8_status)
        self.ops.check(fn(a_ptr, b_ptr, c_ptr), "matmul")

    def cleanup(self) -> None:
        if self.lib is not None and self._ready:
            self.lib.stream_synchronize(None)
            self.lib.tensor_empty_cache()


def register_rocm_backends(active_backends: Dict[str, Any], n_devices: int = 1) -> int:
    """Adds an initialized ROCmPlugin per device under "rocm:{i}"; returns how
    many were registered."""
    n = 0
    for i in range(n_devices):
        p = ROCmPlugin(i)
        if p.initialize():
            active_backends[f"rocm:{i}"] = p
            n += 1
    return n
