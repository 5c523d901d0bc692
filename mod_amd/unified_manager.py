"""UnifiedMemoryManager with ROCm devices (allocator hook).

The reference manager (ip/common/memory/unified_manager.py:5-59) tracks GPU
tensors only when the device string contains "cuda" and gets pinned memory from
a CUDA export that no library provides. This version keeps the same methods and
LRU bookkeeping, recognises "rocm:N" devices, takes pinned host memory from
libtensor_ops_rocm (hipHostMalloc) and reads real occupancy from the library's
caching allocator / arena (tensor_pool_stats). Eviction moves the least
recently used registered tensors' bytes into pinned host buffers and frees their
device memory; ``restore`` brings a tensor back.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Dict

from . import ops
from .backend import Tensor


class UnifiedMemoryManager:
    def __init__(self, gpu_limit_mb: int = 4096):
        self.gpu_limit_bytes = gpu_limit_mb * 1024 * 1024
        self.current_gpu_bytes = 0
        self.tensors: "OrderedDict[int, Tensor]" = OrderedDict()   # id -> tensor, LRU order
        self.evicted: Dict[int, tuple] = {}   # id -> (tensor, shape, pinned, nbytes)

    # ------------------------------------------------------------ pinned
    def malloc_pinned(self, size_bytes: int):
        """Pinned host memory (unified_manager.py:16-24)."""
        p = ops.lib.allocate_pinned_memory(size_bytes)
        if not p:
            raise MemoryError(f"allocate_pinned_memory({size_bytes}) failed: {ops.last_error()}")
        return p

    def free_pinned(self, ptr) -> None:
        ops.lib.free_pinned_memory(ptr)

    # ----------------------------------------------------------- tracking
    @staticmethod
    def _on_gpu(t: Tensor) -> bool:
        return t.device.startswith("rocm") or "cuda" in t.device

    def register(self, tensor: Tensor) -> None:
        if self._on_gpu(tensor) and id(tensor) not in self.tensors:
            self.tensors[id(tensor)] = tensor
            self.current_gpu_bytes += tensor.nbytes
            self.enforce_limit()

    def access(self, tensor: Tensor) -> None:
        if id(tensor) in self.evicted:
            self.restore(tensor)
        if id(tensor) in self.tensors:
            self.tensors.move_to_end(id(tensor))

    def enforce_limit(self) -> None:
        while self.current_gpu_bytes > self.gpu_limit_bytes and self.tensors:
            _, t = next(iter(self.tensors.items()))
            self.evict(t)

    # ------------------------------------------------------ evict/restore
    def evict(self, tensor: Tensor) -> None:
        """Copies the tensor's bytes into pinned host memory and releases its
        device buffer (the Tensor keeps its shape and dtype)."""
        key = id(tensor)
        if key not in self.tensors:
            return
        n = tensor.nbytes
        shape = tensor.shape
        pinned = self.malloc_pinned(max(n, 1))
        ops.check(ops.lib.tensor_get_bytes_status(tensor._handle, pinned, n), "evict")
        ops.lib.free_tensor(tensor._handle)
        tensor._handle = None
        del self.tensors[key]
        self.current_gpu_bytes -= n
        self.evicted[key] = (tensor, shape, pinned, n)

    def restore(self, tensor: Tensor) -> None:
        key = id(tensor)
        if key not in self.evicted:
            return
        t, shape, pinned, n = self.evicted.pop(key)
        fresh = Tensor(shape, device=t.device, dtype=t.dtype)
        ops.check(ops.lib.tensor_load_bytes_status(fresh._handle, pinned, n), "restore")
        t._handle, fresh._handle = fresh._handle, None
        self.free_pinned(pinned)
        self.tensors[key] = t
        self.current_gpu_bytes += n
        self.enforce_limit()

    def stats(self) -> dict:
        s = ops.pool_stats()
        s.update(registered_bytes=self.current_gpu_bytes, registered=len(self.tensors),
                 evicted=len(self.evicted))
        return s
