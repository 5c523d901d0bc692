"""HybridScheduler for ``rocm:N`` devices: layer residency between pinned
host memory and HBM, with prefetch on a transfer stream.

The reference scheduler (ip/common/managers/hybrid_scheduler.py:10-177) places
layers on the GPU or the CPU (device_for_layer, :25-40), moves the current
layer to the GPU before it runs, prefetches the next two layers on a transfer
stream and evicts the layer two back (check_migration_policy, :42-97), and
runs a model whose layers sit on different devices layer by layer
(execute_hybrid / is_model_split / _run_split_execution, :99-177). It reads a
``hardware_backend`` attribute PluginManager does not have (:17) and
synchronizes the whole transfer stream before each layer (:51-53).

This library has no CPU compute path, so "placed on the CPU" means here:
the layer's weights live in pinned host memory (their home copy) and are
streamed into HBM before the layer runs; every layer computes on the GPU.
The same methods, with these mechanics:

* ``plan(model)`` fills HBM (the ``gpu_budget_bytes`` given) with whole layers up to
  ``gpu_memory_fraction`` of the budget, keeping room for the prefetch window;
  the other layers move to pinned host memory. ``device_for_layer`` reports
  the plan.
* ``check_migration_policy`` makes the compute stream wait on the event of the
  layer's prefetch (or fetches it first if it was not prefetched), evicts the
  offloaded layer two back and queues the next ``prefetch_window`` offloaded
  layers on the transfer stream (device memory allocated on that stream, one
  event per layer). Weights are read-only, so
  eviction copies nothing: the layer's parameters return to their pinned home
  copies and the device buffers are released after the transfer stream has
  been ordered behind the compute stream's use of them (an event), so the
  allocator never hands them to the next prefetch while a kernel still reads
  them.
* ``execute_hybrid`` runs a model whose layers sit on different devices layer
  by layer on the compute stream, else calls the model directly.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence

from . import ops
from .backend import HIPEvent, HIPStream, Module, Tensor


def plan_placement(layer_bytes: Sequence[int], gpu_budget_bytes: Optional[int],
                   gpu_memory_fraction: float = 0.8, prefetch_window: int = 2,
                   device: str = "rocm:0") -> List[str]:
    """Per layer "rocm:N" (resident) or "cpu" (pinned host, streamed in).
    Layers stay resident in order while their bytes fit in fraction * budget;
    when any layer is offloaded, the bytes of the largest `prefetch_window + 2`
    offloaded layers are reserved first (the previous layer, the one running
    and the window in flight are on the device together). No budget:
    everything resident."""
    n = len(layer_bytes)
    if gpu_budget_bytes is None:
        return [device] * n
    cap = int(gpu_budget_bytes * gpu_memory_fraction)
    if sum(layer_bytes) <= cap:
        return [device] * n
    place = ["cpu"] * n
    # reserve the streaming window out of the budget, then fill greedily
    for resident in range(n, -1, -1):
        off = sorted(layer_bytes[resident:], reverse=True)[:prefetch_window + 2]
        if sum(layer_bytes[:resident]) + sum(off) <= cap:
            for i in range(resident):
                place[i] = device
            return place
    raise ValueError(f"a GPU budget of {gpu_budget_bytes} B cannot hold the streaming window "
                     f"({prefetch_window + 2} layers)")


def _gpu_present(device: str) -> bool:
    try:
        from .plugin import ROCmPlugin
        ok = ROCmPlugin(int(device.split(":")[1]) if ":" in device else 0).initialize()
    finally:
        ops.lib.tensor_clear_error()
    return bool(ok)


class HybridScheduler:
    """Same methods as the reference HybridScheduler; see the module docstring."""

    def __init__(self, device: str = "rocm:0", gpu_budget_bytes: Optional[int] = None,
                 prefetch_window: int = 2, has_gpu: Optional[bool] = None):
        self.device = device
        self.gpu_budget_bytes = gpu_budget_bytes
        self.prefetch_window = prefetch_window
        self.has_gpu = _gpu_present(device) if has_gpu is None else has_gpu
        self.compute_stream = HIPStream() if self.has_gpu else None
        self.transfer_stream = HIPStream() if self.has_gpu else None
        self._placement: List[str] = []
        self._home: Dict[int, Dict[str, Tensor]] = {}   # id(layer) -> pinned host params
        self._pending: Dict[int, HIPEvent] = {}          # id(layer) -> prefetch-done event
        self.stats = {"prefetched": 0, "evicted": 0, "blocking_loads": 0,
                      "max_offloaded_on_device": 0}

    # --------------------------------------------------------------- placement
    def plan(self, model, gpu_memory_fraction: float = 0.8) -> List[str]:
        """Places model.layers by the budget and moves each layer to its place
        (offloaded layers to pinned host memory, their home copies)."""
        self._need_gpu()
        layers = model.layers
        sizes = [sum(p.nbytes for p in L.parameters()) for L in layers]
        self._placement = plan_placement(sizes, self.gpu_budget_bytes, gpu_memory_fraction,
                                         self.prefetch_window, self.device)
        for L, where in zip(layers, self._placement):
            if where == "cpu":
                L.to("cpu", stream=self.transfer_stream)
                self._home[id(L)] = dict(L.named_parameters())
            else:
                L.to(self.device, stream=self.transfer_stream)
        self.transfer_stream.synchronize()
        return list(self._placement)

    def device_for_layer(self, layer_idx: int, total_layers: int,
                         gpu_memory_fraction: float = 0.8) -> str:
        """hybrid_scheduler.py:25-40: where the layer lives ("cpu" = pinned
        host memory, streamed to the GPU to run)."""
        if not self.has_gpu:
            return "cpu"
        if self._placement and len(self._placement) == total_layers:
            return self._placement[layer_idx]
        return self.device

    # --------------------------------------------------------------- migration
    @staticmethod
    def _on_host(layer: Module) -> bool:
        for p in layer.parameters():
            return p.device == "cpu"
        return False

    def _need_gpu(self) -> None:
        if not self.has_gpu:
            raise ops.RocmError("HybridScheduler: no ROCm device (this library has no CPU path)")

    def _fetch(self, layer: Module) -> HIPEvent:
        """Queues the layer's weights to HBM on the transfer stream; device
        memory is allocated for that stream, so only transfer-stream work can
        reuse it once freed."""
        with self.transfer_stream:
            layer.to(self.device, non_blocking=True, stream=self.transfer_stream)
            return self.transfer_stream.record_event()

    def check_migration_policy(self, layer_idx: int, layer: Module, all_layers=None) -> None:
        """hybrid_scheduler.py:42-97, on events instead of stream-wide syncs."""
        self._need_gpu()
        # 1. the current layer on the GPU
        ev = self._pending.pop(id(layer), None)
        if ev is not None:
            self.compute_stream.wait_event(ev)
        elif self._on_host(layer):
            self.compute_stream.wait_event(self._fetch(layer))
            self.stats["blocking_loads"] += 1
        if not all_layers:
            return
        # 2. evict the offloaded layer two back: the transfer stream is ordered
        # behind the compute work queued so far (which includes that layer's),
        # then the parameters return to their pinned home copies, so its
        # device memory can serve the prefetches below
        if layer_idx >= 2:
            old = all_layers[layer_idx - 2]
            home = self._home.get(id(old))
            if home is not None and not self._on_host(old):
                self._evict([old])
        # 3. prefetch the next offloaded layers
        for off in range(1, self.prefetch_window + 1):
            j = layer_idx + off
            if j < len(all_layers):
                nxt = all_layers[j]
                if id(nxt) not in self._pending and self._on_host(nxt):
                    self._pending[id(nxt)] = self._fetch(nxt)
                    self.stats["prefetched"] += 1
        on_dev = sum(1 for L in all_layers if id(L) in self._home and not self._on_host(L))
        self.stats["max_offloaded_on_device"] = max(self.stats["max_offloaded_on_device"], on_dev)

    def _evict(self, layers) -> None:
        """Offloaded layers back to their pinned home copies, once the transfer
        stream is ordered behind the compute work queued so far."""
        self.transfer_stream.wait_event(self.compute_stream.record_event())
        for L in layers:
            for name, t in self._home[id(L)].items():
                L._set_parameter(name, t)
            self.stats["evicted"] += 1

    # --------------------------------------------------------------- execution
    def is_model_split(self, model) -> bool:
        """hybrid_scheduler.py:119-132: layers on different devices."""
        devs = {p.device for L in getattr(model, "layers", []) for p in list(L.parameters())[:1]}
        return len(devs) > 1

    def execute_hybrid(self, model: Any, input_ids: Tensor) -> Tensor:
        """hybrid_scheduler.py:99-117."""
        self._need_gpu()
        if self.is_model_split(model):
            return self._run_split_execution(model, input_ids)
        self.compute_stream.wait_event(HIPEvent.on_current_stream())
        with self.compute_stream:
            out = model(input_ids)
        self.compute_stream.synchronize()
        return out

    def _run_split_execution(self, model, x: Tensor) -> Tensor:
        """hybrid_scheduler.py:134-177: layer by layer on the compute stream,
        each after its migration policy; the optional embed_tokens / norm /
        lm_head stages run around the layers as in the reference."""
        layers = model.layers
        # the input may come from work on the caller's stream
        self.compute_stream.wait_event(HIPEvent.on_current_stream())
        with self.compute_stream:
            if hasattr(model, "embed_tokens"):
                x = model.embed_tokens(x)
            for i, layer in enumerate(layers):
                self.check_migration_policy(i, layer, layers)
                x = layer(x)
            if hasattr(model, "norm"):
                x = model.norm(x)
            if hasattr(model, "lm_head"):
                x = model.lm_head(x)
            # offloaded layers still on the device (the last two) go home, so
            # the next pass starts from the plan
            rest = [L for L in layers if id(L) in self._home and not self._on_host(L)]
            if rest:
                self._evict(rest)
        self.compute_stream.synchronize()
        return x
