"""HybridScheduler (reference: ip/common/managers/hybrid_scheduler.py:10-177)
on rocm devices: layers that do not fit the HBM budget live in pinned host
memory and are streamed to the GPU on a transfer stream ahead of use; every
layer computes on the GPU.

CPU tests: the placement rule and the no-GPU behaviour (device_for_layer says
"cpu" as the reference does without a GPU, and running raises: the library has
no CPU path). GPU test: an 8-layer W8Linear stack with 3 layers resident gives
bit-identical outputs to the same stack fully resident, over two passes, with
every offloaded layer prefetched (never loaded on demand) and at most
prefetch_window + 2 offloaded layers on the device at once."""
import numpy as np
import pytest

# mod_amd is imported inside the tests: in a process that also uses torch on
# the GPU, torch has to initialise the device before the library is loaded.


def test_plan_placement_fills_budget_in_order_and_reserves_the_window():
    from mod_amd.hybrid_scheduler import plan_placement
    b = [10] * 8
    assert plan_placement(b, None) == ["rocm:0"] * 8
    assert plan_placement(b, 100, 0.8) == ["rocm:0"] * 8            # 80 <= 80
    # cap 72: r resident + 4 streamed (window 2 + current + previous) <= 72
    assert plan_placement(b, 90, 0.8, 2) == ["rocm:0"] * 3 + ["cpu"] * 5
    assert plan_placement(b, 90, 0.8, 1) == ["rocm:0"] * 4 + ["cpu"] * 4
    # uneven layers: the reserve is the largest offloaded ones
    assert plan_placement([5, 5, 30, 5, 5, 5], 100, 0.5, 1) == ["rocm:0"] * 2 + ["cpu"] * 4
    with pytest.raises(ValueError, match="streaming window"):
        plan_placement(b, 30, 1.0, 2)


def test_scheduler_without_gpu_places_on_cpu_and_refuses_to_run():
    from mod_amd import ops
    from mod_amd.hybrid_scheduler import HybridScheduler
    s = HybridScheduler(has_gpu=False)
    assert s.device_for_layer(0, 4) == "cpu"
    with pytest.raises(ops.RocmError, match="no CPU path"):
        s.execute_hybrid(None, None)
    with pytest.raises(ops.RocmError, match="no CPU path"):
        s.check_migration_policy(0, None)


class _Stack:
    def __init__(self, layers):
        self.layers = layers

    def __call__(self, x):
        for L in self.layers:
            x = L(x)
        return x


@pytest.mark.gpu
def test_hybrid_execution_matches_resident_stack(torch_dev):
    from mod_amd.backend import Tensor, W8Linear
    from mod_amd.hybrid_scheduler import HybridScheduler
    K, n_layers, M = 1024, 8, 4
    rng = np.random.default_rng(3)
    qs = [rng.integers(-127, 127, size=(K, K), dtype=np.int8) for _ in range(n_layers)]
    ss = [(rng.uniform(0.5, 1.5, K) / K ** 0.5 / 30).astype(np.float32) for _ in range(n_layers)]
    bs = [rng.standard_normal(K).astype(np.float32) * 0.1 for _ in range(n_layers)]

    def stack():
        layers = []
        for q, s, b in zip(qs, ss, bs):
            L = W8Linear(K, K, bias=True)
            L.load_quantized(q, s, b)
            layers.append(L)
        return _Stack(layers)

    x = rng.standard_normal((M, K)).astype(np.float32)
    want = stack()(Tensor.from_numpy(x)).numpy()

    model = stack()
    layer_bytes = K * K + 8 * K
    sched = HybridScheduler(gpu_budget_bytes=int(7.5 * layer_bytes / 0.8), prefetch_window=2)
    place = sched.plan(model)
    assert place == ["rocm:0"] * 3 + ["cpu"] * 5
    assert [sched.device_for_layer(i, n_layers) for i in range(n_layers)] == place
    assert sched.is_model_split(model)
    for p in model.layers[5].parameters():
        assert p.device == "cpu"
        from mod_amd import ops
        assert ops.lib.tensor_is_pinned(p._handle) == 1
    for rep in range(2):
        got = sched.execute_hybrid(model, Tensor.from_numpy(x)).numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        assert sched.stats["prefetched"] == 5 * (rep + 1)
        assert sched.stats["evicted"] == 5 * (rep + 1)
        assert sched.stats["blocking_loads"] == 0
        assert all(p.device == ("cpu" if i >= 3 else "rocm:0")
                   for i, L in enumerate(model.layers) for p in L.parameters())
    assert sched.stats["max_offloaded_on_device"] <= 4


@pytest.mark.gpu
def test_to_on_a_side_stream_is_ordered_after_the_current_stream(torch_dev):
    """Tensor.to(..., stream=s) with s not the current stream: the copy waits
    for the work queued on the current stream that writes the source (here a
    chain of 64 MB fills, the last one with the expected value), to a pinned
    host tensor both blocking and non-blocking, and from there back to the
    device on the side stream."""
    from mod_amd.backend import HIPStream, Tensor
    n = 16 << 20
    x = Tensor((n,), device="rocm:0", dtype="float32")
    s = HIPStream()
    for rep in range(3):
        for v in range(1, 9):
            x.fill(float(v + 10 * rep))          # queued on the current stream
        h = x.to("cpu", stream=s)
        assert np.all(h.numpy() == float(8 + 10 * rep))
        for v in range(1, 5):
            x.fill(float(v + 100 * rep))
        z = x.to("cpu", non_blocking=True, stream=s)
        s.synchronize()
        assert np.all(z.numpy() == float(4 + 100 * rep))
        # back to the device on the side stream: the destination block is
        # allocated for that stream
        d = z.to("rocm:0", non_blocking=True, stream=s)
        s.synchronize()
        assert np.all(d.numpy() == float(4 + 100 * rep))
