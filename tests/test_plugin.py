"""ROCm plugin (GPUHardwareInterface) and UnifiedMemoryManager hook.

CPU tests check the interface contract and the no-GPU behaviour the reference
plugins have (initialize() -> False, manager.py:36-88 then skips the device);
GPU tests drive allocate/memcpy/matmul and evict/restore through the library.
"""
import ctypes
import inspect

import numpy as np
import pytest


def test_plugin_implements_every_interface_method():
    from mod_amd.plugin import GPUHardwareInterface, ROCmPlugin
    abstract = {n for n, f in inspect.getmembers(GPUHardwareInterface)
                if getattr(f, "__isabstractmethod__", False)}
    assert abstract == {"initialize", "get_device_info", "allocate", "free", "memcpy_h2d",
                        "memcpy_d2h", "synchronize", "matmul", "cleanup"}
    p = ROCmPlugin(0)        # instantiable: every abstract method is implemented
    assert isinstance(p, GPUHardwareInterface)
    info = p.get_device_info()
    assert info["vendor"] == "AMD" and info["arch"] == "gfx950"


def test_plugin_without_gpu_reports_unavailable(monkeypatch):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from mod_amd import ops
    from mod_amd.plugin import ROCmPlugin, register_rocm_backends
    p = ROCmPlugin(0)
    assert p.initialize() is False
    active = {}
    assert register_rocm_backends(active, 1) == 0 and active == {}
    ops.lib.tensor_clear_error()


def _typed(lib, shape, dtype):
    c = (ctypes.c_int * len(shape))(*shape)
    h = lib.create_tensor_typed(c, len(shape), 0, dtype)
    assert h
    return h


@pytest.mark.gpu
def test_plugin_matmul_and_memcpy_on_gpu():
    from mod_amd import ops
    from mod_amd.plugin import ROCmPlugin, register_rocm_backends
    active = {}
    assert register_rocm_backends(active, 1) == 1
    p = active["rocm:0"]
    M, K, N = 37, 80, 53
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    b = rng.integers(-128, 128, (K, N), dtype=np.int8)
    ha, hb = _typed(p.lib, (M, K), ops.I8), _typed(p.lib, (K, N), ops.I8)
    hc, hi = _typed(p.lib, (M, N), ops.F32), _typed(p.lib, (M, N), ops.I32)
    try:
        p.memcpy_h2d(ha, a, a.nbytes)
        p.memcpy_h2d(hb, b, b.nbytes)
        p.matmul(ha, hb, hc, M, N, K)
        p.matmul(ha, hb, hi, M, N, K)
        p.synchronize()
        want = a.astype(np.int32) @ b.astype(np.int32)
        out_f = np.empty((M, N), np.float32)
        out_i = np.empty((M, N), np.int32)
        p.memcpy_d2h(out_f, hc, out_f.nbytes)
        p.memcpy_d2h(out_i, hi, out_i.nbytes)
        assert np.array_equal(out_i, want)
        assert np.array_equal(out_f, want.astype(np.float32))
        with pytest.raises(ValueError):
            p.matmul(ha, hb, hc, M, N, K + 1)
        # allocate() follows the reference plugins: ceil(bytes/4) fp32 elements.
        h = p.allocate(10)
        assert h.contents.size == 3 and h.contents.device_id == 0
        p.free(h)
    finally:
        for h in (ha, hb, hc, hi):
            p.free(h)
        p.cleanup()


@pytest.mark.gpu
def test_unified_manager_evicts_lru_and_restores_bytes():
    from mod_amd.backend import Tensor
    from mod_amd.unified_manager import UnifiedMemoryManager
    mm = UnifiedMemoryManager(gpu_limit_mb=1)
    rng = np.random.default_rng(9)
    data = [rng.standard_normal((256, 256)).astype(np.float32) for _ in range(3)]   # 256 KiB each
    ts = [Tensor((256, 256), data=d, device="rocm:0") for d in data]
    for t in ts:
        mm.register(t)
    assert mm.current_gpu_bytes == 3 * 256 * 1024 and not mm.evicted
    mm.access(ts[0])                       # ts[1] becomes least recently used
    big = Tensor((512, 256), device="rocm:0")   # 512 KiB pushes the total over 1 MiB
    mm.register(big)
    assert set(mm.evicted) == {id(ts[1])} and ts[1]._handle is None
    assert mm.current_gpu_bytes == 2 * 256 * 1024 + 512 * 1024
    mm.access(ts[1])                       # restore evicts the next LRU (ts[2])
    assert id(ts[1]) in mm.tensors and id(ts[2]) in mm.evicted
    assert ts[1].shape == (256, 256)
    np.testing.assert_array_equal(ts[1].numpy(), data[1])
    mm.access(ts[2])                       # evicts ts[0]
    np.testing.assert_array_equal(ts[2].numpy(), data[2])
    assert id(ts[0]) in mm.evicted
    mm.access(ts[0])                       # evicts big
    assert id(big) in mm.evicted
    np.testing.assert_array_equal(ts[0].numpy(), data[0])
    assert mm.stats()["registered"] == len(mm.tensors)


@pytest.mark.gpu
def test_allocator_reuses_a_block_only_on_its_stream():
    """A freed block goes back to the cache tagged with the stream it was
    allocated for and is handed out again only for that stream, so work still
    queued on the old stream can never see its memory taken by another
    stream. Checked through the public pool statistics (stats[4] counts
    hipMalloc calls): same stream -> reuse, other stream -> a new block."""
    from mod_amd import ops
    from mod_amd.backend import Tensor
    lib = ops.lib
    stats = (ctypes.c_size_t * 7)()

    def mallocs():
        lib.tensor_pool_stats(stats)
        return stats[4]

    sa, sb = lib.create_stream(), lib.create_stream()
    try:
        shape = [3, 1000, 77]            # an odd size no other test allocates
        lib.set_current_stream(sa)
        t = Tensor(shape)
        del t                            # cached for stream A
        n0 = mallocs()
        t = Tensor(shape)                # same stream: the cached block
        assert mallocs() == n0
        del t
        lib.set_current_stream(sb)
        t = Tensor(shape)                # other stream: never the block cached for A
        assert mallocs() == n0 + 1
        del t
        lib.set_current_stream(sa)
        t = Tensor(shape)
        assert mallocs() == n0 + 1       # A's block again
        del t
    finally:
        lib.set_current_stream(None)
        lib.device_synchronize()
        lib.destroy_stream(sa)
        lib.destroy_stream(sb)
