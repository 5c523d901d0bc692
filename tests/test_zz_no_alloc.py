"""The allocation-free W8A8 entry point (pio_gemm_w8a8_static), through the
C ABI: on shapes whose plan keeps int32 K-slice partials (the skinny kernel in
K slices, the tile engine's split-K), its output equals pio_gemm_w8a8's bit
for bit, on two calls in a row (the second smaller, reusing the same scratch),
for int32, fp32 and fp16 outputs; the library's allocator sees no allocation
during the calls; a shape needing more than the 16 MiB scratch is refused
with an error."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (M, N, K): skinny W8A8 with 6 K slices (6.3 MB of partials), then smaller
# ones: skinny with 4 slices (1 MiB) and the tile engine's split-K plan
SHAPES = [(64, 4096, 12288), (16, 4096, 12288), (200, 1024, 4096)]


def _say(m):
    print(m, flush=True)


def _run(fn, torch, ops, q, sa, w, sw, b, y, M, N, K, dt):
    st = torch.cuda.current_stream().cuda_stream
    rc = fn(q.data_ptr(), sa.data_ptr(), w.data_ptr(), sw.data_ptr(),
            None if b is None else b.data_ptr(), y.data_ptr(), dt, M, N, K, st)
    ops.check(rc, fn.__name__)


def test_static_entry_matches_allocating_entry(torch_dev):
    import torch
    from mod_amd import ops
    lib = ops.lib
    d = torch_dev
    cases = []
    for i, (M, N, K) in enumerate(SHAPES):
        rng = np.random.default_rng(100 + i)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(d)  # noqa: E731
        cases.append((M, N, K,
                      t(rng.integers(-127, 128, size=(M, K), dtype=np.int8)),
                      t(rng.uniform(0.001, 0.05, size=M).astype(np.float32)),
                      t(rng.integers(-127, 128, size=(N, K), dtype=np.int8)),
                      t(rng.uniform(0.001, 0.02, size=N).astype(np.float32)),
                      t(rng.standard_normal(N).astype(np.float32))))
    outs = {ops.I32: torch.int32, ops.F32: torch.float32, ops.F16: torch.float16}
    # warm both entry points once (kernel attributes, scratch address lookup)
    M, N, K, q, sa, w, sw, b = cases[0]
    y = torch.empty((M, N), dtype=torch.float32, device=d)
    _run(lib.pio_gemm_w8a8_static, torch, ops, q, sa, w, sw, b, y, M, N, K, ops.F32)
    torch.cuda.synchronize()
    for dt, tdt in outs.items():
        for (M, N, K, q, sa, w, sw, b) in cases:     # largest first, then smaller
            _say(f"static vs allocating: M={M} N={N} K={K} out={tdt}")
            ref = torch.full((M, N), 7, dtype=tdt, device=d)
            got = torch.full((M, N), 3, dtype=tdt, device=d)
            bias = None if dt == ops.I32 else b
            _run(lib.pio_gemm_w8a8, torch, ops, q, sa, w, sw, bias, ref, M, N, K, dt)
            torch.cuda.synchronize()
            before = ops.pool_stats()
            _run(lib.pio_gemm_w8a8_static, torch, ops, q, sa, w, sw, bias, got, M, N, K, dt)
            torch.cuda.synchronize()
            after = ops.pool_stats()
            assert after["n_malloc"] == before["n_malloc"], (before, after)
            assert after["in_use"] == before["in_use"] and after["cached"] == before["cached"]
            assert torch.equal(got.view(torch.uint8) if dt != ops.I32 else got,
                               ref.view(torch.uint8) if dt != ops.I32 else ref), (M, N, K, dt)


def test_static_entry_refuses_shapes_beyond_its_scratch(torch_dev):
    """M = 64, K = 65536 plans 16 K slices (256 blocks of 256 B each, the most
    a slice count may be); with N = 6144 that is 16 x 64 x 6144 x 4 B =
    24 MiB of partials, above the 16 MiB array."""
    import torch
    from mod_amd import ops
    d = torch_dev
    M, N, K = 64, 6144, 65536
    q = torch.zeros((M, K), dtype=torch.int8, device=d)
    w = torch.zeros((N, K), dtype=torch.int8, device=d)
    s = torch.ones((max(M, N),), dtype=torch.float32, device=d)
    y = torch.empty((M, N), dtype=torch.int32, device=d)
    rc = ops.lib.pio_gemm_w8a8_static(q.data_ptr(), s.data_ptr(), w.data_ptr(), s.data_ptr(),
                                      None, y.data_ptr(), ops.I32, M, N, K,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == ops.ERR_INVALID
    assert "static scratch" in ops.last_error()
