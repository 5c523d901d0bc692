"""GPU parity of the Tensor* drop-in layer (the entry points reference model
code would call through ctypes, backend.py:37-160), on tensors made by
create_tensor_typed, against the oracle:

* tensor_dequantize, per-tensor (tensor_ops_cuda.cu:923-929: out = q * scale[0])
  and per-row scales;
* tensor_quantize_per_token, fp32 and fp16 inputs, bit-exact;
* tensor_rms_norm_quantize / tensor_fused_add_rms_norm_quantize (the fused
  RMSNorm -> quantizer producer), bit-exact, feeding W8A8Linear;
* tensor_linear_w8a8, int32 / fp32 / fp16 outputs with and without bias, on the
  one-pass, split-K and skinny paths;
* tensor_moe_w8a8 (the routed expert layer);
* the allocator around graph capture (begin_capture / end_capture /
  replay_graph, backend.py:801-810): a workspace an op frees while its stream
  captures stays with the graph, so a tensor allocated afterwards cannot alias
  it; destroy_stream releases what is cached for the stream;
* the arena (init_memory_pool / reset_memory_pool, tensor_ops.c:74-93) and a
  clean process exit after the persistent decoder, in a child process (the
  arena changes where every later tensor of a process lives).
"""
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.conftest import assert_rel

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]


def _say(m):
    print(m, flush=True)


@pytest.fixture(scope="module")
def T(torch_dev):
    from mod_amd import backend
    return backend


def _t(B, a):
    return B.Tensor.from_numpy(np.ascontiguousarray(a))


# --------------------------------------------------------------- dequantize
@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 33), (3072, 1024)])
def test_tensor_dequantize_matches_reference_semantics(T, rows, cols):
    _say(f"dequantize rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols)
    q = rng.integers(-128, 128, size=(rows, cols), dtype=np.int8)
    q.flat[0] = -128
    s1 = np.array([0.0123], np.float32)
    sr = rng.uniform(0.001, 0.02, size=rows).astype(np.float32)
    tq = _t(T, q)
    got1 = tq.dequantize(_t(T, s1)).numpy()
    # one fp32 product per element, exactly as the reference kernel
    assert np.array_equal(got1.view(np.uint32), (q.astype(np.float32) * s1[0]).view(np.uint32))
    gotr = tq.dequantize(_t(T, sr)).numpy()
    assert np.array_equal(gotr.view(np.uint32),
                          (q.astype(np.float32) * sr[:, None]).view(np.uint32))
    if rows > 1:
        with pytest.raises(Exception, match="scale has"):
            tq.dequantize(_t(T, np.ones(rows + 1, np.float32)))


# ------------------------------------------------------- per-token quantizer
@pytest.mark.parametrize("M,K,dt", [(1, 1024, np.float32), (5, 48, np.float16),
                                    (2048, 1024, np.float16), (64, 12288, np.float32)])
def test_tensor_quantize_per_token_bit_exact(T, M, K, dt):
    _say(f"tensor_quantize_per_token M={M} K={K} {np.dtype(dt).name}")
    rng = np.random.default_rng(M * 7 + K)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(dt)
    x[0, :] = 0                       # zero row: s = 1, q = 0
    q, s = _t(T, x).quantize_per_token()
    qr, sr = oracle.quant_per_token(x)
    assert np.array_equal(q.numpy(), qr)
    assert np.array_equal(s.numpy().view(np.uint32), sr.view(np.uint32))


# ------------------------------------------- RMSNorm -> quantizer producer
@pytest.mark.parametrize("M,K,dt", [(2048, 1024, np.float16), (3, 3072, np.float32)])
def test_tensor_rms_norm_quantize_feeds_w8a8(T, M, K, dt):
    """tensor_rms_norm_quantize and tensor_fused_add_rms_norm_quantize through
    Tensor handles (bit-exact q, s, and the in-place sum), then the W8A8Linear
    on the fused producer's output equals the linear on the oracle's q, s."""
    _say(f"tensor_rms_norm_quantize M={M} K={K} {np.dtype(dt).name}")
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K), dtype=np.float32) * 3).astype(dt)
    r = rng.standard_normal((M, K), dtype=np.float32).astype(dt)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    tx, tg = _t(T, x), _t(T, g)
    q, s = tx.rms_norm_quantize(tg, 1e-6)
    qr, sr, _, _ = oracle.rmsnorm_quant(x, g, 1e-6)
    assert np.array_equal(q.numpy(), qr)
    assert np.array_equal(s.numpy().view(np.uint32), sr.view(np.uint32))
    q2, s2 = tx.fused_add_rms_norm_quantize(_t(T, r), tg, 1e-6)
    qr2, sr2, _, xs = oracle.rmsnorm_quant(x, g, 1e-6, residual=r)
    assert np.array_equal(tx.numpy().view(np.uint8), xs.view(np.uint8))   # x updated in place
    assert np.array_equal(q2.numpy(), qr2)
    assert np.array_equal(s2.numpy().view(np.uint32), sr2.view(np.uint32))
    N = 256
    lin = T.W8A8Linear(K, N, bias=False, out_dtype="float16")
    W = rng.integers(-127, 127, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    lin.load_quantized(W, sw)
    got = lin.forward_quantized(q, s).numpy()
    assert np.array_equal(got.view(np.uint16), oracle.w8a8(qr, sr, W, sw, None, out="f16").view(np.uint16))


# ----------------------------------------------------------------- W8A8 GEMM
# (M, N, K): one-pass tiles; the skinny kernel in K slices (split int32
# partials); the tile engine's split-K plan; ragged M/N.
@pytest.mark.parametrize("M,N,K", [(2048, 3072, 1024), (16, 4096, 12288), (200, 1024, 4096),
                                   (100, 640, 1024)])
def test_tensor_linear_w8a8_matches_oracle(T, M, N, K):
    _say(f"tensor_linear_w8a8 M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    tq, tsa, tw, tsw, tb = (_t(T, a) for a in (q, sa, W, sw, b))
    acc = tq.linear_w8a8(tsa, tw, tsw, None, out_dtype="int32").numpy()
    assert np.array_equal(acc, oracle.matmul_nt_i32(q, W))
    for od, bias in (("float32", None), ("float32", tb), ("float16", tb)):
        got = tq.linear_w8a8(tsa, tw, tsw, bias, out_dtype=od).numpy()
        ref = oracle.w8a8(q, sa, W, sw, None if bias is None else b,
                          out="f32" if od == "float32" else "f16")
        # the epilogue rounds like the oracle: byte-equal
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), (od, bias is not None)


def test_tensor_linear_w8a8_rejects_bad_shapes(T):
    q = _t(T, np.zeros((4, 64), np.int8))
    W = _t(T, np.zeros((32, 64), np.int8))
    with pytest.raises(Exception, match="s_a must be"):
        q.linear_w8a8(_t(T, np.ones(3, np.float32)), W, _t(T, np.ones(32, np.float32)))
    with pytest.raises(Exception, match="s_w must be"):
        q.linear_w8a8(_t(T, np.ones(4, np.float32)), W, _t(T, np.ones(31, np.float32)))


# ----------------------------------------------------------------------- MoE
def test_tensor_moe_w8a8_matches_oracle(T):
    Tk, H, I, E, k = 96, 512, 256, 16, 4
    _say(f"tensor_moe_w8a8 T={Tk} H={H} I={I} E={E} k={k}")
    rng = np.random.default_rng(41)
    x = rng.standard_normal((Tk, H), dtype=np.float32).astype(np.float16)
    lg = rng.standard_normal((Tk, E), dtype=np.float32)
    wgu = rng.integers(-127, 127, size=(E, 2 * I, H), dtype=np.int8)
    sgu = rng.uniform(0.001, 0.02, size=(E, 2 * I)).astype(np.float32)
    wd = rng.integers(-127, 127, size=(E, H, I), dtype=np.int8)
    sd = rng.uniform(0.001, 0.02, size=(E, H)).astype(np.float32)
    layer = T.MoEW8A8(H, I, E, k)
    layer.w_gate_up.load(wgu)
    layer.s_gate_up.load(sgu)
    layer.w_down.load(wd)
    layer.s_down.load(sd)
    got = layer(_t(T, x), _t(T, lg)).numpy()
    ref = oracle.moe_w8a8(x, lg, wgu, sgu, wd, sd, k)
    # bit-identical up to the router's expf ulps (see test_moe_layer_matches_oracle)
    assert_rel(got, ref, 1e-4, "tensor_moe_w8a8")


# ------------------------------------------------------ capture and streams
def test_capture_keeps_workspace_from_later_tensors(T):
    """A skinny W8A8 in K slices writes int32 partials to a 1 MiB workspace
    that the op frees as soon as its kernels are queued. Captured with
    begin_capture, that block must stay the graph's: a 1 MiB tensor allocated
    on the same stream afterwards gets other memory, and replays leave it alone."""
    from mod_amd.ops import lib, check
    M, N, K = 16, 4096, 12288
    ws_bytes = 4 * M * N * 4                      # 4 K slices of int32 [M, N]
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.05, size=M).astype(np.float32)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    tq, tsa, tw, tsw = (_t(T, a) for a in (q, sa, W, sw))
    out = T.Tensor([M, N], dtype="float32")
    T.synchronize()
    held0 = int(lib.tensor_pool_graph_bytes())
    g = T.HIPGraph()
    g.capture_begin()
    rc = lib.tensor_linear_w8a8_status(tq._handle, tsa._handle, tw._handle, tsw._handle, None,
                                       out._handle)
    g.capture_end()
    check(rc, "captured tensor_linear_w8a8")
    held = int(lib.tensor_pool_graph_bytes()) - held0
    _say(f"graph holds {held} workspace bytes")
    assert held >= ws_bytes
    victim = T.Tensor([ws_bytes // 4], dtype="int32")
    pattern = np.full(ws_bytes // 4, 0x5A5A5A5A, np.int32)
    victim.load(pattern)
    ref = oracle.w8a8(q, sa, W, sw, out="f32")
    for r in range(3):
        out.fill(0.0)
        g.replay()
        T.synchronize()
        assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32)), f"replay {r}"
        assert np.array_equal(victim.numpy(), pattern), f"replay {r} overwrote a live tensor"
    # a new capture replaces the graph and returns its workspaces to the cache
    g.capture_begin()
    g.capture_end()
    assert int(lib.tensor_pool_graph_bytes()) == held0


def test_failed_capture_returns_its_parked_blocks(T):
    """A capture that the runtime invalidates (here: a stream synchronize on
    the capturing stream, which HIP rejects) ends in a failed end_capture. The
    workspace the captured op parked under it belongs to no graph, so it
    returns to the cache instead of staying counted as graph-held. The capture
    runs on a stream of its own: HIP leaves a stream whose capture was
    invalidated unusable, so that stream is destroyed afterwards."""
    from mod_amd.ops import check, lib, last_error
    M, N, K = 16, 4096, 12288
    rng = np.random.default_rng(5)
    tq = _t(T, rng.integers(-127, 128, size=(M, K), dtype=np.int8))
    tsa = _t(T, rng.uniform(0.001, 0.05, size=M).astype(np.float32))
    tw = _t(T, rng.integers(-127, 128, size=(N, K), dtype=np.int8))
    tsw = _t(T, rng.uniform(0.001, 0.02, size=N).astype(np.float32))
    out = T.Tensor([M, N], dtype="float32")
    T.synchronize()
    lib.begin_capture()
    lib.end_capture()                        # an empty graph: nothing held
    held0 = int(lib.tensor_pool_graph_bytes())
    lib.tensor_clear_error()
    side = T.HIPStream()
    with side:
        lib.begin_capture()
        rc = lib.tensor_linear_w8a8_status(tq._handle, tsa._handle, tw._handle, tsw._handle,
                                           None, out._handle)
        lib.stream_synchronize(None)         # not allowed while capturing
        lib.end_capture()
        err = last_error()
    lib.tensor_clear_error()
    del side
    if "end_capture failed" not in err:
        pytest.skip("this runtime did not invalidate the capture")
    assert rc == 0
    assert int(lib.tensor_pool_graph_bytes()) == held0
    # the library still works on the default stream
    ref = oracle.w8a8(tq.numpy(), tsa.numpy(), tw.numpy(), tsw.numpy(), out="f32")
    check(lib.tensor_linear_w8a8_status(tq._handle, tsa._handle, tw._handle, tsw._handle,
                                        None, out._handle), "tensor_linear_w8a8 after the failed capture")
    T.synchronize()
    assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32))


def test_torch_graph_of_several_ops_with_workspaces(torch_dev):
    """The capture pattern of bench.py: one warm call outside the capture, then
    a torch.cuda.graph holding several ops whose plans need workspaces (the
    MFMA GEMV in K slices, the skinny W8A8 in K slices). Inside one capture the
    later ops reuse the workspace the earlier ones freed (no hipMalloc while
    capturing); every replay, with eager work and a synchronization between
    replays, gives the eager result."""
    import torch
    from mod_amd import ops
    d = torch_dev
    rng = np.random.default_rng(8)
    M, N, K = 16, 4096, 12288
    xh = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)).to(d)
    q = torch.from_numpy(rng.integers(-127, 128, size=(M, K), dtype=np.int8)).to(d)
    sa = torch.from_numpy(rng.uniform(0.001, 0.05, size=M).astype(np.float32)).to(d)
    Ws = [torch.from_numpy(rng.integers(-127, 128, size=(N, K), dtype=np.int8)).to(d) for _ in range(3)]
    sw = torch.from_numpy(rng.uniform(0.001, 0.02, size=N).astype(np.float32)).to(d)
    ys = [torch.empty((M, N), dtype=torch.float32, device=d) for _ in range(6)]
    st = torch.cuda.Stream()

    def work(s):
        for i in range(3):
            ops.gemv_w8(xh, Ws[i], sw, None, ys[i], M, N, K, s)
            ops.gemm_w8a8(q, sa, Ws[i], sw, None, ys[3 + i], M, N, K, s)

    with torch.cuda.stream(st):
        work(st.cuda_stream)
    st.synchronize()
    ref = [y.clone() for y in ys]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            work(st.cuda_stream)
    for r in range(3):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (y, e) in enumerate(zip(ys, ref)):
            assert torch.equal(y, e), f"replay {r}, output {i}"
        junk = torch.randn(1 << 20, device=d) * 2   # eager work between replays
        del junk


def test_destroy_stream_releases_its_cache(T):
    from mod_amd import ops
    from mod_amd.ops import lib
    s = lib.create_stream()
    assert s
    lib.set_current_stream(s)
    try:
        t = T.Tensor([3 << 20], dtype="int8")     # 3 MiB, on the new stream
        del t
        cached = ops.pool_stats()["cached"]
    finally:
        lib.set_current_stream(None)
    lib.destroy_stream(s)
    assert ops.pool_stats()["cached"] <= cached - (3 << 20)


def test_decoder_close_releases_its_stream_memory(T):
    """A decoder without a caller stream owns one; close() drains it and frees
    the decoder's memory instead of leaving it cached under a dead stream."""
    from mod_amd import ops
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    cfg = Qwen3Config(n_layers=2, vocab=1000, max_seq=64)
    w = random_weights(cfg, seed=5)
    dev_w = {k: (T.Tensor.from_numpy(np.ascontiguousarray(v)) if isinstance(v, np.ndarray) else v)
             for k, v in w.items() if k != "layers"}
    dev_w["layers"] = [{k: (None if v is None else T.Tensor.from_numpy(np.ascontiguousarray(v)))
                        for k, v in L.items()} for L in w["layers"]]
    T.synchronize()
    r0 = ops.pool_stats()["reserved"]
    dec = Qwen3Int8Decoder(cfg, dev_w)
    dec.reset(np.arange(8, dtype=np.int32))
    mode = "persistent" if dec.persistent_supported() else "graph"
    dec.run(4, mode=mode)
    dec.read(12)
    assert ops.pool_stats()["reserved"] > r0
    dec.close()
    assert ops.pool_stats()["reserved"] == r0


CHILD = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    import numpy as np
    import torch
    assert torch.cuda.is_available()
    from mod_amd import backend as B, ops
    # arena: tensors bump-allocate from it, ops run on them, reset rewinds it
    B.init_memory_pool(64)
    st = ops.pool_stats()
    assert st["arena_size"] == 64 << 20, st
    rng = np.random.default_rng(1)
    q = rng.integers(-127, 128, size=(64, 1024), dtype=np.int8)
    W = rng.integers(-127, 128, size=(256, 1024), dtype=np.int8)
    tq, tw = B.Tensor.from_numpy(q), B.Tensor.from_numpy(W)
    sa = B.Tensor.from_numpy(np.ones(64, np.float32))
    sw = B.Tensor.from_numpy(np.ones(256, np.float32))
    acc = tq.linear_w8a8(sa, tw, sw, None, out_dtype="int32").numpy()
    ref = q.astype(np.int64) @ W.astype(np.int64).T
    assert np.array_equal(acc, ref)
    used = ops.pool_stats()["arena_used"]
    assert used >= q.nbytes + W.nbytes, used
    del tq, tw, sa, sw
    B.reset_memory_pool()
    assert ops.pool_stats()["arena_used"] == 0
    # persistent decode, then a normal interpreter exit with the decoder left
    # to __del__ at shutdown
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    cfg = Qwen3Config(n_layers=2, vocab=1000, max_seq=64)
    dec = Qwen3Int8Decoder(cfg, random_weights(cfg, seed=2))
    mode = "persistent" if dec.persistent_supported() else "graph"
    ids = dec.generate(np.arange(6, dtype=np.int32), 8, mode=mode)
    print("CHILD_OK", mode, ids[-3:].tolist(), flush=True)
    sys.exit(0)
""")


def test_arena_and_clean_exit_in_child_process(torch_dev):
    _say("child process: arena pool, persistent decode, normal exit")
    env = dict(os.environ)
    res = subprocess.run([sys.executable, "-c", CHILD.format(root=str(ROOT))], env=env,
                         capture_output=True, text=True, timeout=240)
    _say(res.stdout[-2000:] + res.stderr[-2000:])
    assert res.returncode == 0, f"child exited with {res.returncode}"
    assert "CHILD_OK" in res.stdout
