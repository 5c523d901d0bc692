"""GPU tests of the int8 on-disk weight path: safetensors data into device
tensors, per-channel quantization of fp checkpoints on the GPU, the int8
checkpoint format written by quantize_checkpoint, and a decoder built from a
checkpoint.

Bars: stored bytes land bit-exact; fp32 conversions equal the oracle's
(safetensors_ref.to_f32, pinned in test_weights.py); int8 weights and their
scales equal the oracle quantizer's (int8_ref.c ref_quant_per_token over weight
rows) bit for bit; a decoder built from a checkpoint gives logits identical to
one built from the oracle-quantized arrays (same kernels, same int8 weights).
"""
import ctypes
import json
import sys

import numpy as np
import pytest

import oracle
from oracle import safetensors_ref as stref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
st_t = pytest.importorskip("safetensors.torch")


def _say(m):
    print(m, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def M():
    from mod_amd import backend, ops, qwen3, weights
    return backend, ops, weights, qwen3


def _bf16(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def _save(path, arrays: dict, bf16=()):
    """Write with the safetensors package; names in ``bf16`` stored as BF16."""
    st_t.save_file({k: (_bf16(v) if k in bf16 else torch.from_numpy(np.ascontiguousarray(v)))
                    for k, v in arrays.items()}, str(path))


def test_device_loads_every_dtype(tmp_path, M):
    backend, ops, W, _ = M
    rng = np.random.default_rng(0)
    big = rng.integers(-128, 128, (5000, 4200), dtype=np.int8)   # 21 MB: three staging chunks
    data = {"i8": rng.integers(-128, 128, (40, 96), dtype=np.int8), "big": big,
            "f32": rng.standard_normal((33, 65)).astype(np.float32),
            "f16": rng.standard_normal((17, 130)).astype(np.float16),
            "bf": rng.standard_normal((9, 300)).astype(np.float32),
            "u8": rng.integers(0, 256, (77,), dtype=np.uint8),
            "i16": rng.integers(-2 ** 15, 2 ** 15, (3, 41), dtype=np.int16),
            "i32": rng.integers(-2 ** 24, 2 ** 24, (5, 7), dtype=np.int32),
            "flag": rng.integers(0, 2, (19,)).astype(np.bool_),
            "bf_big": rng.standard_normal((3000, 1111)).astype(np.float32)}
    p = tmp_path / "d.safetensors"
    _say("test_device_loads_every_dtype: writing")
    _save(p, data, bf16=("bf", "bf_big"))
    ref = stref.read_all(p)
    with W.SafetensorsFile(p) as f:
        T = backend.Tensor
        for name, dt in (("i8", "int8"), ("big", "int8"), ("u8", "int8"), ("f32", "float32"),
                         ("f16", "float16"), ("f16", "float32"), ("bf", "float32"),
                         ("i8", "float32"), ("u8", "float32"), ("i16", "float32"),
                         ("i32", "float32"), ("flag", "float32"), ("bf_big", "float32")):
            _say(f"  load {name} -> {dt}")
            t = T(list(ref[name].shape), dtype=dt)
            f.load_into(name, t)
            got = t.numpy()
            inf = f.info(name)
            if dt == "int8":
                exp = ref[name].view(np.int8)
            elif dt == "float16":
                exp = ref[name]
            else:
                exp = stref.to_f32(inf.dtype, ref[name])
            assert got.dtype == exp.dtype and np.array_equal(got.view(np.uint8),
                                                             exp.view(np.uint8)), (name, dt)
        # refused combinations: no silent reinterpretation
        for name, dt in (("bf", "float16"), ("f32", "int8"), ("f32", "int32")):
            t = T(list(ref[name].shape), dtype=dt)
            with pytest.raises(ops.RocmError):
                f.load_into(name, t)
        with pytest.raises(ops.RocmError):
            f.load_into("f32", T([65, 33]))          # same count, other shape
        t = T([33 * 65 + 1])
        assert ops.lib.tensor_load_safetensors_status(f._ctx, b"f32", t._handle) == ops.ERR_INVALID
        # raw device copy on an explicit stream
        s = ops.lib.create_stream()
        try:
            t = T([40, 96], dtype="int8")
            ops.check(ops.lib.pio_safetensors_to_device(f._ctx, b"i8", t.data_ptr(), 40 * 96, s))
            assert np.array_equal(t.numpy(), data["i8"])
            assert ops.lib.pio_safetensors_to_device(f._ctx, b"i8", t.data_ptr(), 40 * 96 - 1,
                                                     s) == ops.ERR_INVALID
        finally:
            ops.lib.destroy_stream(s)


@pytest.mark.parametrize("shape,dtype", [((3072, 1024), "BF16"), ((130, 520), "F16"),
                                         ((7, 4096), "F32"), ((1, 12288), "BF16"),
                                         ((257, 96), "F32")])
def test_fp_weight_quantized_on_gpu(tmp_path, M, shape, dtype):
    backend, ops, W, _ = M
    rng = np.random.default_rng(hash(shape) & 0xFFFF)
    w = (rng.standard_normal(shape) * rng.uniform(0.01, 3.0, (shape[0], 1))).astype(np.float32)
    w[min(3, shape[0] - 1)] = 0.0   # an all-zero channel: scale 1, q 0
    p = tmp_path / "q.safetensors"
    store = {"F32": w, "F16": w.astype(np.float16), "BF16": w}[dtype]
    _save(p, {"layer.weight": store}, bf16=("layer.weight",) if dtype == "BF16" else ())
    stored = stref.read_all(p)["layer.weight"]
    eq, es = stref.quant_per_channel(stref.to_f32(dtype, stored))
    _say(f"test_fp_weight_quantized_on_gpu {shape} {dtype}")
    q = backend.Tensor(list(shape), dtype="int8")
    s = backend.Tensor([shape[0]])
    with W.SafetensorsFile(p) as f:
        W.load_int8_weight(f, "layer.weight", q, s)
    assert np.array_equal(q.numpy(), eq)
    assert np.array_equal(s.numpy().view(np.uint32), es.view(np.uint32))


class _Net:
    """Two int8 linears registered the way reference modules register
    submodules (Module._modules, backend.py:656-692)."""

    def __new__(cls, backend, bias):
        net = backend.Module()
        net.a = backend.W8Linear(256, 384, bias=bias)
        net.b = backend.W8Linear(384, 128, bias=False)
        net._modules["proj_a"] = net.a
        net._modules["proj_b"] = net.b
        return net


def test_load_safetensors_fp_and_int8_formats(tmp_path, M):
    backend, ops, W, _ = M
    rng = np.random.default_rng(5)
    wa = rng.standard_normal((384, 256)).astype(np.float32)
    wb = rng.standard_normal((128, 384)).astype(np.float32) * 0.05
    ba = rng.standard_normal(384).astype(np.float32)
    src = tmp_path / "fp.safetensors"
    _save(src, {"proj_a.weight": wa, "proj_a.bias": ba, "proj_b.weight": wb,
                "unrelated.norm.weight": np.ones(8, np.float32)},
          bf16=("proj_a.weight", "proj_b.weight"))
    stored = stref.read_all(src)
    ea = stref.quant_per_channel(stref.to_f32("BF16", stored["proj_a.weight"]))
    eb = stref.quant_per_channel(stref.to_f32("BF16", stored["proj_b.weight"]))

    _say("load_safetensors: fp (BF16) checkpoint")
    n1 = _Net(backend, True)
    assert W.load_safetensors(src, n1.state_dict())
    for lin, (eq, es) in ((n1.a, ea), (n1.b, eb)):
        assert np.array_equal(lin.weight.numpy(), eq)
        assert np.array_equal(lin.weight_scale.numpy(), es)
    assert np.array_equal(n1.a.bias.numpy(), ba)

    _say("quantize_checkpoint -> int8 format")
    dst = tmp_path / "int8.safetensors"
    got = W.quantize_checkpoint(src, dst)
    assert sorted(got) == ["proj_a.weight", "proj_b.weight"]
    out = stref.read_all(dst)
    assert out["proj_a.weight"].dtype == np.int8 and np.array_equal(out["proj_a.weight"], ea[0])
    assert np.array_equal(out["proj_a.weight_scale"], ea[1])
    assert np.array_equal(out["proj_b.weight"], eb[0])
    assert np.array_equal(out["proj_a.bias"], ba)
    assert np.array_equal(out["unrelated.norm.weight"], np.ones(8, np.float32))
    with open(dst, "rb") as fh:
        n = int.from_bytes(fh.read(8), "little")
        meta = json.loads(fh.read(n))["__metadata__"]
    assert "int8" in meta["quantization"]

    _say("load_weights from the int8 checkpoint (strict)")
    n2 = _Net(backend, True)
    names = W.load_weights(n2, dst, strict=True)
    assert set(names) == set(n2.state_dict())
    for l1, l2 in ((n1.a, n2.a), (n1.b, n2.b)):
        assert np.array_equal(l1.weight.numpy(), l2.weight.numpy())
        assert np.array_equal(l1.weight_scale.numpy(), l2.weight_scale.numpy())
    x = backend.Tensor.from_numpy(rng.standard_normal((4, 256)).astype(np.float32))
    y1, y2 = n1.b(n1.a(x)).numpy(), n2.b(n2.a(x)).numpy()
    assert np.array_equal(y1, y2)
    ref = oracle.gemv_w8(oracle.gemv_w8(x.numpy(), ea[0], ea[1], ba), eb[0], eb[1])
    np.testing.assert_allclose(y1, ref, rtol=1e-3, atol=1e-3 * float(np.abs(ref).max()))

    _say("strict load with a parameter the file lacks")
    n3 = _Net(backend, True)
    n3._modules["proj_c"] = backend.W8Linear(8, 8, bias=False)
    with pytest.raises(ops.RocmError):
        W.load_weights(n3, dst, strict=True)
    assert not W.load_safetensors(tmp_path / "absent.safetensors", n3.state_dict())

    _say("W8Linear.load_float quantizes on the GPU")
    lin = backend.W8Linear(256, 384, bias=False)
    lin.load_float(stref.to_f32("BF16", stored["proj_a.weight"]))
    assert np.array_equal(lin.weight.numpy(), ea[0])
    assert np.array_equal(lin.weight_scale.numpy(), ea[1])


def _tiny_cfg(qwen3):
    kw = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512,
              vocab=1000, max_seq=64)
    return qwen3.Qwen3Config(**kw)


def _hf_checkpoint(cfg, rng, tied: bool):
    H, D, I, V = cfg.hidden, cfg.head_dim, cfg.intermediate, cfg.vocab
    nq, nkv = cfg.n_heads * D, cfg.n_kv_heads * D
    t = {}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        t[p + "post_attention_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(H)).astype(
            np.float32)
        for n, r, k in (("self_attn.q_proj", nq, H), ("self_attn.k_proj", nkv, H),
                        ("self_attn.v_proj", nkv, H), ("self_attn.o_proj", H, nq),
                        ("mlp.gate_proj", I, H), ("mlp.up_proj", I, H), ("mlp.down_proj", H, I)):
            t[p + n + ".weight"] = (rng.standard_normal((r, k)) / np.sqrt(k)).astype(np.float32)
        for n, r in (("q_proj", nq), ("k_proj", nkv), ("v_proj", nkv)):
            t[p + f"self_attn.{n}.bias"] = (0.1 * rng.standard_normal(r)).astype(np.float32)
    t["model.embed_tokens.weight"] = rng.standard_normal((V, H)).astype(np.float32)
    t["model.norm.weight"] = np.ones(H, np.float32)
    if not tied:
        t["lm_head.weight"] = (rng.standard_normal((V, H)) / np.sqrt(H)).astype(np.float32)
    return t


def _oracle_weights(cfg, stored: dict, tied: bool):
    """Host decoder weights from the stored checkpoint values, quantized by the
    oracle (rows stacked q,k,v and gate,up before per-row quantization)."""
    f = {k: stref.to_f32("BF16" if v.dtype == np.uint16 else "F32", v) for k, v in stored.items()}
    layers = []
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        L = {"in_norm": f[p + "input_layernorm.weight"],
             "post_norm": f[p + "post_attention_layernorm.weight"]}
        L["w_qkv"], L["s_qkv"] = stref.quant_per_channel(np.concatenate(
            [f[p + f"self_attn.{n}_proj.weight"] for n in "qkv"]))
        L["b_qkv"] = np.concatenate([f[p + f"self_attn.{n}_proj.bias"] for n in "qkv"])
        L["w_o"], L["s_o"] = stref.quant_per_channel(f[p + "self_attn.o_proj.weight"])
        L["w_gu"], L["s_gu"] = stref.quant_per_channel(np.concatenate(
            [f[p + "mlp.gate_proj.weight"], f[p + "mlp.up_proj.weight"]]))
        L["w_down"], L["s_down"] = stref.quant_per_channel(f[p + "mlp.down_proj.weight"])
        layers.append(L)
    lm, s_lm = stref.quant_per_channel(f["model.embed_tokens.weight" if tied else "lm_head.weight"])
    return {"embed": f["model.embed_tokens.weight"], "final_norm": f["model.norm.weight"],
            "lm_head": lm, "s_lm_head": s_lm, "layers": layers}


@pytest.mark.parametrize("tied", [False, True])
def test_qwen3_decoder_from_checkpoint(tmp_path, M, tied):
    backend, ops, W, qwen3 = M
    cfg = _tiny_cfg(qwen3)
    rng = np.random.default_rng(11 + tied)
    t = _hf_checkpoint(cfg, rng, tied)
    src = tmp_path / "model.safetensors"
    bf = [k for k in t if k.endswith("proj.weight") or k == "lm_head.weight"]
    _save(src, t, bf16=bf)
    stored = stref.read_all(src)
    ids = np.random.default_rng(3).integers(0, cfg.vocab, 12).astype(np.int32)

    _say(f"qwen3 from checkpoint (tied={tied}): oracle-quantized reference decoder")
    ref = qwen3.Qwen3Int8Decoder(cfg, _oracle_weights(cfg, stored, tied))
    exp = ref.teacher_forced_logits(ids)
    ref.close()

    _say("  fp checkpoint directory, quantized on load")
    dec = qwen3.Qwen3Int8Decoder(cfg, qwen3.weights_from_checkpoint(tmp_path, cfg))
    assert np.array_equal(dec.teacher_forced_logits(ids), exp)
    dec.close()

    _say("  int8 checkpoint written by quantize_checkpoint (split q/k/v, gate/up)")
    dst = tmp_path / "int8.safetensors"
    W.quantize_checkpoint(src, dst)
    dec = qwen3.Qwen3Int8Decoder(cfg, qwen3.weights_from_checkpoint(dst, cfg))
    assert np.array_equal(dec.teacher_forced_logits(ids), exp)
    dec.close()

    _say("  int8 checkpoint in the fused reference layout (qkv_proj, gate_up_proj)")
    ow = _oracle_weights(cfg, stored, tied)
    fused, dts = {}, {}
    for i, L in enumerate(ow["layers"]):
        p = f"model.layers.{i}."
        fused[p + "input_layernorm.weight"] = L["in_norm"]
        fused[p + "post_attention_layernorm.weight"] = L["post_norm"]
        for nm, wk, sk in (("self_attn.qkv_proj", "w_qkv", "s_qkv"),
                           ("self_attn.o_proj", "w_o", "s_o"),
                           ("mlp.gate_up_proj", "w_gu", "s_gu"),
                           ("mlp.down_proj", "w_down", "s_down")):
            fused[p + nm + ".weight"], fused[p + nm + ".weight_scale"] = L[wk], L[sk]
        fused[p + "self_attn.qkv_proj.bias"] = L["b_qkv"]
    fused["model.embed_tokens.weight"] = stored["model.embed_tokens.weight"]
    fused["model.norm.weight"] = ow["final_norm"]
    if not tied:
        fused["lm_head.weight"], fused["lm_head.weight_scale"] = ow["lm_head"], ow["s_lm_head"]
    fdir = tmp_path / "fused"
    fdir.mkdir()
    W.save_safetensors(fdir / "model.safetensors", fused)
    dec =qwen3.Qwen3Int8Decoder(cfg, qwen3.weights_from_checkpoint(fdir, cfg))
    assert np.array_equal(dec.teacher_forced_logits(ids), exp)
    dec.close()


def test_qwen3_checkpoint_errors(tmp_path, M):
    backend, ops, W, qwen3 = M
    cfg = _tiny_cfg(qwen3)
    t = _hf_checkpoint(cfg, np.random.default_rng(2), tied=False)
    t["model.layers.0.self_attn.q_norm.weight"] = np.ones(cfg.head_dim, np.float32)
    p = tmp_path / "extra.safetensors"
    _save(p, t)
    _say("qwen3 checkpoint with an unused q_norm (strict)")
    with pytest.raises(ops.RocmError, match="q_norm"):
        qwen3.weights_from_checkpoint(p, cfg)
    del t["model.layers.0.self_attn.q_norm.weight"]
    t["model.layers.1.mlp.down_proj.weight"] = t["model.layers.1.mlp.down_proj.weight"][:, :-1]
    p2 = tmp_path / "bad.safetensors"
    _save(p2, t)
    with pytest.raises(ops.RocmError, match="down_proj"):
        qwen3.weights_from_checkpoint(p2, cfg)
