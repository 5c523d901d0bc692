"""safetensors reader (weights.hip) on the CPU: header parsing, dtype
conversion, reference parity of the drop-in entry points, and rejection of
malformed files. No GPU calls here: only the host entry points
(open / load_tensor_data / info / read / close) run.

Pins:
* files written by the ``safetensors`` package (an independent implementation
  of the format) read back equal to that package's own reader;
* F16 conversion equal to numpy's IEEE half for every non-NaN bit pattern and
  bit-equal to the reference's half_to_float (safetensors_loader.c:123-145) for
  all 65536 patterns, through the reference's load_tensor_data;
* BF16 equal to its definition (the top half of an f32), where the reference
  returns F16 values (the byte-count dispatch of safetensors_loader.c:183-196).
"""
import ctypes
import json
import struct

import numpy as np
import pytest

import oracle
from oracle import safetensors_ref as stref

st_np = pytest.importorskip("safetensors.numpy")


@pytest.fixture(scope="module")
def W():
    from mod_amd import weights
    return weights


def _ref_loader():
    if not (oracle.HERE / "_ref" / "libsafetensors_ref.so").exists():
        pytest.skip("reference safetensors loader not built (needs /root/reference)")
    L = ctypes.CDLL(str(oracle.HERE / "_ref" / "libsafetensors_ref.so"))
    L.open_safetensors.restype = ctypes.c_void_p
    L.open_safetensors.argtypes = [ctypes.c_char_p]
    L.load_tensor_data.restype = ctypes.c_int
    L.load_tensor_data.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                   ctypes.POINTER(ctypes.c_float), ctypes.c_int]
    L.close_safetensors.argtypes = [ctypes.c_void_p]
    return L


def _load_f32(L, ctx, name, n):
    buf = np.full(n, np.nan, np.float32)
    rc = L.load_tensor_data(ctx, name.encode(), buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                            n)
    return rc, buf


def _mixed(rng):
    return {
        "a.f64": rng.standard_normal((3, 5)),
        "a.f32": rng.standard_normal((7, 9)).astype(np.float32),
        "b.f16": rng.standard_normal((4, 33)).astype(np.float16),
        "c.i8": rng.integers(-128, 128, (17, 31), dtype=np.int8),
        "d.u8": rng.integers(0, 256, (5,), dtype=np.uint8),
        "e.i32": rng.integers(-2 ** 31, 2 ** 31, (6, 2), dtype=np.int32),
        "f.i16": rng.integers(-2 ** 15, 2 ** 15, (11,), dtype=np.int16),
        "g.bool": rng.integers(0, 2, (9,)).astype(np.bool_),
        "h.i64": rng.integers(-2 ** 40, 2 ** 40, (3,), dtype=np.int64),
        "scalar": np.array(3.5, np.float32),
        "empty": np.zeros((0, 4), np.float32),
    }


def test_parse_matches_safetensors_package(tmp_path, W):
    rng = np.random.default_rng(0)
    data = _mixed(rng)
    p = tmp_path / "m.safetensors"
    st_np.save_file(data, str(p), metadata={"format": "pt", "note": "\"model.x\" [1, 2]"})
    back = st_np.load_file(str(p))
    with W.SafetensorsFile(p) as f:
        assert sorted(f.names()) == sorted(data)
        for k, v in back.items():
            inf = f.info(k)
            assert inf.shape == v.shape and inf.nbytes == v.nbytes, k
            got = f.read(k)
            assert got.dtype == v.dtype and np.array_equal(got, v), k
        for k in ("a.f32", "b.f16", "c.i8", "d.u8", "e.i32", "f.i16", "g.bool", "scalar", "empty"):
            np.testing.assert_array_equal(f.read_f32(k), back[k].astype(np.float32), err_msg=k)
        assert "a.f32" in f and "a.f3" not in f and "__metadata__" not in f


def test_bf16_by_definition(tmp_path, W):
    torch = pytest.importorskip("torch")
    st_t = pytest.importorskip("safetensors.torch")
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((64, 48)).astype(np.float32)).to(torch.bfloat16)
    p = tmp_path / "bf.safetensors"
    st_t.save_file({"w": x}, str(p))
    bits = x.view(torch.int16).numpy().view(np.uint16)
    with W.SafetensorsFile(p) as f:
        inf = f.info("w")
        assert inf.dtype == "BF16" and inf.shape == (64, 48)
        assert np.array_equal(f.read("w"), bits)
        got = f.read_f32("w")
    assert np.array_equal(got.view(np.uint32), stref.bf16_to_f32(bits).view(np.uint32))
    assert np.array_equal(got, x.float().numpy())


def test_all_f16_patterns_vs_numpy_and_reference(tmp_path, W):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    p = tmp_path / "h.safetensors"
    stref.write(p, {"h": bits.view(np.float16)})
    with W.SafetensorsFile(p) as f:
        got = f.read_f32("h")
    ref_np = bits.view(np.float16).astype(np.float32)
    fin = ~np.isnan(ref_np)
    assert np.array_equal(got[fin].view(np.uint32), ref_np[fin].view(np.uint32))
    assert np.isnan(got[~fin]).all()
    L = _ref_loader()
    ctx = L.open_safetensors(str(p).encode())
    assert ctx
    try:
        rc, ref = _load_f32(L, ctx, "h", 65536)
    finally:
        L.close_safetensors(ctx)
    assert rc == 1
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_drop_in_entry_points_match_reference(tmp_path):
    """open / load_tensor_data / close: same outputs and return codes as the
    reference loader on the files it reads correctly (F32 and F16), including
    a size mismatch and an absent name."""
    from mod_amd import ops
    rng = np.random.default_rng(2)
    data = {"model.layers.0.w": rng.standard_normal((33, 65)).astype(np.float32),
            "model.layers.0.w_h": rng.standard_normal((5, 129)).astype(np.float16),
            "lm_head.weight": rng.standard_normal((1, 7)).astype(np.float32)}
    p = tmp_path / "r.safetensors"
    st_np.save_file(data, str(p))
    L = _ref_loader()
    ours = ops.lib
    c_ref, c_ours = L.open_safetensors(str(p).encode()), ours.open_safetensors(str(p).encode())
    assert c_ref and c_ours
    try:
        for name, n in (("model.layers.0.w", 33 * 65), ("model.layers.0.w_h", 5 * 129),
                        ("lm_head.weight", 7), ("lm_head.weight", 8), ("nope", 4),
                        ("model.layers.0.w", 33 * 65 - 1)):
            r_rc, r_buf = _load_f32(L, c_ref, name, n)
            o_rc, o_buf = _load_f32(ours, c_ours, name, n)
            assert r_rc == o_rc, name
            if r_rc:
                assert np.array_equal(r_buf.view(np.uint32), o_buf.view(np.uint32)), name
    finally:
        L.close_safetensors(c_ref)
        ours.close_safetensors(c_ours)
    assert not ours.open_safetensors(str(tmp_path / "missing.safetensors").encode())
    ours.close_safetensors(None)


def test_header_order_and_metadata_independence(tmp_path, W):
    """Field order inside an entry and names quoted in __metadata__ do not
    change what is read (the reference's text search keys on both)."""
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = -np.arange(6, dtype=np.float32)
    hdr = {"__metadata__": {"alias": "\"b\""},
           "b": {"data_offsets": [48, 72], "shape": [6], "dtype": "F32"},
           "a": {"shape": [3, 4], "dtype": "F32", "data_offsets": [0, 48], "extra": [1, {"x": 2}]}}
    h = json.dumps(hdr).encode()
    p = tmp_path / "o.safetensors"
    p.write_bytes(struct.pack("<Q", len(h)) + h + a.tobytes() + b.tobytes())
    with W.SafetensorsFile(p) as f:
        assert f.names() == ["b", "a"]
        assert np.array_equal(f.read_f32("a"), a) and np.array_equal(f.read_f32("b"), b)


def _raw(p, hdr_bytes, payload=b""):
    p.write_bytes(struct.pack("<Q", len(hdr_bytes)) + hdr_bytes + payload)


@pytest.mark.parametrize("case", [
    "too_short", "hdr_len_beyond", "not_json", "offsets_beyond", "bytes_vs_shape", "dup",
    "neg_dim", "bad_dtype", "missing_field", "reversed_offsets", "float_offset", "bad_escape",
])
def test_malformed_files_rejected(tmp_path, case, W):
    from mod_amd import ops
    p = tmp_path / f"{case}.safetensors"
    ent = lambda dt, shape, b, e: {"dtype": dt, "shape": shape, "data_offsets": [b, e]}  # noqa: E731
    payload = bytes(64)
    if case == "too_short":
        p.write_bytes(b"\x01\x00")
    elif case == "hdr_len_beyond":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "not_json":
        _raw(p, b"{\"a\": {\"dtype\": \"F32\", ", payload)
    elif case == "offsets_beyond":
        _raw(p, json.dumps({"a": ent("F32", [32], 0, 128)}).encode(), payload)
    elif case == "bytes_vs_shape":
        _raw(p, json.dumps({"a": ent("F32", [3, 4], 0, 40)}).encode(), payload)
    elif case == "dup":
        _raw(p, b'{"a": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]}, '
                b'"a": {"dtype": "I8", "shape": [4], "data_offsets": [4, 8]}}', payload)
    elif case == "neg_dim":
        _raw(p, json.dumps({"a": ent("I8", [-4], 0, 4)}).encode(), payload)
    elif case == "bad_dtype":
        _raw(p, json.dumps({"a": ent("F8_E9", [4], 0, 4)}).encode(), payload)
    elif case == "missing_field":
        _raw(p, json.dumps({"a": {"dtype": "I8", "shape": [4]}}).encode(), payload)
    elif case == "reversed_offsets":
        _raw(p, json.dumps({"a": ent("I8", [0], 8, 4)}).encode(), payload)
    elif case == "float_offset":
        _raw(p, b'{"a": {"dtype": "I8", "shape": [4], "data_offsets": [0.0, 4]}}', payload)
    elif case == "bad_escape":
        _raw(p, b'{"a\\u00zz": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]}}', payload)
    assert not ops.lib.open_safetensors(str(p).encode())
    assert ops.last_error()
    with pytest.raises(ops.RocmError):
        W.SafetensorsFile(p)


def test_read_rejects_wrong_sizes(tmp_path, W):
    from mod_amd import ops
    p = tmp_path / "s.safetensors"
    st_np.save_file({"a": np.ones((4, 4), np.int8), "b": np.ones(3, np.float64)}, str(p))
    with W.SafetensorsFile(p) as f:
        buf = np.empty(15, np.int8)
        assert ops.lib.pio_safetensors_read(f._ctx, b"a", buf.ctypes.data, 15) == ops.ERR_INVALID
        assert ops.lib.pio_safetensors_read(f._ctx, b"zz", buf.ctypes.data, 15) == ops.ERR_INVALID
        with pytest.raises(ops.RocmError):
            f.read_f32("b")   # F64 has no fp32 conversion in the loader
        assert ops.lib.pio_safetensors_name(f._ctx, 2) is None
        assert ops.lib.pio_safetensors_name(f._ctx, -1) is None
    with pytest.raises(ValueError):
        f.names()


def test_checkpoint_index_and_shards(tmp_path, W):
    rng = np.random.default_rng(3)
    a = {"x.weight": rng.standard_normal((4, 8)).astype(np.float32)}
    b = {"y.weight": rng.integers(-127, 128, (2, 8), dtype=np.int8),
         "y.weight_scale": np.ones(2, np.float32)}
    st_np.save_file(a, str(tmp_path / "model-00001-of-00002.safetensors"))
    st_np.save_file(b, str(tmp_path / "model-00002-of-00002.safetensors"))
    idx = {"weight_map": {"x.weight": "model-00001-of-00002.safetensors",
                          "y.weight": "model-00002-of-00002.safetensors",
                          "y.weight_scale": "model-00002-of-00002.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert len(W.checkpoint_files(tmp_path)) == 2
    with W.Checkpoint(tmp_path) as ck:
        assert sorted(ck.names()) == ["x.weight", "y.weight", "y.weight_scale"]
        assert np.array_equal(ck.read("y.weight"), b["y.weight"])
        assert np.array_equal(ck.read_f32("x.weight"), a["x.weight"])
        assert W.iter_int8_pairs(ck.names()) == ["y.weight"]
    assert W.checkpoint_files(tmp_path / "nothing") == []


def test_writer_roundtrip(tmp_path, W):
    """save_safetensors output reads back equal through the safetensors package
    and through the product reader (incl. BF16 bits, 0-d and empty arrays)."""
    rng = np.random.default_rng(4)
    data = {"w": rng.integers(-127, 128, (33, 70), dtype=np.int8),
            "w_scale": rng.uniform(0.001, 0.02, 33).astype(np.float32),
            "bf": stref.f32_to_bf16_rne(rng.standard_normal((3, 5)).astype(np.float32)),
            "h": rng.standard_normal(9).astype(np.float16),
            "z": np.array(7, np.int32), "e": np.zeros((0, 3), np.float32)}
    p = tmp_path / "w.safetensors"
    W.save_safetensors(p, data, dtypes={"bf": "BF16"}, metadata={"k": "v"})
    back = stref.read_all(p)
    for k, v in data.items():
        assert back[k].dtype == v.dtype and np.array_equal(back[k], v), k
    from safetensors import safe_open
    with safe_open(str(p), framework="np") as pkg:
        for k in ("w", "w_scale", "h", "z", "e"):
            v = pkg.get_tensor(k)
            assert v.shape == data[k].shape and np.array_equal(v, data[k]), k
        assert pkg.metadata()["k"] == "v"
    with W.SafetensorsFile(p) as f:
        assert f.info("bf").dtype == "BF16" and np.array_equal(f.read("bf"), data["bf"])
        assert np.array_equal(f.read_f32("bf"), stref.bf16_to_f32(data["bf"]))
    with pytest.raises(ValueError):
        W.save_safetensors(tmp_path / "x.safetensors", {"a": np.ones(3, np.float32)},
                           dtypes={"a": "BF16"})
