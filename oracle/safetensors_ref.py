"""safetensors format restated in numpy -- TEST INFRASTRUCTURE ONLY.

The checker of the product's safetensors reader (``weights.hip``) and of the
int8 checkpoint format built on it. Only ``tests/`` may import it.

Format (the published safetensors layout; the reference reads the same files in
plugins/cpu/c_src/safetensors_loader.c:40-120): a little-endian u64 header
length N, N bytes of JSON mapping names to {"dtype", "shape", "data_offsets":
[begin, end]} plus an optional "__metadata__" object, then the data region;
offsets count from byte 8 + N.

Parity pins:
* ``read_all`` against the ``safetensors`` package (an independent reader of the
  same format) on files it wrote, every dtype the product handles;
* ``to_f32`` of F16 against numpy's IEEE half conversion over all 65536 bit
  patterns, and of BF16 by the definition (bf16 = top 16 bits of an f32);
* ``load_tensor_data`` of the reference itself (``_ref/libsafetensors_ref.so``,
  built from safetensors_loader.c:147-243) for the F32 and F16 files it reads
  correctly.
* ``quant_per_channel`` is the per-token quantizer (``int8_ref.c``) applied to
  weight rows; that function is pinned in ``test_oracle.py``.
"""
from __future__ import annotations

import json
import struct

import numpy as np

# safetensors dtype string -> numpy dtype of the stored element (BF16 as its
# raw 16-bit pattern; numpy has no bfloat16).
NP_OF = {
    "F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16,
    "I64": np.int64, "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8,
    "BOOL": np.bool_, "U16": np.uint16, "U32": np.uint32, "U64": np.uint64,
}


def read_header(path):
    """(entries, data_start): entries maps name -> (dtype, shape, begin, end)."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
    hdr.pop("__metadata__", None)
    return ({k: (v["dtype"], tuple(v["shape"]), v["data_offsets"][0], v["data_offsets"][1])
             for k, v in hdr.items()}, 8 + n)


def read_all(path) -> dict:
    """name -> numpy array of the stored element type (BF16 as uint16 bits)."""
    entries, d0 = read_header(path)
    raw = np.fromfile(path, dtype=np.uint8)
    out = {}
    for k, (dt, shape, b, e) in entries.items():
        out[k] = raw[d0 + b:d0 + e].view(NP_OF[dt]).reshape(shape).copy()
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (NaNs kept quiet)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def to_f32(dtype: str, a: np.ndarray) -> np.ndarray:
    """The f32 value of each stored element."""
    if dtype == "BF16":
        return bf16_to_f32(a)
    return a.astype(np.float32)


def quant_per_channel(w_f32: np.ndarray):
    """Offline per-output-channel quantization of an fp weight [N, K]:
    s[n] = amax_k |w[n,k]| / 127 (1 for an all-zero row), q = clamp(rint(w/s)).
    The same arithmetic as the per-token activation quantizer, row for row."""
    from . import quant_per_token
    return quant_per_token(np.ascontiguousarray(w_f32, np.float32))


def write(path, tensors: dict, dtypes: dict | None = None, metadata: dict | None = None,
          order=None) -> None:
    """Minimal writer used to build malformed / edge-case files for tests.
    ``dtypes`` overrides the dtype string per name (e.g. "BF16" for uint16 bits)."""
    dtypes = dtypes or {}
    inv = {np.dtype(v).str: k for k, v in NP_OF.items() if k not in ("BF16",)}
    hdr, blobs, off = {}, [], 0
    for k in (order or list(tensors)):
        a = np.ascontiguousarray(tensors[k])
        dt = dtypes.get(k) or inv[a.dtype.str]
        b = a.tobytes()
        hdr[k] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata is not None:
        hdr["__metadata__"] = metadata
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
