"""int8 on-disk weights: safetensors checkpoints for the int8 linear path.

Replaces the reference's weight loading -- ``load_safetensors``
(ip/core/engine/backend.py:812-835) over the C loader
(plugins/cpu/c_src/safetensors_loader.c) and ``CustomModelLoader.load_weights``
(common/custom_components/model_loader.py:77-123) -- and adds the int8 format:

* an int8 linear is stored as ``<prefix>.weight`` (I8 [N, K], one row per
  output channel) plus ``<prefix>.weight_scale`` (F32 [N]), the names
  ``W8Linear`` registers, so a model's ``state_dict`` names the file's tensors;
* an fp checkpoint (F32 / F16 / BF16 weights) loads into int8 layers by
  per-output-channel quantization on the GPU: the per-token quantizer run over
  weight rows, s[n] = amax_k |w[n,k]| / 127 (1 for a zero row),
  q[n,k] = clamp(rint(w[n,k] / s[n]), -127, 127);
* ``quantize_checkpoint`` rewrites an fp checkpoint in the int8 format once,
  offline, so later loads move int8 bytes only.

Parsing, dtype conversion and the host-to-device copies run in
libtensor_ops_rocm.so (``open_safetensors`` and the ``pio_safetensors_*``
entry points); quantization runs on the GPU. Nothing here computes on the CPU
beyond the format's own element conversions.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from . import ops
from .backend import Tensor
from .ops import RocmError, check, lib

# Stored dtype codes of pio_safetensors_info, in enum order.
ST_DTYPES = ("F64", "F32", "F16", "BF16", "I64", "I32", "I16", "I8", "U8", "BOOL", "U16", "U32",
             "U64")
# numpy dtype of each stored element (BF16 as its raw 16-bit pattern).
ST_NUMPY = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16,
            "I64": np.int64, "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8,
            "BOOL": np.bool_, "U16": np.uint16, "U32": np.uint32, "U64": np.uint64}
FLOAT_DTYPES = ("F32", "F16", "BF16")
SCALE_SUFFIX = "_scale"
FORMAT_NOTE = ("int8 per-output-channel symmetric: <name> I8 [N,K], <name>_scale F32 [N], "
               "w ~= q * scale[n]")


@dataclass(frozen=True)
class TensorInfo:
    dtype: str
    shape: Tuple[int, ...]
    nbytes: int


class SafetensorsFile:
    """One mapped safetensors file (``open_safetensors`` .. ``close_safetensors``)."""

    def __init__(self, path):
        self.path = os.fspath(path)
        self._ctx = lib.open_safetensors(os.fsencode(self.path))
        if not self._ctx:
            raise RocmError(f"open_safetensors({self.path}): {ops.last_error()}")

    # ------------------------------------------------------------ lifetime
    def close(self) -> None:
        if getattr(self, "_ctx", None):
            lib.close_safetensors(self._ctx)
            self._ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:   # interpreter shutdown: the library may already be gone
            pass

    def _c(self):
        if not self._ctx:
            raise ValueError(f"{self.path} is closed")
        return self._ctx

    # ------------------------------------------------------------- queries
    def names(self) -> List[str]:
        c = self._c()
        return [lib.pio_safetensors_name(c, i).decode() for i in range(lib.pio_safetensors_count(c))]

    def __contains__(self, name: str) -> bool:
        return lib.pio_safetensors_info(self._c(), name.encode(), None, None, 0, None, None) == 0

    def info(self, name: str) -> TensorInfo:
        dt, nd, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        shape = (ctypes.c_int64 * 16)()
        check(lib.pio_safetensors_info(self._c(), name.encode(), ctypes.byref(dt), shape, 16,
                                       ctypes.byref(nd), ctypes.byref(nb)), "pio_safetensors_info")
        if nd.value > 16:
            raise RocmError(f"{name}: rank {nd.value} exceeds 16")
        return TensorInfo(ST_DTYPES[dt.value], tuple(shape[i] for i in range(nd.value)), nb.value)

    # --------------------------------------------------------------- reads
    def read(self, name: str) -> np.ndarray:
        """Stored elements as numpy (BF16 as uint16 bit patterns)."""
        inf = self.info(name)
        out = np.empty(inf.shape, dtype=ST_NUMPY[inf.dtype])
        check(lib.pio_safetensors_read(self._c(), name.encode(), out.ctypes.data, inf.nbytes),
              "pio_safetensors_read")
        return out

    def read_f32(self, name: str) -> np.ndarray:
        """fp32 values through the reference entry point ``load_tensor_data``."""
        inf = self.info(name)
        out = np.empty(inf.shape, dtype=np.float32)
        n = int(out.size)
        if n >= 2 ** 31:
            raise RocmError(f"{name}: {n} elements exceed load_tensor_data's int size")
        if not lib.load_tensor_data(self._c(), name.encode(),
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n):
            raise RocmError(f"load_tensor_data({name}): {ops.last_error()}")
        return out

    def to_device(self, name: str, ptr: int, nbytes: int, stream=None) -> None:
        """Stored bytes into device memory at ``ptr`` (e.g. a row slice)."""
        check(lib.pio_safetensors_to_device(self._c(), name.encode(), ptr, nbytes, stream),
              f"pio_safetensors_to_device({name})")

    def to_device_f32(self, name: str, ptr: int, count: int, stream=None) -> None:
        """fp32 values into device memory at ``ptr``, converted on the GPU."""
        check(lib.pio_safetensors_to_device_f32(self._c(), name.encode(), ptr, count, stream),
              f"pio_safetensors_to_device_f32({name})")

    def load_into(self, name: str, t: Tensor) -> None:
        """Stored tensor into ``t`` (same shape): raw bytes for matching int8 /
        fp16 / fp32 storage, fp32 conversion (on the GPU) otherwise."""
        inf = self.info(name)
        if tuple(inf.shape) != tuple(t.shape):
            raise RocmError(f"{name}: checkpoint shape {inf.shape} != tensor shape {t.shape}")
        if t.device == "cpu":
            if t.dtype == "int8" and inf.dtype in ("I8", "U8"):
                t.load(self.read(name).view(np.int8))
            elif t.dtype == "float16" and inf.dtype == "F16":
                t.load(self.read(name))
            elif t.dtype == "float32":
                t.load(self.read_f32(name))
            else:
                raise RocmError(f"{name}: cannot load {inf.dtype} into a {t.dtype} tensor")
            return
        check(lib.tensor_load_safetensors_status(self._c(), name.encode(), t._handle),
              f"tensor_load_safetensors({name})")


def checkpoint_files(model_path) -> List[str]:
    """The safetensors files of a checkpoint: the file itself, the shards named
    by ``model.safetensors.index.json``, or ``model.safetensors`` (the search
    order of model_loader.py:95-110)."""
    p = os.fspath(model_path)
    if os.path.isfile(p):
        return [p]
    index = os.path.join(p, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f).get("weight_map", {})
        return [os.path.join(p, n) for n in sorted(set(wm.values()))]
    single = os.path.join(p, "model.safetensors")
    return [single] if os.path.exists(single) else []


class Checkpoint:
    """All files of a (possibly sharded) checkpoint behind one name table."""

    def __init__(self, model_path):
        files = checkpoint_files(model_path)
        if not files:
            raise RocmError(f"no .safetensors files at {model_path}")
        self.files: List[SafetensorsFile] = []
        self._where: Dict[str, SafetensorsFile] = {}
        try:
            for fp in files:
                f = SafetensorsFile(fp)
                self.files.append(f)
                for n in f.names():
                    if n in self._where:
                        raise RocmError(f"{n} is in both {self._where[n].path} and {fp}")
                    self._where[n] = f
        except Exception:
            self.close()
            raise

    def close(self) -> None:
        for f in getattr(self, "files", []):
            f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self) -> List[str]:
        return list(self._where)

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def _f(self, name: str) -> SafetensorsFile:
        f = self._where.get(name)
        if f is None:
            raise RocmError(f"checkpoint has no tensor '{name}'")
        return f

    def info(self, name: str) -> TensorInfo:
        return self._f(name).info(name)

    def read(self, name: str) -> np.ndarray:
        return self._f(name).read(name)

    def read_f32(self, name: str) -> np.ndarray:
        return self._f(name).read_f32(name)

    def load_into(self, name: str, t: Tensor) -> None:
        self._f(name).load_into(name, t)

    def to_device(self, name: str, ptr: int, nbytes: int, stream=None) -> None:
        self._f(name).to_device(name, ptr, nbytes, stream)

    def to_device_f32(self, name: str, ptr: int, count: int, stream=None) -> None:
        self._f(name).to_device_f32(name, ptr, count, stream)


# ------------------------------------------------------------------ int8 weights
def quantize_rows(w: Tensor, q: Tensor, s: Tensor) -> None:
    """Per-row symmetric int8 quantization of a device fp weight [N, K] into
    q (int8 [N, K]) and s (fp32 [N]) on the GPU."""
    check(lib.tensor_quantize_per_token_status(w._handle, q._handle, s._handle),
          "tensor_quantize_per_token")


def _staging(inf: TensorInfo, device: str) -> Tensor:
    return Tensor(list(inf.shape), device=device,
                  dtype="float16" if inf.dtype == "F16" else "float32")


def load_int8_weight(src, name: str, weight: Tensor, scale: Tensor,
                     scale_name: Optional[str] = None) -> None:
    """Fill an int8 weight [N, K] and its fp32 scales [N] from ``src`` (a
    SafetensorsFile or Checkpoint): I8 data plus ``<name>_scale`` load as
    stored; F32 / F16 / BF16 data is quantized per output channel on the GPU."""
    inf = src.info(name)
    if weight.dtype != "int8" or scale.dtype != "float32":
        raise RocmError(f"{name}: needs an int8 weight and an fp32 scale tensor")
    if inf.dtype in ("I8",):
        sn = scale_name or name + SCALE_SUFFIX
        if sn not in src:
            raise RocmError(f"{name} is stored int8 but '{sn}' is missing")
        src.load_into(name, weight)
        src.load_into(sn, scale)
    elif inf.dtype in FLOAT_DTYPES:
        if tuple(inf.shape) != tuple(weight.shape) or len(inf.shape) != 2:
            raise RocmError(f"{name}: checkpoint shape {inf.shape} != weight shape {weight.shape}")
        if weight.device == "cpu":
            raise RocmError(f"{name}: fp weights quantize on the GPU; the int8 weight is on the host")
        tmp = _staging(inf, weight.device)
        src.load_into(name, tmp)
        quantize_rows(tmp, weight, scale)
    else:
        raise RocmError(f"{name}: stored dtype {inf.dtype} is neither int8 nor floating point")


def _load_file(f: SafetensorsFile, model_layers: Dict[str, Tensor]) -> List[str]:
    loaded, filled = [], set()
    for name, t in model_layers.items():
        if t is None or name in filled or name not in f:
            continue
        inf = f.info(name)
        if t.dtype == "int8" and inf.dtype in FLOAT_DTYPES:
            sn = name + SCALE_SUFFIX
            s = model_layers.get(sn)
            if s is None:
                raise RocmError(f"{name}: an fp checkpoint tensor for an int8 parameter needs "
                                f"'{sn}' in the model")
            load_int8_weight(f, name, t, s)
            filled.add(sn)
            loaded += [name, sn]
        else:
            f.load_into(name, t)
            loaded.append(name)
    return loaded


def load_safetensors(filepath, model_layers: Dict[str, Tensor]) -> bool:
    """Drop-in for backend.py:812-835: load every tensor of ``model_layers``
    the file holds; False when the file is missing or cannot be opened, names
    the file lacks are left as they are. int8 parameters take I8 data with its
    ``_scale`` partner, or fp data quantized on the GPU. Unlike the reference,
    a shape or dtype mismatch raises instead of being skipped."""
    if not os.path.exists(os.fspath(filepath)):
        return False
    try:
        f = SafetensorsFile(filepath)
    except RocmError:
        return False
    with f:
        _load_file(f, model_layers)
    return True


def load_weights(model, model_path, device: str = "rocm:0", strict: bool = False) -> List[str]:
    """Counterpart of CustomModelLoader.load_weights (model_loader.py:77-123):
    fills ``model.state_dict()`` from every safetensors file of the checkpoint
    and returns the names loaded. ``strict`` raises if a parameter was not
    found in any file. ``device`` is kept for signature parity; tensors load
    where they live."""
    state = model.state_dict()
    files = checkpoint_files(model_path)
    if not files:
        raise RocmError(f"no .safetensors files at {model_path}")
    loaded: List[str] = []
    for fp in files:
        with SafetensorsFile(fp) as f:
            loaded += _load_file(f, state)
    if strict:
        missing = sorted(set(state) - set(loaded))
        if missing:
            raise RocmError(f"parameters missing from the checkpoint: {missing[:8]}"
                            + (" ..." if len(missing) > 8 else ""))
    return loaded


# --------------------------------------------------------- offline conversion
def default_select(name: str, info: TensorInfo) -> bool:
    """Which fp tensors become int8: 2-D ``*.weight`` matrices other than
    embeddings and norms (the linears, lm_head included)."""
    return (info.dtype in FLOAT_DTYPES and len(info.shape) == 2 and name.endswith(".weight")
            and "embed" not in name and "norm" not in name)


def _header(entries: Sequence[Tuple[str, str, Tuple[int, ...], int]], metadata: dict) -> bytes:
    hdr, off = {}, 0
    for name, dt, shape, nb in entries:
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + nb]}
        off += nb
    hdr["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(hdr, separators=(",", ":")).encode()
    return h + b" " * (-len(h) % 8)


_NUMPY_ST = {np.dtype(v).str: k for k, v in ST_NUMPY.items() if k not in ("BF16",)}


def save_safetensors(path, tensors: Dict[str, np.ndarray], dtypes: Optional[Dict[str, str]] = None,
                     metadata: Optional[dict] = None) -> None:
    """Write host arrays as a safetensors file (names in the given order).
    ``dtypes`` overrides the stored dtype per name, e.g. ``"BF16"`` for a
    uint16 array of bfloat16 bit patterns. An int8 linear saved with its
    ``_scale`` partner is the int8 format ``load_safetensors`` reads."""
    dtypes = dtypes or {}
    entries, arrays = [], []
    for name, a in tensors.items():
        a = np.asarray(a)
        if not a.flags.c_contiguous:   # (ascontiguousarray would make 0-d arrays 1-d)
            a = a.copy(order="C")
        dt = dtypes.get(name) or _NUMPY_ST.get(a.dtype.str)
        if dt is None or np.dtype(ST_NUMPY[dt]) != a.dtype:
            raise ValueError(f"{name}: cannot store a {a.dtype} array as {dt}")
        entries.append((name, dt, a.shape, a.nbytes))
        arrays.append(a)
    meta = {"format": "pt"}
    meta.update(metadata or {})
    hdr = _header(entries, meta)
    tmp = os.fspath(path) + ".tmp"
    try:
        with open(tmp, "wb") as out:
            out.write(struct.pack("<Q", len(hdr)))
            out.write(hdr)
            for a in arrays:
                a.tofile(out)
        os.replace(tmp, os.fspath(path))
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise


def quantize_checkpoint(src_path, dst_path, select: Callable[[str, TensorInfo], bool] = None,
                        device: str = "rocm:0", metadata: Optional[dict] = None) -> List[str]:
    """Write ``src_path`` (a file or checkpoint directory) as one int8
    safetensors file at ``dst_path``: each selected fp weight becomes
    ``<name>`` I8 [N, K] + ``<name>_scale`` F32 [N], quantized on the GPU;
    every other tensor is copied byte for byte. Returns the quantized names."""
    select = select or default_select
    meta = {"format": "pt", "quantization": FORMAT_NOTE}
    meta.update(metadata or {})
    with Checkpoint(src_path) as ck:
        plan, entries = [], []
        for name in ck.names():
            inf = ck.info(name)
            if select(name, inf):
                if inf.dtype not in FLOAT_DTYPES or len(inf.shape) != 2:
                    raise RocmError(f"{name}: only 2-D fp tensors can be quantized ({inf})")
                n, k = inf.shape
                plan.append((name, True))
                entries += [(name, "I8", (n, k), n * k), (name + SCALE_SUFFIX, "F32", (n,), 4 * n)]
            else:
                plan.append((name, False))
                entries.append((name, inf.dtype, inf.shape, inf.nbytes))
        names = [e[0] for e in entries]
        if len(set(names)) != len(names):
            raise RocmError("a quantized weight's _scale name collides with a checkpoint tensor")
        hdr = _header(entries, meta)
        tmp = os.fspath(dst_path) + ".tmp"
        quantized = []
        try:
            _write_quantized(ck, plan, hdr, tmp, device, quantized)
            os.replace(tmp, os.fspath(dst_path))
        except BaseException:
            if os.path.exists(tmp):
                os.remove(tmp)
            raise
    return quantized


def _write_quantized(ck, plan, hdr: bytes, tmp: str, device: str, quantized: List[str]) -> None:
    """Header, then each planned tensor in order: quantized ones as int8 rows
    followed by their fp32 scales (quantized on the GPU), the rest as stored."""
    with open(tmp, "wb") as out:
        out.write(struct.pack("<Q", len(hdr)))
        out.write(hdr)
        for name, quant in plan:
            if quant:
                inf = ck.info(name)
                q = Tensor(list(inf.shape), device=device, dtype="int8")
                s = Tensor([inf.shape[0]], device=device)
                load_int8_weight(ck, name, q, s)
                out.write(q.numpy().tobytes())
                out.write(s.numpy().tobytes())
                quantized.append(name)
            else:
                out.write(ck.read(name).tobytes())


def quantize_array(w: np.ndarray, device: str = "rocm:0") -> Tuple[np.ndarray, np.ndarray]:
    """Per-output-channel int8 quantization of a host fp weight [N, K] on the
    GPU; returns host (q int8 [N, K], s fp32 [N])."""
    w = np.ascontiguousarray(w)
    if w.ndim != 2:
        raise ValueError("quantize_array: weight must be 2-D")
    if w.dtype not in (np.float32, np.float16):
        w = w.astype(np.float32)
    t = Tensor.from_numpy(w, device)
    q = Tensor(list(w.shape), device=device, dtype="int8")
    s = Tensor([w.shape[0]], device=device)
    quantize_rows(t, q, s)
    return q.numpy(), s.numpy()


def iter_int8_pairs(names: Iterable[str]) -> List[str]:
    """Names whose ``_scale`` partner is also present (the int8 linears of a file)."""
    ns = set(names)
    return sorted(n for n in ns if n + SCALE_SUFFIX in ns)
