"""Safetensors checkpoints: header parsing, sharded index, and tensors uploaded straight to the device.

Reference: packages/core/src/io/safetensor/parser.ts (header and per-tensor checks), sharded.ts
(model.safetensors.index.json), dtypes.ts (dtype table), io/tensor-loaders.ts
(tensorFromSafetensorLayer).

File format: an 8-byte little-endian header length n, n bytes of JSON mapping each tensor name to
{"dtype", "shape", "data_offsets": [begin, end)} (offsets relative to the data area that follows the
header) plus an optional "__metadata__" string map.

One deliberate difference from the reference: BF16 tensors stay bf16.  The reference widens them to
float32 on load (dtypes.ts:17-31, tensor-loaders.ts:33-36) because its dtype system has no bfloat16;
this backend stores bf16 natively, so a 0.6B checkpoint occupies 1.19 GB on the device, not 2.38 GB.
`dtype="float32"` restores the reference behaviour.

Parsing reads only the header; tensor bytes are read when a layer is loaded, through a read-only
memory map, and copied to the device without a host-side conversion.
"""
from __future__ import annotations

import json
import math
import mmap
import os
import struct
from dataclasses import dataclass, field
from typing import Dict, Iterator, Optional, Tuple

import numpy as np

# safetensors dtype -> (bytes per element, numpy dtype of the stored bits, dtype it loads as).
# Reference table: dtypes.ts:11-45.  Here BF16 loads as the native bfloat16 storage dtype and the
# float types without storage on this backend (F16, F64) load widened/narrowed to float32.
SAFETENSORS_DTYPES: Dict[str, Tuple[int, np.dtype, str]] = {
    "F64": (8, np.dtype("<f8"), "float32"),
    "F32": (4, np.dtype("<f4"), "float32"),
    "F16": (2, np.dtype("<f2"), "float32"),
    "BF16": (2, np.dtype("<u2"), "bfloat16"),
    "I64": (8, np.dtype("<i8"), "int64"),   # no int64 storage: loading raises
    "I32": (4, np.dtype("<i4"), "int32"),
    "I16": (2, np.dtype("<i2"), "int16"),
    "I8": (1, np.dtype("i1"), "int8"),
    "U64": (8, np.dtype("<u8"), "uint64"),
    "U32": (4, np.dtype("<u4"), "uint32"),
    "U16": (2, np.dtype("<u2"), "uint16"),
    "U8": (1, np.dtype("u1"), "uint8"),
    "BOOL": (1, np.dtype("u1"), "bool"),
}

# The format caps the JSON header at 100 MB (a guard against hostile length fields).
MAX_HEADER_SIZE = 100 * 1024 * 1024
_LEN_FIELD = struct.Struct("<Q")


def parse_header_size(first8: bytes) -> int:
    """Byte length of the JSON header: the file's first 8 bytes as an unsigned little-endian 64-bit
    integer, at most MAX_HEADER_SIZE."""
    if len(first8) < _LEN_FIELD.size:
        raise ValueError(f"safetensors: {len(first8)} bytes where the 8-byte header length belongs (file too small)")
    (n,) = _LEN_FIELD.unpack_from(first8)
    if n > MAX_HEADER_SIZE:
        raise ValueError(f"safetensors: header length {n} bytes exceeds the format's cap of {MAX_HEADER_SIZE} bytes")
    return n


def _tensor_entry(name: str, entry, data_size: int):
    """(dtype, shape, (begin, end)) of a header entry describing a tensor, checked against the
    format: a known dtype, non-negative integer dims, and a byte range [begin, end) inside the data
    area holding exactly numel * element-size bytes.  None for entries that describe no tensor
    (anything but an object with data_offsets), which are ignored like the reference ignores them."""
    if not isinstance(entry, dict) or "data_offsets" not in entry:
        return None
    st, shape, offs = entry.get("dtype"), entry.get("shape"), entry["data_offsets"]
    if not isinstance(st, str) or st not in SAFETENSORS_DTYPES:
        raise ValueError(f"safetensors: tensor {name!r} has dtype {st!r}, which this loader does not read "
                         f"(it reads {', '.join(SAFETENSORS_DTYPES)})")
    if not isinstance(shape, list) or not all(isinstance(d, int) and d >= 0 for d in shape):
        raise ValueError(f"safetensors: tensor {name!r} has shape {shape!r}; a shape is a list of dims >= 0")
    if not (isinstance(offs, list) and len(offs) == 2 and all(isinstance(o, int) and o >= 0 for o in offs)):
        raise ValueError(f"safetensors: tensor {name!r} has data_offsets {offs!r}; they are [begin, end] byte offsets")
    begin, end = offs
    need = math.prod(shape) * SAFETENSORS_DTYPES[st][0]      # Python ints: no wrap on hostile shapes
    if end - begin != need:
        raise ValueError(f"safetensors: tensor {name!r} ({st}, shape {tuple(shape)}) needs {need} bytes but its "
                         f"data_offsets span {end - begin}")
    if end > data_size:
        raise ValueError(f"safetensors: tensor {name!r} occupies bytes [{begin}, {end}) of a {data_size}-byte "
                         f"data area (the file is truncated or the offsets are wrong)")
    return st, tuple(shape), (begin, end)


@dataclass
class SafetensorLayer:
    """One tensor of a file: name, dtype, shape and where its bytes are (types.ts SafetensorLayer)."""

    name: str
    original_dtype: str          # safetensors dtype string
    dtype: str                   # backend dtype it loads as by default
    shape: Tuple[int, ...]
    file: "SafetensorFile"
    data_offsets: Tuple[int, int]

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def byte_size(self) -> int:
        return self.data_offsets[1] - self.data_offsets[0]

    def numpy(self) -> np.ndarray:
        """The stored elements as a read-only array over the file's memory map (bf16 as uint16 bits)."""
        _, npdt, _ = SAFETENSORS_DTYPES[self.original_dtype]
        begin = self.file.data_offset + self.data_offsets[0]
        return np.frombuffer(self.file.buffer(), dtype=npdt, count=self.numel, offset=begin).reshape(self.shape)


@dataclass
class SafetensorFile:
    path: str
    metadata: Dict[str, str]
    data_offset: int
    layers: Dict[str, SafetensorLayer] = field(default_factory=dict)
    _fh: Optional[object] = None
    _map: Optional[mmap.mmap] = None

    def buffer(self) -> mmap.mmap:
        if self._map is None:
            self._fh = open(self.path, "rb")
            size = os.fstat(self._fh.fileno()).st_size
            self._map = mmap.mmap(self._fh.fileno(), size, access=mmap.ACCESS_READ) if size else None
        return self._map

    def close(self) -> None:
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:   # arrays still view the map: it is released with the last of them
                pass
            self._map = None
        if self._fh is not None:
            self._fh.close()
            self._fh = None


def parse_safetensor_file(path: str) -> SafetensorFile:
    """Reads the header of one .safetensors file (the reference's parser: parser.ts:89-172): the
    8-byte length, the JSON object, its __metadata__ string map, and every tensor entry checked by
    _tensor_entry.  No tensor bytes are read."""
    file_size = os.path.getsize(path)
    with open(path, "rb") as fh:
        n = parse_header_size(fh.read(_LEN_FIELD.size))
        if n == 0:
            raise ValueError("safetensors: empty header (length 0)")
        raw = fh.read(n)
    if len(raw) != n:
        raise ValueError(f"safetensors: the header announces {n} bytes but the file holds {len(raw)} after the "
                         f"length field (incomplete)")
    try:
        header = json.loads(raw.decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise ValueError(f"safetensors: the header is not valid UTF-8 JSON ({e})") from None
    if not isinstance(header, dict):
        raise ValueError(f"safetensors: the header is JSON {type(header).__name__}, not an object")
    meta = header.pop("__metadata__", None)
    if meta is None:
        meta = {}
    if not isinstance(meta, dict) or not all(isinstance(v, str) for v in meta.values()):
        raise ValueError("safetensors: __metadata__ must be an object mapping strings to strings")
    f = SafetensorFile(path=path, metadata={str(k): str(v) for k, v in meta.items()},
                       data_offset=_LEN_FIELD.size + n)
    data_size = file_size - f.data_offset
    for name, entry in header.items():
        t = _tensor_entry(name, entry, data_size)
        if t is not None:
            st, shape, rng = t
            f.layers[name] = SafetensorLayer(name, st, SAFETENSORS_DTYPES[st][2], shape, f, rng)
    return f


class SafetensorGroup:
    """All layers of a single file or of a sharded checkpoint, by name (parser.ts:189-243)."""

    def __init__(self, files: Dict[str, SafetensorFile], layers: Dict[str, SafetensorLayer], sharded: bool,
                 metadata: Dict[str, str], total_size: Optional[int] = None):
        self.files, self.layers, self.sharded = files, layers, sharded
        self.metadata, self.total_size = metadata, total_size

    def get_layer(self, name: str) -> Optional[SafetensorLayer]:
        return self.layers.get(name)

    def has_layer(self, name: str) -> bool:
        return name in self.layers

    def __iter__(self) -> Iterator[str]:
        return iter(self.layers)

    def close(self) -> None:
        for f in self.files.values():
            f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def parse_sharded_index(index_path: str) -> SafetensorGroup:
    """model.safetensors.index.json: {"metadata": {...}, "weight_map": {tensor name: shard file}};
    shards resolved relative to the index (sharded.ts:20-96)."""
    with open(index_path, "rb") as fh:
        try:
            index = json.loads(fh.read().decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise ValueError(f"Invalid index.json: {e}") from None
    wm = index.get("weight_map") if isinstance(index, dict) else None
    if not isinstance(wm, dict):
        raise ValueError("Invalid index.json: weight_map must be an object")
    root = os.path.dirname(os.path.abspath(index_path))
    files = {shard: parse_safetensor_file(os.path.join(root, shard)) for shard in sorted(set(wm.values()))}
    layers = {}
    for name, shard in wm.items():
        layer = files[shard].layers.get(name)
        if layer is None:
            raise ValueError(f"Layer not found in shard {shard}: {name}")
        layers[name] = layer
    meta = index.get("metadata") or {}
    total = meta.get("total_size")
    return SafetensorGroup(files, layers, True, {k: v for k, v in meta.items() if isinstance(v, str)},
                           int(total) if total is not None else None)


def load_safetensor(path: str) -> SafetensorGroup:
    """A .safetensors file, a *.index.json, or a directory holding either (index preferred)."""
    if os.path.isdir(path):
        idx = os.path.join(path, "model.safetensors.index.json")
        path = idx if os.path.exists(idx) else os.path.join(path, "model.safetensors")
    if path.endswith(".json"):
        return parse_sharded_index(path)
    f = parse_safetensor_file(path)
    return SafetensorGroup({f.path: f}, dict(f.layers), False, f.metadata)


def host_array(layer: SafetensorLayer, dtype: Optional[str] = None) -> np.ndarray:
    """The layer's data in the storage type of `dtype` (default: the layer's own load dtype):
    bf16 as uint16 bit patterns (F32/F16 rounded to nearest even), float32 (BF16/F16 widened exactly),
    int32.  A BF16 layer kept as bf16 is a view of the memory map (no copy)."""
    from ..dtypes import bf16_bits_to_f32, f32_to_bf16_bits

    arr = layer.numpy()
    st = layer.original_dtype
    target = dtype or layer.dtype
    if target == "bfloat16":
        if st == "BF16":
            return arr
        if st in ("F32", "F16", "F64"):
            return f32_to_bf16_bits(arr.astype(np.float32)).reshape(arr.shape)
    elif target == "float32":
        if st == "BF16":
            return bf16_bits_to_f32(arr).reshape(arr.shape)
        if st in ("F32", "F16", "F64"):
            return arr.astype(np.float32)
    elif target == "int32" and st in ("I32", "I16", "I8", "U16", "U8", "BOOL"):
        return arr.astype(np.int32)
    raise ValueError(f"safetensors layer {layer.name} ({st}) cannot load as {target}: the HIP backend stores "
                     f"float32, bfloat16 and int32")


def tensor_from_safetensor_layer(layer: SafetensorLayer, dtype: Optional[str] = None):
    """The layer as a device tensor (tensor-loaders.ts:19-52): BF16 as bfloat16 (dtype="float32"
    restores the reference's widening), F32 as float32, F16 widened to float32, I32 as int32."""
    from ..tensor import Tensor

    target = dtype or layer.dtype
    return Tensor(np.ascontiguousarray(host_array(layer, target)), dtype=target)


def save_safetensors(path: str, tensors: Dict[str, np.ndarray], dtypes: Optional[Dict[str, str]] = None,
                     metadata: Optional[Dict[str, str]] = None) -> None:
    """Writes `tensors` (name -> host array) as one .safetensors file.  A uint16 array is stored as
    BF16 bit patterns unless `dtypes` names another safetensors dtype for it; other arrays as their
    own dtype (float32 -> F32, int32 -> I32, ...).  Tensors are laid out back to back in name order
    (the format allows no gaps in the data area) after a JSON header padded with spaces to a
    multiple of 8 bytes."""
    by_numpy = {np.dtype(v[1]).str: k for k, v in SAFETENSORS_DTYPES.items() if k not in ("BF16", "BOOL")}
    header: Dict[str, object] = {}
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    arrays = []
    offset = 0
    for name in sorted(tensors):
        arr = np.ascontiguousarray(tensors[name])
        st = (dtypes or {}).get(name) or ("BF16" if arr.dtype == np.uint16 else by_numpy.get(arr.dtype.str))
        if st not in SAFETENSORS_DTYPES:
            raise ValueError(f"save_safetensors: {name} has dtype {arr.dtype}, which has no safetensors dtype")
        if arr.dtype.itemsize != SAFETENSORS_DTYPES[st][0]:
            raise ValueError(f"save_safetensors: {name} ({arr.dtype}) does not match {st}")
        header[name] = {"dtype": st, "shape": [int(d) for d in arr.shape], "data_offsets": [offset, offset + arr.nbytes]}
        arrays.append(arr)
        offset += arr.nbytes
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * ((-len(text)) % 8)
    with open(path, "wb") as f:
        f.write(_LEN_FIELD.pack(len(text)))
        f.write(text)
        for arr in arrays:
            f.write(arr.tobytes())
