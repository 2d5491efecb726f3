"""GGUF v3 pack restatement: writer, validating reader and payload decoding.

TEST INFRASTRUCTURE ONLY: imported by tests/ and __graft_entry__.smoke() to
check the pack ingestion path against; the shipped library and the measured
path never import it.

What it restates:

* The GGUF v3 container that the reference reads through ggml's gguf parser
  (the ``ggml`` git submodule, github.com/ggml-org/ggml, which is not vendored
  in the reference tree; its pinned commit is not recorded there).  The layout
  follows the published GGUF specification and the reference's own writer,
  ``scripts/convert_pixal3d_to_gguf.py:232-258`` (key/value encoding),
  ``850-919`` (tensor table, offsets, alignment, padding).
* ``load_pack_info`` of ``src/pack.cpp:127-288``: the checks on top of the
  container (version, architecture, name scheme, required keys, component
  list, payload bounds and alignment, tensor-name rules) with the reference's
  messages, and ``read_u32`` / ``read_string`` / the metadata accessors
  (``src/pack.cpp:24-88, 387-462``).
* ``read_tensor_f32`` (``src/slat_flow.cpp:360-395``,
  ``src/slat_decoder.cpp:453-491``): F32 payloads as is, F16 widened exactly,
  BF16 by a 16-bit shift; a non-finite value is an error.

Pinned by ``tests/test_pack.py``: the packs in ``tests/golden/`` were written
by the reference's converter itself; this writer reproduces them byte for
byte and this reader recovers their metadata and tensors; the reference's
``tests/test_pack_reader.cpp`` case (offset 0, byte round trip, missing and
closed-reader errors) holds.  F16 decoding is numpy's IEEE half conversion;
BF16 rounding is checked against torch's.
"""

from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = b"GGUF"
GGML_MAX_DIMS = 4
GGML_MAX_NAME = 64
DEFAULT_ALIGNMENT = 32

# Metadata value types of the GGUF specification.
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STRING, VT_ARRAY, \
    VT_U64, VT_I64, VT_F64 = range(13)
_SCALAR = {VT_U8: "<B", VT_I8: "<b", VT_U16: "<H", VT_I16: "<h", VT_U32: "<I", VT_I32: "<i",
           VT_F32: "<f", VT_U64: "<Q", VT_I64: "<q", VT_F64: "<d"}

# ggml tensor types: id -> (name, block size in elements, bytes per block).
# Sizes are those of the ggml block formats (a block of 32 or 256 values).
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
GGML_TYPES = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20),
    6: ("q5_0", 32, 22), 7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 9: ("q8_1", 32, 36),
    10: ("q2_K", 256, 84), 11: ("q3_K", 256, 110), 12: ("q4_K", 256, 144),
    13: ("q5_K", 256, 176), 14: ("q6_K", 256, 210), 15: ("q8_K", 256, 292),
    24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8),
    28: ("f64", 1, 8), 30: ("bf16", 1, 2),
}


class PackError(RuntimeError):
    """A load failure carrying the reference's message."""


def align(value, alignment):
    return (value + alignment - 1) // alignment * alignment


# --- writer ------------------------------------------------------------------------

def _utf8(value):
    return value.encode("utf-8", errors="surrogateescape")


def gguf_string(value):
    raw = _utf8(value) if isinstance(value, str) else bytes(value)
    return struct.pack("<Q", len(raw)) + raw


def encode_value(vtype, value):
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], value)
    if vtype == VT_BOOL:
        return struct.pack("<B", int(value))
    if vtype == VT_STRING:
        return gguf_string(value)
    if vtype == VT_ARRAY:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(encode_value(etype, v)
                                                               for v in items)
    raise ValueError(f"unknown GGUF value type {vtype}")


def encode_kv(key, vtype, value):
    return gguf_string(key) + struct.pack("<I", vtype) + encode_value(vtype, value)


@dataclass
class Tensor:
    """One tensor table entry: dims in GGUF order (dims[0] innermost)."""
    name: str
    ggml_type: int
    dims: tuple
    payload: bytes
    offset: int | None = None  # override of the computed offset (malformed packs)


def tensor_nbytes(ggml_type, dims):
    _, block, size = GGML_TYPES[ggml_type]
    rows = 1
    for d in dims[1:]:
        rows *= d
    return dims[0] // block * size * rows if dims else size


def pack_bytes(kvs, tensors, alignment=DEFAULT_ALIGNMENT, version=3, magic=GGUF_MAGIC):
    """The file image of a pack: header, key/values (kvs = [(key, vtype,
    value)] in order), tensor table, zero padding to `alignment`, payloads
    each padded to `alignment` (the converter's layout)."""
    header = bytearray(magic) + struct.pack("<I", version)
    header += struct.pack("<QQ", len(tensors), len(kvs))
    for key, vtype, value in kvs:
        header += encode_kv(key, vtype, value)
    offsets, off = [], 0
    for t in tensors:
        offsets.append(off if t.offset is None else t.offset)
        off = align(off + len(t.payload), alignment)
    table = bytearray()
    for t, o in zip(tensors, offsets):
        table += gguf_string(t.name) + struct.pack("<I", len(t.dims))
        for d in t.dims:
            table += struct.pack("<Q", d)
        table += struct.pack("<IQ", t.ggml_type, o)
    out = bytearray(header + table)
    out += b"\0" * (align(len(out), alignment) - len(out))
    for t in tensors:
        out += t.payload
        out += b"\0" * (align(len(t.payload), alignment) - len(t.payload))
    return bytes(out)


def pixal3d_kvs(name="pack", file_type=0, alignment=DEFAULT_ALIGNMENT, components=(),
                extra=()):
    """The general and pixal3d keys a component pack carries
    (scripts/convert_pixal3d_to_gguf.py:692-695, 1094-1098)."""
    kvs = [("general.architecture", VT_STRING, "pixal3d"), ("general.name", VT_STRING, name),
           ("general.file_type", VT_U32, file_type), ("general.alignment", VT_U32, alignment),
           ("pixal3d.bundle_format", VT_U32, 1),
           ("pixal3d.tensor_name_scheme", VT_STRING, "compact-v1"),
           ("pixal3d.bundle_kind", VT_STRING, "component"),
           ("pixal3d.component_count", VT_U32, len(components))]
    kvs += [(f"pixal3d.component.{i}", VT_STRING, c) for i, c in enumerate(components)]
    return kvs + list(extra)


def f32_tensor(name, array, ggml_type=GGML_F32):
    """Tensor entry for a float array stored as F32, F16 or BF16 (the dims
    are the array shape reversed, as the converter writes them)."""
    a = np.ascontiguousarray(array, np.float32)
    if ggml_type == GGML_F32:
        raw = a.astype("<f4").tobytes()
    elif ggml_type == GGML_F16:
        raw = a.astype("<f2").tobytes()
    elif ggml_type == GGML_BF16:
        raw = bf16_bits(a).astype("<u2").tobytes()
    else:
        raise ValueError(ggml_type)
    return Tensor(name, ggml_type, tuple(reversed(a.shape)) or (1,), raw)


# --- reader ------------------------------------------------------------------------

@dataclass
class TensorInfo:
    name: str
    n_dims: int
    ne: tuple
    ggml_type: int
    type_name: str
    n_bytes: int
    offset: int


@dataclass
class PackInfo:
    path: str
    gguf_version: int = 0
    alignment: int = 0
    data_offset: int = 0
    architecture: str = ""
    name: str = ""
    tensor_name_scheme: str = ""
    file_type: int = 0
    bundle_format: int = 0
    components: list = field(default_factory=list)  # (key, stage, model_class, variant)
    tensors: list = field(default_factory=list)
    kv: dict = field(default_factory=dict)  # key -> (vtype, value)

    def tensor(self, name):
        for t in self.tensors:
            if t.name == name:
                return t
        return None


class _Cursor:
    def __init__(self, data):
        self.data, self.pos = data, 0

    def take(self, n):
        if n < 0 or self.pos + n > len(self.data):
            raise EOFError
        out = self.data[self.pos:self.pos + n]
        self.pos += n
        return out

    def unpack(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        # GGUF strings are bytes (ggml does not check their encoding); keep
        # them round-trippable.
        return self.take(self.unpack("<Q")).decode("utf-8", errors="surrogateescape")


def _value(cur, vtype, nested=False):
    if vtype in _SCALAR:
        return cur.unpack(_SCALAR[vtype])
    if vtype == VT_BOOL:
        b = cur.unpack("<B")
        if b > 1:
            raise ValueError("bool")
        return bool(b)
    if vtype == VT_STRING:
        return cur.string()
    if vtype == VT_ARRAY and not nested:
        etype, n = cur.unpack("<I"), cur.unpack("<Q")
        if etype == VT_ARRAY or (etype not in _SCALAR and etype not in (VT_BOOL, VT_STRING)):
            raise ValueError("array type")
        return (etype, [_value(cur, etype, True) for _ in range(n)])
    raise ValueError("value type")


def parse_container(data):
    """The GGUF container as ggml's parser accepts it: returns (version,
    kv dict, tensor list [(name, ne, type, offset)], alignment, data_offset);
    raises ValueError for anything it rejects (bad magic, version 1 or > 3,
    duplicate keys, bad alignment, more than 4 dims, negative or overflowing
    dims, unknown types, a row not a whole number of blocks, names of 64 bytes
    or more, duplicate names, offsets other than the running padded sizes)."""
    cur = _Cursor(data)
    try:
        if cur.take(4) != GGUF_MAGIC:
            raise ValueError("magic")
        version = cur.unpack("<I")
        if version == 1 or version > 3:
            raise ValueError("version")
        n_tensors, n_kv = cur.unpack("<q"), cur.unpack("<q")
        if n_tensors < 0 or n_kv < 0:
            raise ValueError("counts")
        kv = {}
        for _ in range(n_kv):
            key = cur.string()
            vtype = cur.unpack("<I")
            if key in kv:
                raise ValueError("duplicate key")
            kv[key] = (vtype, _value(cur, vtype))
        alignment = DEFAULT_ALIGNMENT
        if "general.alignment" in kv:
            vt, v = kv["general.alignment"]
            if vt != VT_U32 or v == 0 or (v & (v - 1)) != 0:
                raise ValueError("alignment")
            alignment = v
        tensors, names = [], set()
        for _ in range(n_tensors):
            name = cur.string()
            if len(_utf8(name)) >= GGML_MAX_NAME or name in names:
                raise ValueError("name")
            names.add(name)
            n_dims = cur.unpack("<I")
            if n_dims > GGML_MAX_DIMS:
                raise ValueError("dims")
            ne = [cur.unpack("<q") for _ in range(n_dims)] + [1] * (GGML_MAX_DIMS - n_dims)
            if any(d < 0 for d in ne):
                raise ValueError("ne")
            total = 1
            for d in ne:
                total *= d
            if total >= 2 ** 63:
                raise ValueError("overflow")
            gtype = cur.unpack("<I")
            if gtype not in GGML_TYPES or ne[0] % GGML_TYPES[gtype][1] != 0:
                raise ValueError("type")
            offset = cur.unpack("<Q")
            tensors.append((name, tuple(ne), gtype, offset))
        data_offset = align(cur.pos, alignment)
        running = 0
        for name, ne, gtype, offset in tensors:
            if offset != running:
                raise ValueError("offset")
            running += align(tensor_nbytes(gtype, ne), alignment)
    except (EOFError, struct.error):
        raise ValueError("truncated")
    return version, kv, tensors, alignment, data_offset


def _u32(kv, key, required):
    """read_u32 (src/pack.cpp:24-66)."""
    if key not in kv:
        if required:
            raise PackError("missing GGUF metadata: " + key)
        return 0
    vt, v = kv[key]
    if vt in (VT_U8, VT_U16, VT_U32) or (vt in (VT_I8, VT_I16, VT_I32) and v >= 0):
        return int(v)
    raise PackError("GGUF metadata is not a non-negative integer: " + key)


def _string(kv, key, required):
    """read_string (src/pack.cpp:68-88)."""
    if key not in kv:
        if required:
            raise PackError("missing GGUF metadata: " + key)
        return ""
    vt, v = kv[key]
    if vt != VT_STRING:
        raise PackError("GGUF metadata is not a string: " + key)
    return v


def n_dims_of(ne):
    """ggml_n_dims: one past the last dimension above 1, at least 1."""
    for i in range(GGML_MAX_DIMS - 1, 0, -1):
        if ne[i] > 1:
            return i + 1
    return 1


def load_pack_info(path):
    """load_pack_info (src/pack.cpp:127-288)."""
    path = str(path)
    try:
        with open(path, "rb") as f:
            data = f.read()
        version, kv, table, alignment, data_offset = parse_container(data)
    except (OSError, ValueError):
        raise PackError("gguf_init_from_file failed: " + path)
    info = PackInfo(path, version, alignment, data_offset, kv=kv)
    if version != 3:
        raise PackError(f"unsupported GGUF version: {version}")
    info.architecture = _string(kv, "general.architecture", True)
    if info.architecture != "pixal3d":
        raise PackError("unexpected GGUF architecture: " + info.architecture)
    info.name = _string(kv, "general.name", True)
    info.tensor_name_scheme = _string(kv, "pixal3d.tensor_name_scheme", True)
    if info.tensor_name_scheme != "compact-v1":
        raise PackError("unsupported Pixal3D tensor name scheme: " + info.tensor_name_scheme)
    info.file_type = _u32(kv, "general.file_type", True)
    info.bundle_format = _u32(kv, "pixal3d.bundle_format", True)
    i = 0
    while f"pixal3d.component.{i}" in kv:
        key = f"pixal3d.component.{i}"
        vt, value = kv[key]
        if vt != VT_STRING:
            raise PackError("component metadata is not a string: " + key)
        parts = value.split("|")
        if len(parts) >= 3:
            stage, model_class, variant = parts[0], parts[1], "|".join(parts[2:])
        else:
            stage = value
            model_class = _string(kv, f"pixal3d.{value}.model_class", False)
            variant = _string(kv, f"pixal3d.{value}.variant", False)
        info.components.append((value, stage, model_class, variant))
        i += 1
    size = len(data)
    if data_offset > size:
        raise PackError("GGUF tensor data offset is beyond end of file")
    names = set()
    for name, ne, gtype, offset in table:
        if not name or len(_utf8(name)) >= GGML_MAX_NAME or name in names:
            raise PackError("GGUF tensor names must be non-empty, unique, and <64 bytes")
        names.add(name)
        nbytes = tensor_nbytes(gtype, ne)
        if offset > size or nbytes > size - offset or data_offset > size - offset - nbytes:
            raise PackError("GGUF tensor payload is outside the file: " + name)
        if alignment == 0 or offset % alignment != 0:
            raise PackError("GGUF tensor offset is not aligned: " + name)
        nd = n_dims_of(ne)
        info.tensors.append(TensorInfo(name, nd, tuple(ne[d] if d < nd else 1 for d in range(4)),
                                       gtype, GGML_TYPES[gtype][0], nbytes, offset))
    return info


def read_tensor(info, name):
    """Pixal3DPackReader::read_tensor (src/pack.cpp:331-385): the payload bytes."""
    t = info.tensor(name)
    if t is None:
        raise PackError("tensor not found: " + name)
    with open(info.path, "rb") as f:
        f.seek(info.data_offset + t.offset)
        raw = f.read(t.n_bytes)
    if len(raw) != t.n_bytes:
        raise PackError("short read for tensor: " + name)
    return raw


def metadata(info, key, kind, required=True):
    """The metadata accessors (src/pack.cpp:387-462): kind u32, f32, bool or
    string; a missing optional key reads 0 / 0.0 / False / ""."""
    if kind == "u32":
        return _u32(info.kv, key, required)
    if kind == "string":
        return _string(info.kv, key, required)
    vt_want, label, default = {"f32": (VT_F32, "float32", 0.0),
                               "bool": (VT_BOOL, "bool", False)}[kind]
    if key not in info.kv:
        if required:
            raise PackError("missing GGUF metadata: " + key)
        return default
    vt, v = info.kv[key]
    if vt != vt_want:
        raise PackError(f"GGUF metadata is not {label}: " + key)
    return v


def decode_f32(raw, ggml_type):
    """Payload -> float32 values as read_tensor_f32 converts them
    (src/slat_flow.cpp:376-387): F32 as is, F16 widened (exact), BF16 as the
    high half of a float32."""
    if ggml_type == GGML_F32:
        return np.frombuffer(raw, "<f4").astype(np.float32)
    if ggml_type == GGML_F16:
        return np.frombuffer(raw, "<f2").astype(np.float32)
    if ggml_type == GGML_BF16:
        return (np.frombuffer(raw, "<u2").astype(np.uint32) << 16).view(np.float32)
    raise PackError("unsupported tensor type")


def bf16_bits(a):
    """float32 -> bfloat16 bit patterns, round to nearest even (finite inputs;
    NaN keeps a quiet NaN)."""
    bits = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    out = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(a, np.float32))
    out[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def write_pack(path, kvs, tensors, **kw):
    data = pack_bytes(kvs, tensors, **kw)
    tmp = str(path) + ".tmp"
    with open(tmp, "wb") as f:
        f.write(data)
    os.replace(tmp, path)
    return data
