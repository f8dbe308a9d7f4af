"""GGUF v3 files without gguf-py: a reader that memory-maps the tensor data and a writer that streams it.

The reference's host tools read and write GGUF through llama.cpp's gguf-py (`gguf.GGUFReader`, `gguf.GGUFWriter`,
`gguf.GGML_QUANT_SIZES`; tools/requant_experts.py:220-272, 280-293, 476-500). This module restates the file format
itself so the requant driver runs with numpy alone:

    magic "GGUF" | u32 version (3) | u64 tensor count | u64 key/value count
    key/value:   string key | u32 value type | value          (string = u64 length + UTF-8 bytes)
    tensor info: string name | u32 n_dims | u64 ne[n_dims] (ne0 first) | u32 ggml type | u64 offset
    padding to the alignment (general.alignment, default 32), then the tensors, each at an aligned offset from there

Metadata is kept as the file's own encoded bytes, so a copied key/value is re-emitted bit for bit (value types,
array element types and float bit patterns included).
"""
import mmap
import os
import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32

# value types of the key/value section
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# ggml tensor types: id -> (name, weights a block, bytes a block) (ggml.h's enum ggml_type and its type traits)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
    39: ("MXFP4", 32, 17),
}
TYPE_BY_NAME = {v[0]: k for k, v in GGML_TYPES.items()}


def type_name(t):
    return GGML_TYPES[t][0] if t in GGML_TYPES else "type%d" % t


def row_bytes(t, ne0):
    """bytes of one row of ne0 weights in ggml type t (ValueError when ne0 is not a whole number of blocks)"""
    if t not in GGML_TYPES:
        raise ValueError("unknown ggml type %d" % t)
    _, bs, ts = GGML_TYPES[t]
    if ne0 % bs:
        raise ValueError("%d weights are not whole %s blocks of %d" % (ne0, type_name(t), bs))
    return ne0 // bs * ts


def tensor_bytes(t, shape):
    n_rows = 1
    for d in shape[1:]:
        n_rows *= int(d)
    return row_bytes(t, int(shape[0])) * n_rows


def _align(n, a):
    return (n + a - 1) // a * a


# ---- encoding -------------------------------------------------------------------------------------------------

def _enc_str(s):
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _enc_value(vtype, value, sub=None):
    if vtype == STRING:
        return _enc_str(value)
    if vtype == ARRAY:
        if sub is None:
            raise ValueError("an array needs its element type")
        items = list(value)
        return struct.pack("<IQ", sub, len(items)) + b"".join(_enc_value(sub, v) for v in items)
    if vtype not in _SCALAR:
        raise ValueError("unknown GGUF value type %d" % vtype)
    return struct.pack(_SCALAR[vtype], value)


def encode_kv(key, vtype, value, sub=None):
    """one key/value entry as the file holds it"""
    return _enc_str(key) + struct.pack("<I", vtype) + _enc_value(vtype, value, sub)


# ---- reading --------------------------------------------------------------------------------------------------

class KV:
    """a key/value entry: its name, value type (array: element type in `sub`), decoded value and encoded bytes"""
    __slots__ = ("name", "type", "sub", "value", "raw")

    def __init__(self, name, vtype, sub, value, raw):
        self.name, self.type, self.sub, self.value, self.raw = name, vtype, sub, value, raw

    def contents(self):
        return self.value


class TensorInfo:
    """a tensor of a GGUF file: name, shape (ne0 first), ggml type, offset in the data section, size; `data` is the
    stored bytes (a read-only uint8 view of the mapped file)"""
    __slots__ = ("name", "shape", "tensor_type", "offset", "n_bytes", "data")

    def __init__(self, name, shape, ttype, offset, n_bytes, data=None):
        self.name, self.shape, self.tensor_type = name, tuple(int(d) for d in shape), ttype
        self.offset, self.n_bytes, self.data = offset, n_bytes, data

    @property
    def n_elements(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def f32(self):
        """the tensor as float32 (stored F32 / F16 / BF16 only; numpy order: ne0 last)"""
        return widen(self.tensor_type, self.data, self.name).reshape(tuple(reversed(self.shape)))


def widen(ttype, raw, name="tensor"):
    """stored F32 / F16 / BF16 bytes as float32, exactly (a flat array)"""
    if ttype == 0:
        return raw.view(np.float32)
    if ttype == 1:
        return raw.view(np.float16).astype(np.float32)
    if ttype == 30:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError("%s is stored as %s, not a float type" % (name, type_name(ttype)))


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if self.pos + n > len(self.buf):
            raise ValueError("GGUF file ends inside its header")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        return bytes(self.take(self.unpack("<Q"))).decode("utf-8")

    def value(self, vtype):
        if vtype == STRING:
            return self.string()
        if vtype == ARRAY:
            sub, n = self.unpack("<I"), self.unpack("<Q")
            if sub in _SCALAR and sub != BOOL:
                fmt = _SCALAR[sub]
                size = struct.calcsize(fmt)
                return np.frombuffer(bytes(self.take(size * n)), dtype=np.dtype(fmt)).tolist()
            return [self.value(sub) for _ in range(n)]
        if vtype not in _SCALAR:
            raise ValueError("unknown GGUF value type %d" % vtype)
        return self.unpack(_SCALAR[vtype])


class GGUFReader:
    """A GGUF file: `fields` (name -> KV, file order), `tensors` (file order), `alignment`, `data_offset`.
    Tensor data stays in the mapped file; nothing is read until it is used."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = memoryview(self._mm)
        c = _Cursor(buf)
        if bytes(c.take(4)) != GGUF_MAGIC:
            raise ValueError("%s is not a GGUF file" % path)
        self.version = c.unpack("<I")
        if self.version not in (2, 3):
            raise ValueError("%s: GGUF version %d is not supported" % (path, self.version))
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        self.fields = {}
        for _ in range(n_kv):
            start = c.pos
            key = c.string()
            vtype = c.unpack("<I")
            sub = None
            if vtype == ARRAY:
                sub = struct.unpack("<I", bytes(buf[c.pos:c.pos + 4]))[0]
            value = c.value(vtype)
            self.fields[key] = KV(key, vtype, sub, value, bytes(buf[start:c.pos]))
        al = self.fields.get("general.alignment")
        self.alignment = int(al.value) if al is not None else DEFAULT_ALIGNMENT
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError("%s: alignment %d is not a power of two" % (path, self.alignment))
        infos = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            shape = [c.unpack("<Q") for _ in range(nd)]
            ttype = c.unpack("<I")
            off = c.unpack("<Q")
            infos.append((name, shape, ttype, off))
        self.data_offset = _align(c.pos, self.alignment)
        size = len(self._mm)
        whole = np.frombuffer(self._mm, dtype=np.uint8)
        self.tensors = []
        for name, shape, ttype, off in infos:
            if ttype not in GGML_TYPES:
                raise ValueError("%s: tensor %s has type %d, which this reader does not know" % (path, name, ttype))
            nb = tensor_bytes(ttype, shape)
            a = self.data_offset + off
            if a + nb > size:
                raise ValueError("%s: tensor %s runs past the end of the file" % (path, name))
            self.tensors.append(TensorInfo(name, shape, ttype, off, nb, whole[a:a + nb]))
        self._by_name = {t.name: t for t in self.tensors}

    def tensor(self, name):
        return self._by_name[name]

    def get(self, key, default=None):
        f = self.fields.get(key)
        return default if f is None else f.value


# ---- writing --------------------------------------------------------------------------------------------------

class GGUFWriter:
    """Writes a GGUF v3 file in three steps, as gguf-py's writer does: key/values and tensor infos are collected,
    `write_header` writes them, then `write_tensor_data` is called once per tensor in the order they were added.

    add_kv(name, type, value[, sub]) encodes a value; add_raw_kv(kv) copies a KV read from another file unchanged.
    Tensors are declared with add_tensor_info(name, shape (ne0 first), ggml type)."""

    def __init__(self, path, alignment=DEFAULT_ALIGNMENT):
        self.path = path
        self.alignment = alignment
        self._kv = []
        self._keys = set()
        self._tensors = []
        self._f = None
        self._next = 0

    def _add(self, name, raw):
        if name in self._keys:
            raise ValueError("duplicate key %s" % name)
        self._keys.add(name)
        self._kv.append(raw)

    def add_kv(self, name, vtype, value, sub=None):
        self._add(name, encode_kv(name, vtype, value, sub))

    def add_raw_kv(self, kv):
        if kv.name == "general.alignment":
            self.alignment = int(kv.value)
        self._add(kv.name, kv.raw)

    def add_tensor_info(self, name, shape, ttype):
        if any(t[0] == name for t in self._tensors):
            raise ValueError("duplicate tensor %s" % name)
        nb = tensor_bytes(ttype, shape)
        off = _align(sum(_align(t[3], self.alignment) for t in self._tensors), self.alignment)
        self._tensors.append((name, tuple(int(d) for d in shape), ttype, nb, off))

    def write_header(self):
        if "general.alignment" not in self._keys and self.alignment != DEFAULT_ALIGNMENT:
            self.add_kv("general.alignment", UINT32, self.alignment)
        self._f = open(self.path, "wb")
        out = [GGUF_MAGIC, struct.pack("<IQQ", GGUF_VERSION, len(self._tensors), len(self._kv))]
        out += self._kv
        for name, shape, ttype, nb, off in self._tensors:
            out.append(_enc_str(name) + struct.pack("<I", len(shape)) +
                       struct.pack("<%dQ" % len(shape), *shape) + struct.pack("<IQ", ttype, off))
        head = b"".join(out)
        self._f.write(head + b"\0" * (_align(len(head), self.alignment) - len(head)))
        self._next = 0

    def write_tensor_data(self, data):
        """the next declared tensor's bytes (any buffer of exactly its size)"""
        if self._f is None:
            raise RuntimeError("write_header first")
        if self._next >= len(self._tensors):
            raise RuntimeError("more tensors written than declared")
        name, shape, ttype, nb, off = self._tensors[self._next]
        mv = memoryview(data).cast("B")
        if mv.nbytes != nb:
            raise ValueError("tensor %s: %d bytes given, %d declared" % (name, mv.nbytes, nb))
        self._f.write(mv)
        self._f.write(b"\0" * (_align(nb, self.alignment) - nb))
        self._next += 1

    def close(self):
        if self._f is not None:
            if self._next != len(self._tensors):
                self._f.close()
                self._f = None
                os.remove(self.path)
                raise RuntimeError("%s: %d of %d tensors written; file removed" % (self.path, self._next,
                                                                                  len(self._tensors)))
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        if exc_type is not None and self._f is not None:
            self._f.close()
            self._f = None
            os.remove(self.path)
            return False
        self.close()
        return False
