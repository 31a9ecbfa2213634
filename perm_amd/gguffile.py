"""GGUF v3 files: a reader and a writer, with no dependency on the pip ``gguf`` package.

Layout (little-endian throughout):
  header        magic b"GGUF", version u32 (3), tensor count u64, key-value count u64
  key-values    key: string; value type u32; value
  tensor infos  name: string; n_dims u32; ne[n_dims] u64 (ne[0] innermost); ggml type u32;
                offset u64 (from the start of the data section, a multiple of the alignment)
  padding       to the alignment (``general.alignment`` when present, else 32)
  data          each tensor's bytes, padded to the alignment
A string is a u64 byte length and UTF-8 bytes; an array is an item type u32, a count u64 and
the items.

The reader maps the file (numpy memmap) and exposes, per tensor, the same views the
reference's code reads from gguf-py (coldpress/ggufio.py module docstring):
``data`` is [rows..., ne0] of float32 / float16 / bfloat16-as-uint16 for the float types and
uint8 [rows..., row_bytes] for block-quantized ones; ``shape`` is in ne order. The writer
lays a file out the way gguf-py's GGUFWriter does: general.architecture first, then the
key-values in insertion order, tensor infos in insertion order with offsets accumulating
padded sizes, the data section aligned.
"""
import struct
from collections import OrderedDict

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32


class ValueType:
    UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, \
        FLOAT64 = range(13)


_SCALAR = {ValueType.UINT8: "<B", ValueType.INT8: "<b", ValueType.UINT16: "<H",
           ValueType.INT16: "<h", ValueType.UINT32: "<I", ValueType.INT32: "<i",
           ValueType.FLOAT32: "<f", ValueType.BOOL: "<?", ValueType.UINT64: "<Q",
           ValueType.INT64: "<q", ValueType.FLOAT64: "<d"}
_VT_NAMES = {v: k for k, v in vars(ValueType).items() if not k.startswith("_")}


class GGMLType:
    """ggml tensor types: code -> (name, weights per block, bytes per block)."""
    TABLE = {
        0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
        6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36),
        10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144),
        13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
        16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98),
        19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110),
        22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136), 24: ("I8", 1, 1), 25: ("I16", 1, 2),
        26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8), 29: ("IQ1_M", 256, 56),
        30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
    }
    BY_NAME = {v[0]: k for k, v in TABLE.items()}
    # element dtype of the reader's view for the unquantized types
    DTYPE = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "F64": np.float64,
             "I8": np.int8, "I16": np.int16, "I32": np.int32, "I64": np.int64}

    def __init__(self, code):
        if code not in self.TABLE:
            raise ValueError(f"unknown ggml type {code}")
        self.value = code
        self.name, self.block_weights, self.block_bytes = self.TABLE[code]

    @classmethod
    def from_name(cls, name):
        return cls(cls.BY_NAME[name])

    def __eq__(self, other):
        return isinstance(other, GGMLType) and other.value == self.value

    def __hash__(self):
        return hash(self.value)

    def __repr__(self):
        return f"GGMLType.{self.name}"


def pad(n, align):
    return (n + align - 1) // align * align


class Field:
    """One key-value: ``value`` (python scalar, str or list), ``vtype`` and ``itype`` (item
    type of an array, else None)."""
    __slots__ = ("name", "value", "vtype", "itype", "offset")

    def __init__(self, name, value, vtype, itype=None, offset=0):
        self.name, self.value, self.vtype, self.itype, self.offset = name, value, vtype, itype, offset

    def __repr__(self):
        return f"Field({self.name!r}, {_VT_NAMES[self.vtype]})"


class Tensor:
    __slots__ = ("name", "tensor_type", "shape", "n_elements", "n_bytes", "data_offset", "data")

    def __init__(self, name, tensor_type, shape, n_elements, n_bytes, data_offset, data):
        self.name, self.tensor_type, self.shape = name, tensor_type, shape
        self.n_elements, self.n_bytes, self.data_offset, self.data = \
            n_elements, n_bytes, data_offset, data


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        if n > len(self.buf) - self.pos:
            raise ValueError("string runs past the end of the file")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, vtype):
        if vtype == ValueType.STRING:
            return self.string()
        if vtype == ValueType.ARRAY:
            itype = self.take("<I")
            count = self.take("<Q")
            if itype == ValueType.STRING:
                return [self.string() for _ in range(count)], itype
            if itype == ValueType.ARRAY:
                return [self.value(ValueType.ARRAY) for _ in range(count)], itype
            fmt = _SCALAR[itype]
            size = struct.calcsize(fmt)
            arr = np.frombuffer(self.buf, dtype=np.dtype(fmt), count=count, offset=self.pos)
            self.pos += size * count
            out = arr.tolist()
            if itype == ValueType.BOOL:
                out = [bool(v) for v in out]
            return out, itype
        if vtype not in _SCALAR:
            raise ValueError(f"unknown value type {vtype}")
        v = self.take(_SCALAR[vtype])
        return bool(v) if vtype == ValueType.BOOL else v


class GGUFReader:
    """Read a GGUF v2/v3 file. ``fields``: OrderedDict name -> Field, starting with the
    pseudo-fields GGUF.version, GGUF.tensor_count, GGUF.kv_count (as gguf-py lists them);
    ``tensors``: list of Tensor with memory-mapped ``data``."""

    def __init__(self, path, mode="r"):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode=mode)
        buf = memoryview(self.mm)
        cur = _Cursor(buf)
        if bytes(buf[:4]) != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file")
        cur.pos = 4
        version = cur.take("<I")
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version} is not supported")
        n_tensors = cur.take("<Q")
        n_kv = cur.take("<Q")
        self.fields = OrderedDict()
        self.fields["GGUF.version"] = Field("GGUF.version", version, ValueType.UINT32)
        self.fields["GGUF.tensor_count"] = Field("GGUF.tensor_count", n_tensors, ValueType.UINT64)
        self.fields["GGUF.kv_count"] = Field("GGUF.kv_count", n_kv, ValueType.UINT64)
        for _ in range(n_kv):
            off = cur.pos
            key = cur.string()
            vtype = cur.take("<I")
            v = cur.value(vtype)
            if vtype == ValueType.ARRAY:
                val, itype = v
                self.fields[key] = Field(key, val, vtype, itype, off)
            else:
                self.fields[key] = Field(key, v, vtype, None, off)
        align = self.fields.get("general.alignment")
        self.alignment = int(align.value) if align is not None else DEFAULT_ALIGNMENT
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError(f"{path}: alignment {self.alignment} is not a power of two")
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.take("<I")
            ne = [cur.take("<Q") for _ in range(n_dims)]
            ttype = GGMLType(cur.take("<I"))
            offset = cur.take("<Q")
            infos.append((name, ne, ttype, offset))
        self.data_offset = pad(cur.pos, self.alignment)
        self.tensors = []
        for name, ne, ttype, offset in infos:
            n_el = int(np.prod(ne)) if ne else 1
            if ne and ne[0] % ttype.block_weights:
                raise ValueError(f"{name}: ne[0]={ne[0]} is not a multiple of the "
                                 f"{ttype.name} block ({ttype.block_weights})")
            n_bytes = n_el // ttype.block_weights * ttype.block_bytes
            start = self.data_offset + offset
            if start + n_bytes > self.mm.size:
                raise ValueError(f"{name}: data runs past the end of the file")
            outer = tuple(int(v) for v in reversed(ne[1:]))
            if ttype.name in GGMLType.DTYPE:
                dt = GGMLType.DTYPE[ttype.name]
                data = self.mm[start:start + n_bytes].view(dt).reshape(outer + (int(ne[0]),))
            else:
                row = int(ne[0]) // ttype.block_weights * ttype.block_bytes
                data = self.mm[start:start + n_bytes].reshape(outer + (row,))
            self.tensors.append(Tensor(name, ttype, [int(v) for v in ne], n_el, n_bytes, start,
                                       data))


class GGUFWriter:
    """Build a GGUF v3 file. ``add_kv`` in order, ``add_tensor`` in order, then ``write``."""

    def __init__(self, path, arch=None, alignment=None):
        self.path = path
        self.kv = OrderedDict()
        self.tensors = []
        self.alignment = alignment or DEFAULT_ALIGNMENT
        if arch is not None:
            self.add_kv("general.architecture", arch, ValueType.STRING)

    def add_kv(self, key, value, vtype, itype=None):
        if key in self.kv:
            raise KeyError(f"duplicate key {key}")
        if vtype == ValueType.ARRAY and itype is None:
            raise ValueError(f"{key}: an array needs its item type")
        if key == "general.alignment":
            self.alignment = int(value)
        self.kv[key] = (value, vtype, itype)

    def add_tensor(self, name, data, tensor_type=None):
        """data: for a float/int type, the array in its own dtype (shape [rows..., ne0]);
        for a block-quantized type, uint8 [rows..., row_bytes] with ``tensor_type``."""
        a = np.ascontiguousarray(data)
        if tensor_type is None:
            inv = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
                   np.dtype(np.float64): "F64", np.dtype(np.int8): "I8",
                   np.dtype(np.int16): "I16", np.dtype(np.int32): "I32",
                   np.dtype(np.int64): "I64"}
            if a.dtype not in inv:
                raise TypeError(f"{name}: give tensor_type for dtype {a.dtype}")
            tensor_type = inv[a.dtype]
        tt = tensor_type if isinstance(tensor_type, GGMLType) else GGMLType.from_name(tensor_type)
        if tt.name in GGMLType.DTYPE:
            ne = [int(v) for v in reversed(a.shape)] or [1]
            if a.dtype.itemsize != tt.block_bytes:
                raise TypeError(f"{name}: {a.dtype} data for a {tt.name} tensor")
        else:
            if a.dtype != np.uint8 or a.ndim < 1:
                raise TypeError(f"{name}: a {tt.name} tensor takes uint8 [rows..., row_bytes]")
            if a.shape[-1] % tt.block_bytes:
                raise ValueError(f"{name}: row of {a.shape[-1]} bytes is not whole "
                                 f"{tt.name} blocks")
            ne = [a.shape[-1] // tt.block_bytes * tt.block_weights] + \
                [int(v) for v in reversed(a.shape[:-1])]
        if any(t[0] == name for t in self.tensors):
            raise KeyError(f"duplicate tensor {name}")
        self.tensors.append((name, ne, tt, a))

    @staticmethod
    def _string(s):
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _value(self, value, vtype, itype):
        if vtype == ValueType.STRING:
            return self._string(value)
        if vtype == ValueType.ARRAY:
            out = [struct.pack("<IQ", itype, len(value))]
            for v in value:
                out.append(self._value(v, itype, None) if itype != ValueType.ARRAY
                           else self._value(v[0], ValueType.ARRAY, v[1]))
            return b"".join(out)
        return struct.pack(_SCALAR[vtype], value)

    def header_bytes(self):
        """Everything before the data section, padding included."""
        out = [GGUF_MAGIC, struct.pack("<IQQ", GGUF_VERSION, len(self.tensors), len(self.kv))]
        for key, (value, vtype, itype) in self.kv.items():
            out += [self._string(key), struct.pack("<I", vtype), self._value(value, vtype, itype)]
        offset = 0
        for name, ne, tt, a in self.tensors:
            out += [self._string(name), struct.pack("<I", len(ne)),
                    struct.pack(f"<{len(ne)}Q", *ne), struct.pack("<IQ", tt.value, offset)]
            offset += pad(a.nbytes, self.alignment)
        head = b"".join(out)
        return head + b"\0" * (pad(len(head), self.alignment) - len(head))

    def write(self):
        with open(self.path, "wb") as f:
            f.write(self.header_bytes())
            for _name, _ne, _tt, a in self.tensors:
                f.write(a.tobytes())
                f.write(b"\0" * (pad(a.nbytes, self.alignment) - a.nbytes))
