"""GGUF artifact operations of the encode stage, with coldpress/ggufio.py's interface,
on this package's GGUF v3 reader (perm_amd.gguffile):

  reemit(src, dst, replace=None, replace_f32=None)   ggufio.py:45-91
  compare(a_path, b_path)                            ggufio.py:88-102
  load_imatrix_means(path)                           ggufio.py:105-123
  read_typemap(path)                                 ggufio.py:126-137
  read_arch(reader)                                  ggufio.py:38-42

Re-emission never rebuilds a file. A replacement keeps a tensor's type and byte size,
so the output is the source file byte for byte (header, key-values, tensor infos,
alignment padding) with only the replaced tensors' payload ranges overwritten: the
metadata is identical by construction, and a file is re-emitted at copy speed.
"""
import os
import shutil

import numpy as np

from .gguffile import GGUFReader, GGUFWriter, ValueType


class ReemitError(AssertionError):
    """A replacement that does not fit the tensor it replaces (the reference asserts)."""


def read_arch(reader):
    """general.architecture of an open GGUFReader, or None."""
    field = reader.fields.get("general.architecture")
    return None if field is None else field.value


def _payload(tensor, value, want_quantized):
    """The bytes that go into ``tensor``'s range: uint8 container bytes for a block-
    quantized tensor, float32 values (an array or their bytes) for an F32 one."""
    kind = tensor.tensor_type.name
    if want_quantized:
        if tensor.tensor_type.block_weights == 1:
            raise ReemitError(f"{tensor.name}: {kind} is not a block-quantized type; "
                              f"container bytes cannot replace it")
        blob = np.ascontiguousarray(value, dtype=np.uint8).tobytes()
    else:
        if kind != "F32":
            raise ReemitError(f"{tensor.name}: float32 values cannot replace a {kind} tensor")
        blob = value if isinstance(value, (bytes, bytearray)) else \
            np.ascontiguousarray(value, dtype=np.float32).tobytes()
    if len(blob) != tensor.n_bytes:
        raise ReemitError(f"{tensor.name}: {len(blob)} bytes given for a {tensor.n_bytes}-byte "
                          f"{kind} tensor")
    return blob


def reemit(src, dst, replace=None, replace_f32=None, log=print):
    """Write dst as src with some tensors' data replaced. replace: {name: container bytes}
    for block-quantized tensors; replace_f32: {name: float32 array or bytes} for F32
    tensors (norm gains). Each replacement must have the tensor's exact byte size. Names
    that are not tensors of src are ignored (and counted in the log line), as the
    reference's re-emit, which walks the source's tensors, ignores them."""
    reader = GGUFReader(src)
    if not read_arch(reader):
        raise ReemitError(f"{src}: no general.architecture key")
    ranges = {t.name: t for t in reader.tensors}
    edits, ignored = [], 0
    for table, quantized in ((replace or {}, True), (replace_f32 or {}, False)):
        for name, value in table.items():
            if name not in ranges:
                ignored += 1
                continue
            edits.append((ranges[name].data_offset, _payload(ranges[name], value, quantized)))
    del reader, ranges  # release the map before the copy
    if os.path.abspath(src) != os.path.abspath(dst):
        shutil.copyfile(src, dst)
    with open(dst, "r+b") as f:
        for offset, blob in sorted(edits):
            f.seek(offset)
            f.write(blob)
    log(f"reemit: {src} -> {dst}, {len(edits)} tensor payload(s) replaced"
        + (f", {ignored} name(s) not in the source ignored" if ignored else ""))


def _kv_table(reader):
    """Key-values without the header's pseudo-fields: name -> value."""
    return {f.name: f.value for f in reader.fields.values() if not f.name.startswith("GGUF.")}


def compare(a_path, b_path, log=print):
    """True when the two files hold the same tensors with identical bytes and the same
    key-values. The tensor name sets must match (AssertionError otherwise)."""
    ra, rb = GGUFReader(a_path), GGUFReader(b_path)
    ta = {t.name: t for t in ra.tensors}
    tb = {t.name: t for t in rb.tensors}
    if set(ta) != set(tb):
        raise AssertionError(f"tensor sets differ: {sorted(set(ta) ^ set(tb))[:4]}")
    differ = [name for name, t in ta.items()
              if t.n_bytes != tb[name].n_bytes
              or not np.array_equal(np.asarray(t.data).reshape(-1).view(np.uint8),
                                    np.asarray(tb[name].data).reshape(-1).view(np.uint8))]
    ka, kb = _kv_table(ra), _kv_table(rb)
    kv_differ = sorted(k for k in set(ka) | set(kb) if ka.get(k) != kb.get(k))
    log(f"compare: {len(differ)} of {len(ta)} tensors differ {differ[:5]}; "
        f"{len(kv_differ)} of {len(set(ka) | set(kb))} keys differ {kv_differ[:5]}")
    return not differ and not kv_differ


def load_imatrix_means(path):
    """{tensor name: float32 [ne0]} importance vectors from an imatrix GGUF: each
    ``<name>.in_sum2`` (the per-column sum of squared activations) divided by the
    count stored in ``<name>.counts``, in float32 -- the qw of the weighted encoders."""
    tensors = {t.name: t for t in GGUFReader(path).tensors}
    means = {}
    for name, t in tensors.items():
        base, _, kind = name.rpartition(".")
        if kind != "in_sum2":
            continue
        count = np.float32(np.asarray(tensors[base + ".counts"].data, np.float32).reshape(-1)[0])
        means[base] = np.asarray(t.data, dtype=np.float32) / count
    return means


def read_typemap(path):
    """{name: {"type": ggml type name, "shape": ne order, "n_bytes": payload size}} of
    every tensor, the description the byte-parity gate compares."""
    out = {}
    for t in GGUFReader(path).tensors:
        out[t.name] = dict(type=t.tensor_type.name, shape=list(map(int, t.shape)),
                           n_bytes=int(t.n_bytes))
    return out


__all__ = ["reemit", "compare", "load_imatrix_means", "read_typemap", "read_arch",
           "ReemitError", "GGUFReader", "GGUFWriter", "ValueType"]
