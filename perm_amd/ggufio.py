"""GGUF re-emission, comparison, type maps and imatrix means, with the API of
coldpress/ggufio.py, on this package's own GGUF reader/writer (perm_amd.gguffile).

  reemit(src, dst, replace=None, replace_f32=None)   ggufio.py:45-91
  compare(a_path, b_path)                            ggufio.py:88-102
  load_imatrix_means(path)                           ggufio.py:105-123
  read_typemap(path)                                 ggufio.py:126-137
  read_arch(reader)                                  ggufio.py:38-42

Re-emitting a file without replacements reproduces it byte for byte (same key-values in the
same order and types, same tensor order, offsets and alignment).
"""
import numpy as np

from .gguffile import GGUFReader, GGUFWriter, ValueType


def read_arch(reader):
    f = reader.fields.get("general.architecture")
    return f.value if f is not None else None


def reemit(src, dst, replace=None, replace_f32=None, log=print):
    """Copy src to dst through the writer. replace: {name: uint8 raw bytes} for quantized
    tensors; replace_f32: {name: float32 array or bytes} for F32 tensors (norm gains).
    Sizes and types must match the tensor replaced."""
    r = GGUFReader(src)
    arch = read_arch(r)
    assert arch, "no architecture key"
    w = GGUFWriter(dst, arch, alignment=r.alignment)
    skip = {"GGUF.version", "GGUF.tensor_count", "GGUF.kv_count", "general.architecture"}
    for f in r.fields.values():
        if f.name not in skip:
            w.add_kv(f.name, f.value, f.vtype, f.itype)
    n_replaced = 0
    for t in r.tensors:
        data = np.asarray(t.data)
        if replace and t.name in replace:
            assert data.dtype == np.uint8, f"replace needs a quantized tensor: {t.name}"
            raw = np.asarray(replace[t.name], dtype=np.uint8)
            assert raw.nbytes == t.n_bytes, (t.name, raw.nbytes, t.n_bytes)
            data = raw.reshape(data.shape)
            n_replaced += 1
        if replace_f32 and t.name in replace_f32:
            assert data.dtype == np.float32, f"replace_f32 needs an F32 tensor: {t.name}"
            v = replace_f32[t.name]
            v = np.frombuffer(v if isinstance(v, bytes) else np.asarray(v).tobytes(),
                              dtype=np.float32)
            assert v.nbytes == t.n_bytes, (t.name, v.nbytes, t.n_bytes)
            data = v.reshape(data.shape)
            n_replaced += 1
        w.add_tensor(t.name, data, t.tensor_type)
    w.write()
    log(f"re-emitted {len(r.tensors)} tensors ({n_replaced} replaced) -> {dst}")


def compare(a_path, b_path, log=print):
    """Tensor-level byte comparison + key-value logical comparison."""
    a, b = GGUFReader(a_path), GGUFReader(b_path)
    ta = {t.name: t for t in a.tensors}
    tb = {t.name: t for t in b.tensors}
    assert set(ta) == set(tb)
    bad = [n for n in ta
           if not np.array_equal(np.asarray(ta[n].data).view(np.uint8).reshape(-1),
                                 np.asarray(tb[n].data).view(np.uint8).reshape(-1))]
    ka = {f.name: f.value for f in a.fields.values() if not f.name.startswith("GGUF.")}
    kb = {f.name: f.value for f in b.fields.values() if not f.name.startswith("GGUF.")}
    kv_bad = [k for k in ka if ka.get(k) != kb.get(k)] + [k for k in kb if k not in ka]
    log(f"tensors: {len(ta)} compared, {len(bad)} data mismatches: {bad[:5]}")
    log(f"kv: {len(ka)} vs {len(kb)}, {len(kv_bad)} mismatches: {kv_bad[:5]}")
    return not bad and not kv_bad


def load_imatrix_means(path):
    """{tensor_name: in_sum2 / count, float32 [ne0]} from an imatrix GGUF."""
    r = GGUFReader(path)
    sums, counts = {}, {}
    for t in r.tensors:
        if t.name.endswith(".in_sum2"):
            sums[t.name[:-len(".in_sum2")]] = np.array(t.data, dtype=np.float32)
        elif t.name.endswith(".counts"):
            counts[t.name[:-len(".counts")]] = np.array(t.data, dtype=np.float32)
    means = {}
    for k, s in sums.items():
        cc = float(counts[k].reshape(-1)[0])
        means[k] = (s / np.float32(cc)).astype(np.float32)
    return means


def read_typemap(path):
    """{name: {type, shape (ne order), n_bytes}} for the byte-parity gate."""
    r = GGUFReader(path)
    return {t.name: {"type": t.tensor_type.name, "shape": [int(x) for x in t.shape],
                     "n_bytes": int(t.n_bytes)} for t in r.tensors}


def write_gguf(path, arch, tensors, kv=()):
    """Convenience writer: tensors is an iterable of (name, array, type-or-None); kv of
    (key, value, vtype[, itype])."""
    w = GGUFWriter(path, arch)
    for item in kv:
        w.add_kv(*item)
    for name, arr, tt in tensors:
        w.add_tensor(name, arr, tt)
    w.write()


__all__ = ["reemit", "compare", "load_imatrix_means", "read_typemap", "read_arch", "write_gguf",
           "GGUFReader", "GGUFWriter", "ValueType"]
