"""GGUF v3 reader/writer and ggufio (host code, no GPU), and the Hessian storage oracle.

The file format is pinned by a file assembled byte by byte from the GGUF v3 layout (magic,
version, counts, key-values, tensor infos, alignment padding, data), independently of the
writer; ggufio's behaviour by the reference's own tests (test_ggufio.py: re-emission is
byte-identical, a replaced tensor keeps its type and layout, the type map reads ne order)
and gates.py's byte-parity rules. The storage oracle is pinned by the expectations of
test_hessian_fp16.py."""
import os
import struct

import numpy as np
import pytest

from conftest import heavy_tailed
from oracle import hess_oracle as Ho
from oracle import kquant_oracle as K
from perm_amd import gates
from perm_amd import ggufio
from perm_amd.gguffile import GGMLType, GGUFReader, GGUFWriter, ValueType


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def hand_built(path):
    """A two-tensor GGUF written from the layout itself."""
    q = K.QUANTIZE["Q2_K"](heavy_tailed(2, 256, seed=1))          # [2, 84]
    norm = np.arange(3, dtype=np.float32)
    kv = [(_s("general.architecture") + struct.pack("<I", 8) + _s("qwen3")),
          (_s("qwen3.block_count") + struct.pack("<I", 4) + struct.pack("<I", 2)),
          (_s("tokenizer.ggml.tokens") + struct.pack("<I", 9) + struct.pack("<IQ", 8, 2)
           + _s("a") + _s("bc")),
          (_s("x.eps") + struct.pack("<I", 6) + struct.pack("<f", 1e-6)),
          (_s("x.flag") + struct.pack("<I", 7) + struct.pack("<?", True)),
          (_s("x.ids") + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3)
           + struct.pack("<3i", -1, 0, 7))]
    infos = [(_s("blk.0.weight") + struct.pack("<I", 2) + struct.pack("<2Q", 256, 2)
              + struct.pack("<IQ", 10, 0)),
             (_s("norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 3)
              + struct.pack("<IQ", 0, 192))]   # 168 bytes padded to 192
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv)) + b"".join(kv) + b"".join(infos)
    head += b"\0" * ((-len(head)) % 32)
    data = q.tobytes() + b"\0" * (192 - q.nbytes) + norm.tobytes() + b"\0" * (32 - 12)
    with open(path, "wb") as f:
        f.write(head + data)
    return q, norm


def test_reader_parses_the_layout(tmp_path):
    p = str(tmp_path / "h.gguf")
    q, norm = hand_built(p)
    r = GGUFReader(p)
    vals = {f.name: f.value for f in r.fields.values()}
    assert vals["GGUF.version"] == 3 and vals["GGUF.tensor_count"] == 2
    assert vals["general.architecture"] == "qwen3" and vals["qwen3.block_count"] == 2
    assert vals["tokenizer.ggml.tokens"] == ["a", "bc"] and vals["x.flag"] is True
    assert vals["x.ids"] == [-1, 0, 7] and vals["x.eps"] == float(np.float32(1e-6))
    t0, t1 = r.tensors
    assert t0.tensor_type == GGMLType.from_name("Q2_K") and t0.shape == [256, 2]
    assert t0.n_bytes == 168 and np.array_equal(t0.data, q)
    assert t1.tensor_type.name == "F32" and np.array_equal(t1.data, norm)


def test_writer_reproduces_the_layout(tmp_path):
    p, p2 = str(tmp_path / "h.gguf"), str(tmp_path / "w.gguf")
    q, norm = hand_built(p)
    w = GGUFWriter(p2, "qwen3")
    w.add_kv("qwen3.block_count", 2, ValueType.UINT32)
    w.add_kv("tokenizer.ggml.tokens", ["a", "bc"], ValueType.ARRAY, ValueType.STRING)
    w.add_kv("x.eps", 1e-6, ValueType.FLOAT32)
    w.add_kv("x.flag", True, ValueType.BOOL)
    w.add_kv("x.ids", [-1, 0, 7], ValueType.ARRAY, ValueType.INT32)
    w.add_tensor("blk.0.weight", q, "Q2_K")
    w.add_tensor("norm.weight", norm)
    w.write()
    assert open(p, "rb").read() == open(p2, "rb").read()


def _build(path, seed=1):
    """The reference test's file (test_ggufio.py:11-24) plus more value and tensor types."""
    raw = K.QUANTIZE["Q2_K"](heavy_tailed(8, 512, seed))
    w = GGUFWriter(path, "qwen3")
    w.add_kv("qwen3.block_count", 2, ValueType.UINT32)
    w.add_kv("general.name", "tiny", ValueType.STRING)
    w.add_kv("tokenizer.ggml.tokens", ["a", "b", "c"], ValueType.ARRAY, ValueType.STRING)
    w.add_kv("qwen3.attention.layer_norm_rms_epsilon", 1e-6, ValueType.FLOAT32)
    w.add_kv("some.bool", True, ValueType.BOOL)
    w.add_kv("some.u64", 2 ** 40 + 3, ValueType.UINT64)
    w.add_kv("some.f64", -0.1, ValueType.FLOAT64)
    w.add_kv("some.i8s", [-3, 4], ValueType.ARRAY, ValueType.INT8)
    w.add_tensor("blk.0.weight", raw, "Q2_K")
    w.add_tensor("norm.weight", heavy_tailed(1, 16, 2)[0])
    w.add_tensor("blk.0.f16.weight", heavy_tailed(3, 64, 3).astype(np.float16))
    w.add_tensor("blk.0.q6.weight", K.QUANTIZE["Q6_K"](heavy_tailed(4, 256, 4)), "Q6_K")
    w.add_tensor("blk.0.q8.weight", K.QUANTIZE["Q8_0"](heavy_tailed(5, 96, 5)), "Q8_0")
    w.write()
    return raw


def test_reemit_byte_identical(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    _build(a)
    ggufio.reemit(a, b, log=lambda *_: None)
    assert ggufio.compare(a, b, log=lambda *_: None)
    assert open(a, "rb").read() == open(b, "rb").read()


def test_reemit_replace_quant_tensor(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    _build(a)
    raw2 = K.QUANTIZE["Q2_K"](heavy_tailed(8, 512, 42))
    ggufio.reemit(a, b, replace={"blk.0.weight": raw2.reshape(-1)}, log=lambda *_: None)
    tm = ggufio.read_typemap(b)
    assert tm["blk.0.weight"]["type"] == "Q2_K"
    assert not ggufio.compare(a, b, log=lambda *_: None)
    r = GGUFReader(b)
    assert np.array_equal([t for t in r.tensors if t.name == "blk.0.weight"][0].data, raw2)
    with pytest.raises(AssertionError):
        ggufio.reemit(a, b, replace={"blk.0.weight": raw2.reshape(-1)[:-1]}, log=lambda *_: None)
    with pytest.raises(AssertionError):
        ggufio.reemit(a, b, replace={"norm.weight": np.zeros(64, np.uint8)}, log=lambda *_: None)
    # a superset dict: names that are not tensors of the source are ignored, as the
    # reference's re-emit (which walks the source's tensors) ignores them
    said = []
    ggufio.reemit(a, b, replace={"blk.0.weight": raw2.reshape(-1), "blk.9.absent.weight": raw2},
                  replace_f32={"absent_norm.weight": np.zeros(4, np.float32)}, log=said.append)
    assert np.array_equal([t for t in GGUFReader(b).tensors if t.name == "blk.0.weight"][0].data,
                          raw2)
    assert "1 tensor payload(s) replaced, 2 name(s) not in the source ignored" in said[-1]


def test_reemit_keeps_any_layout_and_touches_only_the_payload(tmp_path):
    """A file laid out unlike gguf-py's writer (the architecture key after others, 64-byte
    alignment): re-emission keeps every byte outside the replaced tensor's range, and that
    range holds the new container bytes."""
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    w = GGUFWriter(a)
    w.add_kv("general.alignment", 64, ValueType.UINT32)
    w.add_kv("general.name", "odd", ValueType.STRING)
    w.add_kv("general.architecture", "llama", ValueType.STRING)
    w.add_tensor("norm.weight", heavy_tailed(1, 48, 3)[0])
    w.add_tensor("blk.0.ffn_down.weight", K.QUANTIZE["Q4_K"](heavy_tailed(3, 512, 4)), "Q4_K")
    w.write()
    new = K.QUANTIZE["Q4_K"](heavy_tailed(3, 512, 5))
    ggufio.reemit(a, b, replace={"blk.0.ffn_down.weight": new}, log=lambda *_: None)
    t = [t for t in GGUFReader(a).tensors if t.name == "blk.0.ffn_down.weight"][0]
    old_bytes, new_bytes = open(a, "rb").read(), open(b, "rb").read()
    lo, hi = t.data_offset, t.data_offset + t.n_bytes
    assert len(old_bytes) == len(new_bytes) and t.data_offset % 64 == 0
    assert old_bytes[:lo] == new_bytes[:lo] and old_bytes[hi:] == new_bytes[hi:]
    assert new_bytes[lo:hi] == new.tobytes()
    assert gates.byte_parity(b, a)["passed"]


def test_reemit_replace_f32(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    _build(a)
    g = np.linspace(0, 1, 16, dtype=np.float32)
    ggufio.reemit(a, b, replace_f32={"norm.weight": g}, log=lambda *_: None)
    r = GGUFReader(b)
    assert np.array_equal([t for t in r.tensors if t.name == "norm.weight"][0].data, g)


def test_typemap(tmp_path):
    a = str(tmp_path / "a.gguf")
    _build(a)
    tm = ggufio.read_typemap(a)
    assert tm["blk.0.weight"]["type"] == "Q2_K" and tm["blk.0.weight"]["shape"] == [512, 8]
    assert tm["blk.0.weight"]["n_bytes"] == 8 * 2 * 84
    assert tm["norm.weight"]["type"] == "F32" and tm["norm.weight"]["shape"] == [16]
    assert tm["blk.0.q8.weight"]["n_bytes"] == 5 * 3 * 34
    assert tm["blk.0.f16.weight"]["type"] == "F16"


def test_imatrix_means(tmp_path):
    p = str(tmp_path / "imat.gguf")
    rng = np.random.default_rng(0)
    s = (rng.random(512) + 0.1).astype(np.float32)
    w = GGUFWriter(p, "qwen3")
    w.add_tensor("blk.0.attn_q.weight.in_sum2", s)
    w.add_tensor("blk.0.attn_q.weight.counts", np.array([100.0], np.float32))
    w.write()
    m = ggufio.load_imatrix_means(p)
    assert np.array_equal(m["blk.0.attn_q.weight"], (s / np.float32(100.0)).astype(np.float32))


def test_byte_parity_gate(tmp_path):
    a, b, c = (str(tmp_path / f"{k}.gguf") for k in "abc")
    _build(a)
    ggufio.reemit(a, b, replace={"blk.0.weight": K.QUANTIZE["Q2_K"](heavy_tailed(8, 512, 9))},
                  log=lambda *_: None)
    rep = gates.byte_parity(b, a)
    assert rep["passed"] and rep["total_final"] == rep["total_stock"]
    w = GGUFWriter(c, "qwen3")   # one tensor at another type
    for t in GGUFReader(a).tensors:
        if t.name == "blk.0.weight":
            w.add_tensor(t.name, K.QUANTIZE["Q4_K"](heavy_tailed(8, 512, 1)), "Q4_K")
        else:
            w.add_tensor(t.name, np.asarray(t.data), t.tensor_type)
    w.write()
    with pytest.raises(gates.GateError):
        gates.byte_parity(c, a)


def test_reader_rejects_bad_files(tmp_path):
    p = str(tmp_path / "bad.gguf")
    with open(p, "wb") as f:
        f.write(b"GGML" + b"\0" * 60)
    with pytest.raises(ValueError):
        GGUFReader(p)
    q = str(tmp_path / "trunc.gguf")
    hand_built(q)
    data = open(q, "rb").read()
    with open(q, "wb") as f:
        f.write(data[:-40])
    with pytest.raises(ValueError):
        GGUFReader(q)


# ---------------------------------------------------------------- storage oracle

def _sym_psd(n, seed):
    rng = np.random.default_rng(seed)
    M = rng.standard_normal((n, n))
    return (M @ M.T).astype(np.float64) + n * np.eye(n)


def test_h2_oracle_unscaled_roundtrip():
    """test_hessian_fp16.py:20-42: exact diagonal; off-diagonal = f16(f32(H)) within eps."""
    n = 128
    H = _sym_psd(n, 0)
    H16, d32, hs = Ho.h2_pack(H.astype(np.float32))
    assert hs == 1.0
    Hr = Ho.h2_expand(H16, hs, d32)
    assert np.array_equal(np.diag(Hr), np.diag(H).astype(np.float32).astype(np.float64))
    off = ~np.eye(n, dtype=bool)
    assert np.array_equal(Hr[off], H.astype(np.float32).astype(np.float16).astype(np.float64)[off])
    eps = np.finfo(np.float16).eps
    assert float(np.max(np.abs(Hr[off] - H[off]) / np.maximum(np.abs(H[off]), 1e-6))) <= eps


def test_h2_oracle_large_hessian_stays_finite():
    """test_hessian_fp16.py:66-90: massive-activation channels push X^T X far past 65504;
    the scale keeps every stored value finite and the round trip close."""
    rng = np.random.default_rng(0)
    X = rng.standard_normal((4000, 96)).astype(np.float32)
    X[:, :4] *= 80.0
    H = (X.T @ X).astype(np.float32)
    assert np.abs(H).max() > 65504
    H16, d32, hs = Ho.h2_pack(H)
    assert hs > 1 and np.isfinite(H16.astype(np.float32)).all()
    assert hs == np.float32(float(np.abs(H).max()) / 32768.0)
    Hr = Ho.h2_expand(H16, hs, d32)
    assert np.array_equal(np.diag(Hr), np.diag(H).astype(np.float64))
    assert np.allclose(Hr, H, rtol=2e-3, atol=float(hs) * 1e-3)


def test_h2_oracle_old_float32_format():
    H = _sym_psd(16, 3).astype(np.float32)
    assert np.array_equal(Ho.h2_expand(H), H.astype(np.float64))


def test_stored_digest_keys_hessian_files_by_content(tmp_path):
    """encode_gguf shares one factorization between tensors whose stored Hessian files
    have the same content; the key comes from the zip members' stored bytes (no
    decompression) and ignores the tensor name. Equal content with another compression
    keys apart (a missed share, never a wrong one); any change in H, diag32, hscale or
    n changes the key; read_stored returns the arrays as written."""
    from perm_amd import hessians as hs
    rng = np.random.default_rng(0)
    H = rng.standard_normal((96, 96)).astype(np.float16)
    dg = rng.standard_normal(96).astype(np.float32)

    def write(name, H=H, dg=dg, hscale=2.0, n=7, compressed=True):
        path = str(tmp_path / f"{name}.npz")
        (np.savez_compressed if compressed else np.savez)(
            path, H=H, diag32=dg, hscale=np.float32(hscale), n=n, name=name)
        return path

    base = hs.stored_digest(write("a"))
    assert hs.stored_digest(write("b")) == base                 # another name, same content
    assert hs.stored_digest(write("c", compressed=False)) != base
    H2 = H.copy()
    H2[5, 7] = np.float16(H2[5, 7] + 1)
    assert hs.stored_digest(write("d", H=H2)) != base
    dg2 = dg.copy()
    dg2[3] += 1
    assert hs.stored_digest(write("e", dg=dg2)) != base
    assert hs.stored_digest(write("f", hscale=3.0)) != base
    assert hs.stored_digest(write("g", n=8)) != base
    Hs, hscale, diag, n = hs.read_stored(str(tmp_path / "a.npz"))
    assert np.array_equal(Hs, H) and hscale == 2.0 and np.array_equal(diag, dg) and n == 7


def test_stored_keys_share_exactly_the_equal_files(tmp_path, monkeypatch):
    """stored_keys (what encode_gguf groups by) gives equal keys exactly to the files whose
    stored bytes are equal, and hashes member data only where two files' zip directories
    (member sizes and CRC-32s) agree."""
    from perm_amd import hessians as hs
    rng = np.random.default_rng(1)
    H = rng.standard_normal((64, 64)).astype(np.float16)
    dg = rng.standard_normal(64).astype(np.float32)

    def write(name, H=H, dg=dg, n=7):
        path = str(tmp_path / f"{name}.npz")
        np.savez_compressed(path, H=H, diag32=dg, hscale=np.float32(2.0), n=n, name=name)
        return path

    H2 = H.copy()
    H2[3, 4] = np.float16(H2[3, 4] + 1)
    same = [write("a"), write("b"), write("c")]
    other = [write("d", H=H2), write("e", n=8), write("f", dg=dg[::-1].copy())]
    hashed = []
    real = hs.stored_digest
    monkeypatch.setattr(hs, "stored_digest", lambda p: hashed.append(p) or real(p))
    keys = hs.stored_keys(same + other)
    assert keys[same[0]] == keys[same[1]] == keys[same[2]]
    assert len({keys[p] for p in same + other}) == 4
    assert sorted(hashed) == sorted(same)  # the three files with one directory, nothing else
    hashed.clear()
    keys = hs.stored_keys(other)
    assert len(set(keys.values())) == 3 and not hashed
