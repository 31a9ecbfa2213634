"""GPU side of the Hessian storage and the GGUF driver: cp_h2_pack / cp_h2_expand
bit-identical to the storage oracle, save_hessians / load_hessian files in the reference's
format, the shared-input Hessian dedup, and encode_gguf end to end on a synthetic artifact
(the reference's test_encode_integration.py, restated) with per-tensor parity."""
import numpy as np
import pytest
import torch

from conftest import correlated_hessian, heavy_tailed
from oracle import ef_oracle as E
from oracle import hess_oracle as Ho
from oracle import kquant_oracle as K

pytestmark = pytest.mark.gpu
F32 = np.float32


def _say(msg):
    print(msg, flush=True)


def _cases():
    rng = np.random.default_rng(1)
    A = rng.standard_normal((96, 96)).astype(F32)
    yield "psd", (A @ A.T + 96 * np.eye(96)).astype(F32)
    X = rng.standard_normal((3000, 80)).astype(F32)
    X[:, :3] *= 90.0
    yield "scaled", (X.T @ X).astype(F32)
    S = (rng.standard_normal((40, 40)) * 1e-6).astype(F32)   # float16 subnormals
    S[3, 5] = -0.0
    yield "tiny", S
    yield "ragged", rng.standard_normal((33, 33)).astype(F32) * 70000


@pytest.mark.parametrize("case", ["psd", "scaled", "tiny", "ragged"])
def test_pack_and_expand_bit_identical(case):
    from perm_amd import _lib, hessians as hs
    H = dict(_cases())[case]
    _say(f"h2 {case} {H.shape}")
    H16, d32, sc = hs.pack_hessian(H)
    w16, wd, ws = Ho.h2_pack(H)
    assert np.array_equal(H16.cpu().numpy().view(np.uint16), w16.view(np.uint16))
    assert np.array_equal(d32.cpu().numpy(), wd) and sc.item() == float(ws)
    lib = _lib.load()
    n = H.shape[0]
    out = torch.empty((n, n), dtype=torch.float64, device="cuda")
    _lib.check(lib.cp_h2_expand(_lib.ptr(H16), 1, n, float(ws), _lib.ptr(d32), _lib.ptr(out),
                                _lib.stream_ptr()))
    assert np.array_equal(out.cpu().numpy(), Ho.h2_expand(w16, ws, wd))


@pytest.mark.parametrize("offset", [0, 1])
def test_pack_large_and_misaligned(offset):
    """max |H| over more entries than the reduction grid covers in one sweep (each block
    strides), with the extreme planted near the end; the input 16-byte aligned and 4 bytes
    off (the 4-byte-load path). Same bytes as the storage oracle."""
    from perm_amd import hessians as hs
    d = 3000
    rng = np.random.default_rng(5)
    H = (rng.standard_normal((d, d)) * 100).astype(F32)
    H[d - 1, d - 3] = -123456.0
    _say(f"h2 pack d={d} offset={offset}")
    buf = torch.empty(d * d + 4, dtype=torch.float32, device="cuda")
    view = buf[offset:offset + d * d].view(d, d)
    view.copy_(torch.from_numpy(H))
    assert (view.data_ptr() % 16 == 0) == (offset == 0)
    H16, d32, sc = hs.pack_hessian(view)
    w16, wd, ws = Ho.h2_pack(H)
    assert float(ws) == 123456.0 / 32768.0 and sc.item() == float(ws)
    assert np.array_equal(H16.cpu().numpy().view(np.uint16), w16.view(np.uint16))
    assert np.array_equal(d32.cpu().numpy(), wd)


def test_hessian_files(tmp_path):
    from perm_amd import hessians as hs
    H = dict(_cases())["scaled"]
    hs.save_hessians({"blk.0.attn_q.weight": {"H": H, "n": 777}}, str(tmp_path))
    with np.load(str(tmp_path / "blk_0_attn_q_weight.npz")) as z:
        w16, wd, ws = Ho.h2_pack(H)
        assert sorted(z.files) == ["H", "diag32", "hscale", "n", "name"]
        assert np.array_equal(z["H"].view(np.uint16), w16.view(np.uint16))
        assert np.array_equal(z["diag32"], wd) and z["hscale"] == ws and int(z["n"]) == 777
        assert str(z["name"]) == "blk.0.attn_q.weight"
    Hr, n = hs.load_hessian(str(tmp_path), "blk.0.attn_q.weight")
    assert n == 777 and np.array_equal(Hr, Ho.h2_expand(w16, ws, wd))
    # the older float32-only file, and the family-keyed fallback (blk.0.qkv_in for attn_k)
    old = dict(_cases())["psd"]
    np.savez_compressed(str(tmp_path / "blk_0_qkv_in.npz"), H=old, n=42, name="x")
    Hk, nk = hs.load_hessian(str(tmp_path), "blk.0.attn_k.weight")
    assert nk == 42 and np.array_equal(Hk, old.astype(np.float64))
    assert hs.has_hessian(str(tmp_path), "blk.0.attn_v.weight")
    assert not hs.has_hessian(str(tmp_path), "blk.1.attn_q.weight")
    with pytest.raises(FileNotFoundError):
        hs.load_hessian(str(tmp_path), "blk.3.ffn_down.weight")
    Hd, _ = hs.load_hessian(str(tmp_path), "blk.0.attn_q.weight", device="cuda")
    assert Hd.is_cuda and Hd.dtype == torch.float64


def test_shared_input_hessians_are_formed_once():
    """q/k/v read one input tensor: one accumulator, shared; values equal the per-module
    sums (hessians.py:137-154)."""
    import torch.nn as nn
    from oracle.hess_oracle import accumulate, rel_fro
    from perm_amd import hessians as hs

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q, self.k, self.v = nn.Linear(64, 64), nn.Linear(64, 32), nn.Linear(64, 32)
            self.o = nn.Linear(64, 64)

        def forward(self, x):
            return self.o(self.q(x) + torch.cat([self.k(x), self.v(x)], -1))

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            self.l0, self.l1 = Block(), Block()

        def forward(self, ids):
            x = ids
            return self.l1(self.l0(x))

    torch.manual_seed(0)
    m = M().cuda().eval()
    names = {f"l{i}.{k}": f"blk.{i}.attn_{k}" for i in (0, 1) for k in "qkv"}
    names.update({f"l{i}.o": f"blk.{i}.attn_output" for i in (0, 1)})
    ne0 = {g + ".weight": 64 for g in names.values()}
    batches = [torch.randn(4, 16, 64, device="cuda") for _ in range(3)]
    got, unmapped = hs.collect_hessians(m, batches, ne0, "qwen3", 2, name_map=names,
                                        keep_on_device=True, log=lambda *_: None)
    assert not unmapped
    for i in (0, 1):
        assert got[f"blk.{i}.attn_q.weight"]["H"] is got[f"blk.{i}.attn_k.weight"]["H"]
        assert got[f"blk.{i}.attn_q.weight"]["H"] is got[f"blk.{i}.attn_v.weight"]["H"]
        assert got[f"blk.{i}.attn_q.weight"]["H"] is not got[f"blk.{i}.attn_output.weight"]["H"]
    assert got["blk.0.attn_q.weight"]["H"] is not got["blk.1.attn_q.weight"]["H"]
    want, cnt = accumulate([b.reshape(-1, 64).cpu().numpy() for b in batches])
    assert got["blk.0.attn_k.weight"]["n"] == cnt == 192
    assert rel_fro(got["blk.0.attn_v.weight"]["H"].cpu().numpy(), want) < 1e-5


# (name, ttype, ne0, nrow): the reference integration test's artifact plus Q4_K / Q5_K / Q8_0
SPEC = [("token_embd.weight", "Q6_K", 256, 512), ("output.weight", "Q6_K", 256, 512),
        ("blk.0.attn_q.weight", "Q2_K", 256, 256), ("blk.0.attn_k.weight", "Q3_K", 256, 128),
        ("blk.0.ffn_down.weight", "Q2_K", 512, 256), ("blk.0.ffn_up.weight", "Q4_K", 256, 192),
        ("blk.1.attn_q.weight", "Q5_K", 256, 128), ("blk.1.ffn_gate.weight", "Q8_0", 256, 64)]


def _artifact(tmp_path):
    from perm_amd import hessians as hs
    from perm_amd.gguffile import GGUFWriter, ValueType
    W = {name: heavy_tailed(nrow, ne0, seed=i) for i, (name, tt, ne0, nrow) in enumerate(SPEC)}
    f16, stock, hdir = (str(tmp_path / k) for k in ("f16.gguf", "stock.gguf", "hess"))
    w = GGUFWriter(f16, "qwen3")
    w.add_kv("qwen3.block_count", 2, ValueType.UINT32)
    for name, a in W.items():
        w.add_tensor(name, a.astype(np.float16))
    w.write()
    w = GGUFWriter(stock, "qwen3")
    w.add_kv("qwen3.block_count", 2, ValueType.UINT32)
    for name, tt, ne0, nrow in SPEC:
        w.add_tensor(name, K.QUANTIZE[tt](W[name].astype(np.float16).astype(F32)), tt)
    w.write()
    Hs = {}
    for i, (name, tt, ne0, nrow) in enumerate(SPEC):
        if name in ("token_embd.weight", "blk.1.ffn_gate.weight"):
            continue   # token_embd uses the attn_q diagonal; ffn_gate has no Hessian (wRTN)
        Hs[name] = {"H": correlated_hessian(ne0, 2048, seed=10 + i).astype(F32), "n": 2048}
    # k shares q's input: the same stored matrix
    Hs["blk.0.attn_k.weight"] = Hs["blk.0.attn_q.weight"]
    hs.save_hessians(Hs, hdir)
    return W, f16, stock, hdir


def test_encode_gguf_end_to_end(tmp_path):
    from perm_amd import ef, gates, ggufio, hessians as hs
    W, f16, stock, hdir = _artifact(tmp_path)
    out = str(tmp_path / "coldpress.gguf")
    _say("encode_gguf")
    stats = ef.encode_gguf(f16, stock, hdir, out, log=lambda *_: None)
    rep = gates.byte_parity(out, stock)
    assert rep["passed"] and rep["total_final"] <= rep["total_stock"]
    assert stats["blk.0.attn_q.weight"]["mode"] == "EF"
    assert stats["token_embd.weight"]["mode"] == "wRTN(attn0-diag)"
    assert stats["blk.1.ffn_gate.weight"]["mode"] == "wRTN"
    a = {t.name: np.asarray(t.data) for t in ggufio.GGUFReader(stock).tensors}
    b = {t.name: np.asarray(t.data) for t in ggufio.GGUFReader(out).tensors}
    assert a["blk.0.attn_q.weight"].tobytes() != b["blk.0.attn_q.weight"].tobytes()
    # per-tensor parity with the oracle on the same inputs
    x = {n: W[n].astype(np.float16).astype(F32) for n in W}
    H0, n0 = hs.load_hessian(hdir, "blk.0.attn_q.weight")
    w_embd = (np.diag(H0) / max(n0, 1)).astype(F32)
    assert np.array_equal(b["token_embd.weight"], K.QUANTIZE["Q6_K"](x["token_embd.weight"], w_embd))
    assert np.array_equal(b["blk.1.ffn_gate.weight"], K.QUANTIZE["Q8_0"](x["blk.1.ffn_gate.weight"]))
    for name, tt, ne0, nrow in SPEC:
        if stats[name]["mode"] != "EF":
            continue
        _say(f"EF parity {name} {tt}")
        H, _ = hs.load_hessian(hdir, name)
        want_raw, want_rec = E.ef_encode(x[name], tt, None, H, stable_order=True)
        got = b[name]
        agree = (K.stored_codes(tt, got) == K.stored_codes(tt, want_raw)).mean()
        rec = K.DEQUANTIZE[tt](got, ne0)
        e_gpu, e_ref = E.h_weighted_err(x[name], rec, H), E.h_weighted_err(x[name], want_rec, H)
        assert agree >= 0.999, (name, agree)
        assert abs(e_gpu - e_ref) / e_ref < 1e-3, (name, e_gpu, e_ref)
        base = K.roundtrip(x[name], tt)
        assert e_gpu < E.h_weighted_err(x[name], base, H)   # EF beats the stock encoding
    # the statistic is the reference's unweighted error ratio (ef.py:297-303); EF lowers the
    # H-weighted error, not necessarily this one
    for name, tt, ne0, nrow in SPEC:
        xs = x[name]
        w = np.ones(ne0, F32)   # no imatrix: the stock baseline is the unweighted encoder
        e_base = float((((K.roundtrip(xs, tt) - xs) ** 2) * w).sum())
        e_ours = float((((K.DEQUANTIZE[tt](b[name], ne0) - xs) ** 2) * w).sum())
        # the reference's arithmetic: float32 terms in numpy's order, the ratio in float64
        assert stats[name]["rel_err_vs_stock"] == e_ours / e_base - 1, name
    with open(out + ".efstats.json") as f:
        assert set(__import__("json").load(f)) == {s[0] for s in SPEC}


def test_encode_gguf_independent_of_layer_grouping(tmp_path):
    """The driver's output does not depend on how many layers share one EF pass: one
    layer per pass and the memory-sized default (here every layer in one pass, with the
    identical q/k Hessian files sharing a factorization) write the same bytes."""
    from perm_amd import ef
    _W, f16, stock, hdir = _artifact(tmp_path)
    outs = []
    for lpp in (1, None):
        out = str(tmp_path / f"ef_{lpp}.gguf")
        _say(f"encode_gguf layers_per_pass={lpp}")
        ef.encode_gguf(f16, stock, hdir, out, log=lambda *_: None, layers_per_pass=lpp)
        with open(out, "rb") as f:
            outs.append(f.read())
    assert outs[0] == outs[1]


def test_encode_gguf_with_perms_and_imatrix(tmp_path):
    """PERM-permuted artifact: the imatrix means and Hessians (original order) are moved by
    the space map's input permutation before EF; the result equals encoding the permuted
    weights with permuted statistics directly."""
    from perm_amd import ef, ggufio, hessians as hs
    from perm_amd.gguffile import GGUFWriter
    dims = {"d_model": 256, "d_ffn": 512, "n_layers": 1, "n_heads": 4, "n_kv": 2, "head_dim": 64}
    rng = np.random.default_rng(3)
    perms = {"res": rng.permutation(256), "ffn": [rng.permutation(512)],
             "vo": [[rng.permutation(64) for _ in range(2)]]}
    names = {"blk.0.attn_q.weight": (256, 256, "Q4_K"), "blk.0.ffn_down.weight": (512, 256, "Q2_K")}
    Worig = {n: heavy_tailed(r, c, seed=i) for i, (n, (c, r, t)) in enumerate(names.items())}
    from perm_amd.perm import input_perm
    P = {n: input_perm(n, perms, dims) for n in names}
    Wp = {n: Worig[n][:, P[n]] for n in names}
    f16, stock, hdir, imat, out = (str(tmp_path / k) for k in
                                   ("f.gguf", "s.gguf", "h", "i.gguf", "o.gguf"))
    w = GGUFWriter(f16, "qwen3")
    for n in names:
        w.add_tensor(n, Wp[n].astype(np.float16))
    w.write()
    w = GGUFWriter(stock, "qwen3")
    for n, (c, r, t) in names.items():
        w.add_tensor(n, K.QUANTIZE[t](Wp[n].astype(np.float16).astype(F32)), t)
    w.write()
    Hs, qws = {}, {}
    w = GGUFWriter(imat, "qwen3")
    for i, (n, (c, r, t)) in enumerate(names.items()):
        Hs[n] = {"H": correlated_hessian(c, 2048, seed=20 + i).astype(F32), "n": 2048}
        qws[n] = (np.abs(rng.standard_normal(c)) + 0.1).astype(F32)
        w.add_tensor(n + ".in_sum2", qws[n] * np.float32(4.0))
        w.add_tensor(n + ".counts", np.array([4.0], F32))
    w.write()
    hs.save_hessians(Hs, hdir)
    ef.encode_gguf(f16, stock, hdir, out, imatrix_path=imat, perms=perms, spacemap="qwen3",
                   dims=dims, log=lambda *_: None)
    got = {t.name: np.asarray(t.data) for t in ggufio.GGUFReader(out).tensors}
    means = ggufio.load_imatrix_means(imat)
    for n, (c, r, t) in names.items():
        p = P[n]
        H, _ = hs.load_hessian(hdir, n)
        raw, _ = ef.ef_encode(Wp[n].astype(np.float16).astype(F32), t, means[n][p],
                              H[np.ix_(p, p)])
        assert np.array_equal(got[n], raw), n
