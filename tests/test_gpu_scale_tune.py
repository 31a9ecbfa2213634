"""GPU linear form of the k-quant containers (coldpress/scale_tune.py), restating the
reference's test_scale_tune.py: extract_linear reproduces the decoder, an unchanged
write_back is byte-identical, perturbed scales round-trip through fp16 with the codes
fixed, the differentiable reconstruct matches with gradients (here against a float64
evaluation of d(sum W^2)/dd), and build_torch_params reads a GGUF file."""
import numpy as np
import pytest
import torch

from conftest import heavy_tailed
from oracle import kquant_oracle as K

pytestmark = pytest.mark.gpu
TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]
F32 = np.float32


@pytest.fixture(scope="module")
def st():
    from perm_amd import scale_tune
    return scale_tune


@pytest.mark.parametrize("tt", TYPES)
@pytest.mark.parametrize("qw_mode", ["ref", "imatrix"])
def test_extract_linear_exact(st, tt, qw_mode):
    nrow, n = 8, 512
    x = heavy_tailed(nrow, n, seed=len(tt) * 7 + (qw_mode == "ref"))
    qw = None if qw_mode == "ref" else np.abs(heavy_tailed(1, n, seed=3))[0] + 1e-3
    raw = K.QUANTIZE[tt](x, qw)
    lin = st.extract_linear(raw, tt, n)
    d, dmin, A, B = K.linear_parts(raw, tt, n)
    assert np.array_equal(lin["d"], d) and np.array_equal(lin["A"], A)
    assert (lin["dmin"] is None) == (dmin is None)
    if dmin is not None:
        assert np.array_equal(lin["dmin"], dmin) and np.array_equal(lin["B"], B)
    W = st.reconstruct_np(lin)
    assert np.array_equal(W, K.DEQUANTIZE[tt](raw, n))
    assert np.array_equal(W.view(np.uint32), K.linear_reconstruct(d, dmin, A, B).view(np.uint32))


@pytest.mark.parametrize("tt", TYPES)
def test_unchanged_writeback_byte_identical(st, tt):
    raw = K.QUANTIZE[tt](heavy_tailed(8, 512, seed=99), None)
    lin = st.extract_linear(raw, tt, 512)
    assert np.array_equal(st.write_back(raw, tt, lin["d"], lin["dmin"]), raw)


@pytest.mark.parametrize("tt", TYPES)
def test_perturb_roundtrips_fp16_codes_fixed(st, tt):
    raw = K.QUANTIZE[tt](heavy_tailed(8, 512, seed=5), None)
    lin = st.extract_linear(raw, tt, 512)
    d_p = (lin["d"] * F32(1.01)).astype(F32)
    dm_p = (lin["dmin"] * F32(1.02)).astype(F32) if lin["dmin"] is not None else None
    raw_p = st.write_back(raw, tt, d_p, dm_p)
    lin_p = st.extract_linear(raw_p, tt, 512)
    assert np.array_equal(lin_p["d"], K.half_round(d_p))
    if dm_p is not None:
        assert np.array_equal(lin_p["dmin"], K.half_round(dm_p))
        assert np.array_equal(lin_p["B"], lin["B"])
    assert np.array_equal(lin_p["A"], lin["A"])
    assert not np.array_equal(lin_p["d"], lin["d"])
    # the bytes differ from the original only in the scale fields
    bp = K.BYTES_PER_SB[tt]
    changed = np.nonzero((raw_p.reshape(-1, bp) != raw.reshape(-1, bp)).any(0))[0]
    fields = {"Q2_K": {80, 81, 82, 83}, "Q3_K": {108, 109}, "Q4_K": {0, 1, 2, 3},
              "Q5_K": {0, 1, 2, 3}, "Q6_K": {208, 209}}[tt]
    assert set(changed.tolist()) <= fields


@pytest.mark.parametrize("tt", TYPES)
@pytest.mark.parametrize("where", ["cuda", "cpu"])
def test_torch_reconstruct_and_grad(st, tt, where):
    nrow, n = 8, 512
    raw = K.QUANTIZE[tt](heavy_tailed(nrow, n, seed=11), None)
    ref = K.DEQUANTIZE[tt](raw, n)
    lin = st.extract_linear(raw, tt, n)
    entry = {"d": torch.nn.Parameter(torch.from_numpy(lin["d"]).to(where)),
             "dmin": (torch.nn.Parameter(torch.from_numpy(lin["dmin"]).to(where))
                      if lin["dmin"] is not None else None),
             "A": torch.from_numpy(lin["A"].astype(np.int16)),
             "B": torch.from_numpy(lin["B"].astype(np.int16)) if lin["B"] is not None else None,
             "ttype": tt, "shape": lin["shape"]}
    W = st.reconstruct(entry)
    assert np.array_equal(W.detach().cpu().numpy(), ref)
    (W ** 2).sum().backward()
    g = entry["d"].grad
    assert g is not None and g.device.type == where
    Wd = ref.astype(np.float64)
    want = (2 * Wd * lin["A"]).reshape(nrow, -1, 256).sum(-1)
    assert np.allclose(g.cpu().numpy(), want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
    if lin["dmin"] is not None:
        wm = -(2 * Wd * lin["B"]).reshape(nrow, -1, 256).sum(-1)
        gm = entry["dmin"].grad.cpu().numpy()
        assert np.allclose(gm, wm, rtol=1e-5, atol=1e-6 * np.abs(wm).max())
    assert st.reconstruct(entry, dtype=torch.bfloat16).dtype == torch.bfloat16


def test_build_torch_params_on_synthetic_gguf(st, tmp_path):
    from perm_amd.gguffile import GGUFWriter
    nrow, n = 8, 512
    raws = {tt: K.QUANTIZE[tt](heavy_tailed(nrow, n, seed=999 + i), None)
            for i, tt in enumerate(TYPES)}
    path = str(tmp_path / "tiny.gguf")
    w = GGUFWriter(path, "tiny")
    for tt, raw in raws.items():
        w.add_tensor(f"blk.0.{tt}.weight", raw, tt)
    w.add_tensor("blk.0.norm.weight", np.ones(16, F32))
    w.write()
    params = st.build_torch_params(path)
    assert set(params) == {f"blk.0.{tt}.weight" for tt in TYPES}
    for tt, raw in raws.items():
        e = params[f"blk.0.{tt}.weight"]
        assert e["shape"] == (nrow, n) and e["A"].dtype == torch.int16
        assert np.array_equal(st.reconstruct(e).detach().cpu().numpy(), K.DEQUANTIZE[tt](raw, n))


def test_full_size_linear_form(st):
    """Qwen3-0.6B gate_proj (3072 x 1024): the device form reproduces the GPU decoder on
    the whole tensor, and write_back of the extracted scales is the identity."""
    from perm_amd import kquant
    rng = np.random.default_rng(0)
    x = torch.from_numpy((rng.standard_normal((3072, 1024)) * 0.02).astype(F32)).cuda()
    for tt in TYPES:
        raw = kquant.quantize_dev(tt, x)
        lin = st.extract_linear_dev(raw, tt, 1024)
        W = st.reconstruct({**lin, "d": lin["d"], "dmin": lin["dmin"]})
        assert torch.equal(W, kquant.dequantize_dev(tt, raw, 1024))
        assert torch.equal(st.write_back(raw, tt, lin["d"], lin["dmin"]), raw)


@pytest.mark.parametrize("tt", TYPES)
def test_empty_tensor(st, tt):
    """Zero rows: extract, reconstruct and write_back return empty results, as the
    reference's numpy code does on an empty container (the oracle's linear_parts)."""
    raw = np.zeros((0, K.BYTES_PER_SB[tt]), np.uint8)
    d, dmin, A, B = K.linear_parts(raw, tt, 256)
    lin = st.extract_linear(raw, tt, 256)
    assert lin["d"].shape == d.shape == (0, 1) and lin["A"].shape == A.shape == (0, 256)
    assert (lin["dmin"] is None) == (dmin is None) and (lin["B"] is None) == (B is None)
    assert st.reconstruct_np(lin).shape == (0, 256)
    out = st.write_back(raw, tt, np.zeros((0, 1), np.float32),
                        np.zeros((0, 1), np.float32) if dmin is not None else None)
    assert out.shape == raw.shape and out.dtype == np.uint8
