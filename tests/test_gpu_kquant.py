"""GPU k-quant codec parity: bit-exact bytes and reconstructions against the
reference's golden vectors and against the oracle on seeded inputs."""
import numpy as np
import pytest
import torch

from conftest import CODEC_TYPES, heavy_tailed
from oracle import kquant_oracle as K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def kq():
    from perm_amd import kquant
    return kquant


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("tt", CODEC_TYPES)
def test_golden_bytes(golden, kq, tt):
    for name in ("heavy", "linear", "edge"):
        x = golden[f"x/{name}"]
        for qn in ("ref", "imat", "imatz"):
            _say(f"golden {tt} {name} {qn} {x.shape}")
            qw = None if qn == "ref" else golden[f"qw/{name}/{qn}"]
            raw = kq.QUANTIZE[tt](x, qw)
            want = golden[f"raw/{name}/{qn}/{tt}"]
            bad = np.nonzero((raw != want).any(1))[0]
            assert bad.size == 0, f"{tt}/{name}/{qn}: rows {bad[:8]} differ"
            rk = f"rec/{name}/{qn}/{tt}"
            if rk in golden.files:
                rec = kq.DEQUANTIZE[tt](want, x.shape[1])
                assert np.array_equal(rec.view(np.uint32), golden[rk].view(np.uint32))


@pytest.mark.parametrize("tt", CODEC_TYPES)
@pytest.mark.parametrize("weighted", [False, True])
def test_matches_oracle_seeded(kq, tt, weighted):
    nrow, n = 48, 2048
    _say(f"seeded {tt} weighted={weighted} [{nrow},{n}]")
    x = heavy_tailed(nrow, n, seed=21)
    x[3] *= 1e-4                       # small rows -> fp16 subnormal scales
    x[5, :512] = 0.0                   # dead superblocks
    qw = np.abs(heavy_tailed(1, n, seed=22))[0] + 1e-3 if weighted else None
    with np.errstate(all="ignore"):
        want = K.QUANTIZE[tt](x, qw)
    got = kq.QUANTIZE[tt](x, qw)
    assert np.array_equal(got, want)
    rec = kq.DEQUANTIZE[tt](want, n)
    with np.errstate(all="ignore"):
        assert np.array_equal(rec.view(np.uint32), K.DEQUANTIZE[tt](want, n).view(np.uint32))


@pytest.mark.parametrize("tt", CODEC_TYPES)
def test_empty_tensors_behave_like_the_reference(kq, tt):
    """Zero rows: the reference's encoders fail in their final reshape(nrow, -1) with
    ValueError (the oracle restates it and fails alike); its decoders return an empty
    [0, n] float32 array. Numpy and device inputs both."""
    x = np.zeros((0, 256), np.float32)
    with pytest.raises(ValueError):
        K.QUANTIZE[tt](x, None)
    with pytest.raises(ValueError):
        kq.QUANTIZE[tt](x, None)
    with pytest.raises(ValueError):
        kq.QUANTIZE[tt](torch.zeros((0, 256), device="cuda"), None)
    raw = np.zeros((0, kq.row_bytes(tt, 256)), np.uint8)
    want = K.DEQUANTIZE[tt](raw, 256)
    got = kq.DEQUANTIZE[tt](raw, 256)
    assert want.shape == got.shape == (0, 256) and got.dtype == want.dtype == np.float32
    gd = kq.DEQUANTIZE[tt](torch.from_numpy(raw).cuda(), 256)
    assert gd.is_cuda and tuple(gd.shape) == (0, 256)


@pytest.mark.parametrize("tt", CODEC_TYPES)
def test_ragged_superblock_counts(kq, tt):
    """Superblock counts that leave partial waves (1, 3, 5, 7, 9 superblocks)."""
    for nrow, n in [(1, 256), (3, 256), (1, 1280), (7, 256), (3, 768)]:
        _say(f"ragged {tt} [{nrow},{n}]")
        x = heavy_tailed(nrow, n, seed=nrow * 1000 + n)
        qw = np.abs(heavy_tailed(1, n, seed=5))[0] + 1e-3
        for q in (None, qw):
            with np.errstate(all="ignore"):
                want = K.QUANTIZE[tt](x, q)
            assert np.array_equal(kq.QUANTIZE[tt](x, q), want)


def test_q8_0_rows_of_whole_blocks(kq):
    """Q8_0 rows need only whole 32-weight blocks: row lengths that leave a wave's
    8-block chunk partly filled (odd and even block counts), the overflow-free
    extremes of the scale, and ties at half a step."""
    for nrow, n in [(1, 32), (3, 96), (5, 160), (2, 224), (7, 288), (1, 4096 + 32)]:
        _say(f"Q8_0 [{nrow},{n}]")
        x = heavy_tailed(nrow, n, seed=nrow * 100 + n)
        want = K.QUANTIZE["Q8_0"](x)
        assert np.array_equal(kq.QUANTIZE["Q8_0"](x), want)
        rec = kq.DEQUANTIZE["Q8_0"](want, n)
        assert np.array_equal(rec.view(np.uint32), K.DEQUANTIZE["Q8_0"](want, n).view(np.uint32))
    x = np.zeros((4, 64), np.float32)
    x[0, :32] = np.float32(1e-38) * np.arange(32)     # 1/d overflows: the reference stores 0 codes
    x[1, :32] = np.arange(32) - 15.5                    # d = 1: codes on exact half-steps
    x[1, 0] = 127.0
    x[2, :32] = 65504.0 * 127                          # fp16 scale at its maximum
    x[2, 32:] = -1e30                                  # scale overflows fp16
    x[3] = -0.0
    with np.errstate(all="ignore"):
        want = K.QUANTIZE["Q8_0"](x)
    assert np.array_equal(kq.QUANTIZE["Q8_0"](x), want)
    with pytest.raises(ValueError):
        kq.QUANTIZE["Q8_0"](np.zeros((2, 48), np.float32))


def test_device_tensors_stay_on_device(kq):
    x = torch.from_numpy(heavy_tailed(16, 1024, seed=1)).cuda()
    raw = kq.QUANTIZE["Q2_K"](x, None)
    assert raw.is_cuda and raw.dtype == torch.uint8 and raw.shape == (16, 4 * 84)
    rec = kq.DEQUANTIZE["Q2_K"](raw, 1024)
    assert rec.is_cuda and rec.shape == (16, 1024)
    want = K.QUANTIZE["Q2_K"](x.cpu().numpy())
    assert np.array_equal(raw.cpu().numpy(), want)


def test_shape_errors(kq):
    with pytest.raises(AssertionError):
        kq.QUANTIZE["Q2_K"](np.zeros((2, 300), np.float32))
    with pytest.raises(ValueError):
        kq.QUANTIZE["Q4_K"](np.zeros((2, 300), np.float32))
    with pytest.raises(KeyError):
        kq.QUANTIZE["Q9_K"]


def test_full_size_roundtrip_properties(kq):
    """Full Qwen3-0.6B gate_proj shape (3072 x 1024): decode(encode(x)) is within the
    grid of every superblock, and a second encode of the reconstruction is stable
    in the codes where the grid is unchanged (idempotence on exact grid points)."""
    rng = np.random.default_rng(0)
    x = torch.from_numpy((rng.standard_normal((3072, 1024)) * 0.02).astype(np.float32)).cuda()
    qw = torch.from_numpy(np.abs(rng.standard_normal(1024)).astype(np.float32) + 0.1).cuda()
    for tt in CODEC_TYPES:
        _say(f"full-size {tt}")
        raw = kq.QUANTIZE[tt](x, qw)
        rec = kq.DEQUANTIZE[tt](raw, 1024)
        assert torch.isfinite(rec).all()
        rel = (torch.linalg.norm(rec - x) / torch.linalg.norm(x)).item()
        assert rel < {"Q2_K": 0.6, "Q3_K": 0.35, "Q4_K": 0.2, "Q5_K": 0.1, "Q6_K": 0.05,
                      "Q8_0": 0.01}[tt]
        # oracle parity on a row slice of the same tensor
        sl = slice(1000, 1032)
        want = K.QUANTIZE[tt](x[sl].cpu().numpy(), qw.cpu().numpy())
        assert np.array_equal(raw[sl].cpu().numpy(), want)
