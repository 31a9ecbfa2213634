"""The PERM objective oracle (coldpress/perm/objective.py, qwen3.py optimize) pinned
without the reference: numpy's summation orders against their restatements, the
objective against an exactly rounded evaluation of its formula, identities of the row
sample and the column permutation, closed forms of col_log_rms, and the expectations
of the reference's optimizer test (test_perm_optimize.py:45-61)."""
import math

import numpy as np
import pytest

from conftest import OPT_DIMS, heavy_tailed, small_qwen3_model
from oracle import kquant_oracle as K
from oracle import perm_oracle as Po

F32 = np.float32


def _values(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))) ** 2


def test_pairwise_sum_is_numpys_float64_sum():
    lengths = list(range(0, 300)) + [511, 1023, 1024, 1025, 2048, 3072, 4096, 5000, 14336]
    seq_differs = 0
    for n in lengths:
        a = _values(n, n)
        assert Po.pairwise_sum(a) == float(a.sum()), n
        s = 0.0
        for v in a:
            s += float(v)
        seq_differs += s != float(a.sum())
    assert seq_differs > 50  # a sequential restatement would not pass


def test_axis0_sum_is_a_sequential_chain():
    rng = np.random.default_rng(2)
    d2 = rng.standard_normal((300, 67)) ** 2 * np.exp(rng.uniform(-30, 30, (300, 67)))
    want = np.zeros(67)
    for r in range(300):
        want = want + d2[r]
    assert np.array_equal(d2.sum(0), want)
    pw = np.array([Po.pairwise_sum(d2[:, c]) for c in range(67)])
    assert not np.array_equal(pw, want)  # the order matters on these values


def _exact_err(x, tt, qw, perm, wvec):
    """math.fsum of w[c] * (recon - x)^2 over every element: the formula with one rounding."""
    xs = x[:, perm] if perm is not None else x
    q = (qw[perm] if perm is not None else qw) if qw is not None else None
    with np.errstate(all="ignore"):
        rec = K.roundtrip(np.ascontiguousarray(xs), tt, q)
    d2 = (rec.astype(np.float64) - xs.astype(np.float64)) ** 2
    if wvec is not None:
        w = wvec[perm] if perm is not None else wvec
    elif q is not None:
        w = q.astype(np.float64)
    else:
        w = np.ones(x.shape[1])
    return math.fsum((d2 * w[None, :]).ravel().tolist())


@pytest.mark.parametrize("tt", ["Q2_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"])
def test_tensor_err_formula(tt):
    x = heavy_tailed(24, 512, seed=3)
    rng = np.random.default_rng(4)
    qw = (np.abs(rng.standard_normal(512)) + 0.05).astype(F32)
    wvec = rng.uniform(0.1, 2.0, 512)
    perm = rng.permutation(512)
    for q, p, w in [(None, None, None), (qw, None, None), (qw, perm, None), (None, perm, wvec),
                    (qw, perm, wvec)]:
        got = Po.tensor_err(x, tt, q, perm=p, wvec=w)
        want = _exact_err(x, tt, q, p, w)
        assert abs(got - want) <= 1e-12 * want, (tt, q is None, p is None, w is None)
    # a wrong weight is far outside that bound
    assert abs(Po.tensor_err(x, tt, qw) - _exact_err(x, tt, None, None, None)) > 1e-6 * \
        _exact_err(x, tt, None, None, None)


def test_tensor_err_identities():
    x = heavy_tailed(40, 256, seed=5)
    rng = np.random.default_rng(6)
    qw = (np.abs(rng.standard_normal(256)) + 0.1).astype(F32)
    wvec = rng.uniform(0.5, 1.5, 256)
    p = rng.permutation(256)
    assert Po.tensor_err(x, "Q4_K", qw, perm=p) == Po.tensor_err(x[:, p], "Q4_K", qw[p])
    assert Po.tensor_err(x, "Q3_K", qw, perm=p, wvec=wvec) == \
        Po.tensor_err(x[:, p], "Q3_K", qw[p], wvec=wvec[p])
    # a sample at least as large as the tensor is the whole tensor
    assert Po.tensor_err(x, "Q2_K", qw, rows_sample=40) == Po.tensor_err(x, "Q2_K", qw)
    idx = Po.sample_rows(40, 16, seed=9)
    assert idx.size == 16 and np.all(np.diff(idx) > 0) and idx.min() >= 0 and idx.max() < 40
    assert Po.tensor_err(x, "Q2_K", qw, rows_sample=16, seed=9) == \
        Po.tensor_err(x[idx], "Q2_K", qw)
    for t in ("F16", "F32", "BF16"):
        assert Po.tensor_err(x, t, qw) == 0.0
    with pytest.raises(ValueError):
        Po.tensor_err(x, "Q9_K", qw)
    # float16 weights are read exactly
    xh = x.astype(np.float16)
    assert Po.tensor_err(xh, "Q6_K", None) == Po.tensor_err(xh.astype(F32), "Q6_K", None)


def test_col_log_rms_closed_forms():
    rng = np.random.default_rng(7)
    c = rng.uniform(0.01, 3.0, 48)
    x = np.tile(c.astype(F32), (1000, 1))
    got = Po.col_log_rms(x)
    want = np.log(np.abs(c.astype(F32).astype(np.float64)) + 1e-12)
    assert np.allclose(got, want, rtol=0, atol=1e-12)  # 1000 sequential adds of c^2
    assert np.allclose(Po.col_log_rms(np.zeros((5, 8), F32)), np.log(1e-12), rtol=0, atol=0)
    # chunking changes the rounding of the sums only
    y = heavy_tailed(3000, 64, seed=8)
    a, b = Po.col_log_rms(y), Po.col_log_rms(y, row_step=7)
    assert np.allclose(a, b, rtol=0, atol=1e-13)
    # the chunked float64 sums are the sequential chains per chunk, added in order
    acc = np.zeros(64)
    for r0 in range(0, 3000, 7):
        s = np.zeros(64)
        for r in range(r0, min(r0 + 7, 3000)):
            v = y[r].astype(np.float64)
            s = s + v * v
        acc = acc + s
    assert np.array_equal(b, np.log(np.sqrt(acc / 3000) + 1e-12))


def test_optimize_valid_and_nonworsening():
    w = small_qwen3_model()
    ttypes = {n: "Q2_K" for n in w}
    perms, report = Po.optimize_qwen3(w, ttypes, {}, OPT_DIMS, rows_sample=4096)
    assert np.array_equal(np.sort(perms["res"]), np.arange(256))
    for l in range(2):
        assert np.array_equal(np.sort(perms["ffn"][l]), np.arange(512))
        for h in range(2):
            assert np.array_equal(np.sort(perms["vo"][l][h]), np.arange(64))
    for space in ("res", "ffn", "vo"):
        assert report[space]["rel"] <= 1e-9, (space, report[space])
