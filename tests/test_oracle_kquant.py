"""The k-quant oracle against the reference's own bytes (golden vectors written by
tests/golden/make_golden.py from coldpress/kquant.py), plus layout invariants."""
import numpy as np
import pytest

from oracle import kquant_oracle as K


def _cases(golden):
    for key in golden.files:
        if key.startswith("raw/"):
            _, name, qn, tt = key.split("/")
            yield key, name, qn, tt


def test_golden_bytes_and_recon(golden):
    n_checked = 0
    for key, name, qn, tt in _cases(golden):
        x = golden[f"x/{name}"]
        qw = None if qn == "ref" else golden[f"qw/{name}/{qn}"]
        with np.errstate(all="ignore"):
            raw = K.QUANTIZE[tt](x, qw)
        assert np.array_equal(raw, golden[key]), key
        rk = f"rec/{name}/{qn}/{tt}"
        if rk in golden.files:
            with np.errstate(all="ignore"):
                rec = K.DEQUANTIZE[tt](golden[key], x.shape[1])
            assert np.array_equal(rec.view(np.uint32), golden[rk].view(np.uint32)), rk
        n_checked += 1
    assert n_checked == 3 * 3 * 6


@pytest.mark.parametrize("tag,args", [
    ("qkx_q2ref", ("x16", "abs", 3, -0.5, 0.1, 15, True, False)),
    ("qkx_q2imp", ("x16", "w16", 3, -0.9, 0.05, 36, False, True)),
    ("qkx_q4ref", ("x32", "w32", 15, -1.0, 0.1, 20, False, False)),
    ("qkx_q4imp", ("x32", "w32", 15, -0.9, 0.05, 36, False, True)),
])
def test_golden_affine_fit(golden, tag, args):
    xk, wk, *rest = args
    x = golden[f"fit/{xk}"]
    w = np.abs(x) if wk == "abs" else golden[f"fit/{wk}"]
    s, m, L = K.fit_affine(x, w, *rest)
    assert np.array_equal(s, golden[f"fit/{tag}/scale"])
    assert np.array_equal(m, golden[f"fit/{tag}/min"])
    assert np.array_equal(L, golden[f"fit/{tag}/L"])


def test_golden_signed_and_nonneg_fits(golden):
    x16, w16 = golden["fit/x16"], golden["fit/w16"]
    for tag, w, nm in [("qx4w", w16, 4), ("qx32", None, 32), ("qx32w", w16, 32)]:
        s, L = K.fit_signed(x16, w, nm)
        assert np.array_equal(s, golden[f"fit/{tag}/scale"]) and np.array_equal(L, golden[f"fit/{tag}/L"])
    s, L = K.fit_signed_descent(x16, 4)
    assert np.array_equal(s, golden["fit/q3/scale"]) and np.array_equal(L, golden["fit/q3/L"])
    for tag, nm in [("qp15", 15), ("qp63", 63)]:
        d, L = K.fit_nonneg(np.abs(x16), w16, nm)
        assert np.array_equal(d, golden[f"fit/{tag}/d"]) and np.array_equal(L, golden[f"fit/{tag}/L"])


def test_rint_magic_closed_form():
    v = np.array([0.5, 1.5, 2.5, -1.5, -0.5, 3.49999, -7.5, 4194303.0], np.float32)
    assert K.rint_magic(v).tolist() == [0, 2, 2, -2, 0, 3, -8, 4194303]
    # numpy's own round-half-even agrees everywhere below 2**22
    rng = np.random.default_rng(0)
    r = (rng.standard_normal(200000) * 1000).astype(np.float32)
    assert np.array_equal(K.rint_magic(r), np.rint(r).astype(np.int32))
    special = np.array([np.inf, -np.inf, np.nan, 1e30], np.float32)
    assert K.rint_magic(special).tolist() == [-4194304, -4194304, 0, 651978]


def test_half_round_is_ieee_rne():
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(10000) * s for s in (1e-8, 1e-5, 1, 1e4, 1e5)])
    v = v.astype(np.float32)
    assert np.array_equal(K.half_round(v), v.astype(np.float16).astype(np.float32))
    assert np.isinf(K.half_round(np.float32(65520.0)))
    assert K.half_round(np.float32(65519.0)) == 65504.0


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_code_layouts_roundtrip(tt):
    rng = np.random.default_rng(2)
    NB = 7
    if tt in ("Q2_K",):
        L = rng.integers(0, 4, (NB, 256))
        assert np.array_equal(K.unpack_2bit(K.pack_2bit(L)), L)
    elif tt == "Q3_K":
        L = rng.integers(0, 8, (NB, 256))
        h, q = K.pack_q3_codes(L)
        assert np.array_equal(K.unpack_q3_codes(h, q) + 4, L)
        s = rng.integers(0, 64, (NB, 16))
        assert np.array_equal(K.unpack_scales_q3(K.pack_scales_q3(s)), s)
    elif tt in ("Q4_K", "Q5_K"):
        L = rng.integers(0, 16, (NB, 256))
        assert np.array_equal(K.unpack_nibbles(K.pack_nibbles(L)), L)
        s, m = rng.integers(0, 64, (NB, 8)), rng.integers(0, 64, (NB, 8))
        s2, m2 = K.unpack_scales_k4(K.pack_scales_k4(s, m))
        assert np.array_equal(s2, s) and np.array_equal(m2, m)
    else:
        L = rng.integers(0, 64, (NB, 256))
        assert np.array_equal(K.unpack_q6_codes(*K.pack_q6_codes(L)), L)


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_roundtrip_error_is_small(tt):
    from conftest import heavy_tailed
    x = heavy_tailed(4, 512, seed=3)
    rec = K.roundtrip(x, tt)
    rel = np.linalg.norm(rec - x) / np.linalg.norm(x)
    assert rel < {"Q2_K": 0.6, "Q3_K": 0.35, "Q4_K": 0.2, "Q5_K": 0.1, "Q6_K": 0.05}[tt]


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_linear_form_reproduces_the_decoder(golden, tt):
    """scale_tune.py's guarantee (:81-83): d (x) A - dmin (x) B in float32 equals the
    decoder's values, here on every golden container of the type; A and B are
    integers within the int16-exact ranges the reference stores them in."""
    for key in golden.files:
        if not key.startswith("raw/") or not key.endswith("/" + tt):
            continue
        raw = golden[key]
        n = golden[f"x/{key.split('/')[1]}"].shape[1]
        d, dmin, A, B = K.linear_parts(raw, tt, n)
        with np.errstate(all="ignore"):
            W = K.linear_reconstruct(d, dmin, A, B)
            ref = K.DEQUANTIZE[tt](raw, n)
        # equal as values (the reference states it with np.array_equal); bit patterns differ
        # only in the sign of zeros: d*(sc*q) takes d's sign where q = 0, (d*sc)*q d*sc's
        # (the edge block whose fp16 scale overflows gives NaN = inf * 0 in both forms)
        with np.errstate(all="ignore"):
            assert np.array_equal(W, ref, equal_nan=True), key
        diff = W.view(np.uint32) != ref.view(np.uint32)
        assert np.all(W[diff] == 0), key
        assert np.array_equal(A, np.round(A)) and np.abs(A).max() <= 4096
        assert (B is None) == (tt in ("Q3_K", "Q6_K"))
        if B is not None:
            assert np.array_equal(B, np.round(B)) and B.min() >= 0 and B.max() <= 63
