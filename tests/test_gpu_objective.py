"""GPU PERM objective parity: tensor_err / col_log_rms (coldpress/perm/objective.py)
bit-identical to the oracle, the batched form equal to single calls, the space-map
optimizer (qwen3.py:284-355) choosing the oracle's permutations with the oracle's
objective values, and the reference's error behaviour."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import CODEC_TYPES, OPT_DIMS, heavy_tailed, small_qwen3_model
from oracle import perm_oracle as Po

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def ob():
    from perm_amd import objective
    return objective


def _say(msg):
    print(msg, flush=True)


def _variants(n, seed):
    rng = np.random.default_rng(seed)
    qw = (np.abs(rng.standard_normal(n)) + 0.05).astype(F32)
    wvec = rng.uniform(0.1, 2.0, n)
    perm = rng.permutation(n)
    return [dict(), dict(qw=qw), dict(qw=qw, perm=perm), dict(perm=perm, wvec=wvec),
            dict(qw=qw, perm=perm, wvec=wvec), dict(qw=qw, rows_sample=37, seed=5),
            dict(qw=qw, perm=perm, rows_sample=20, seed=11)]


@pytest.mark.parametrize("tt", CODEC_TYPES)
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_tensor_err_bit_identical(ob, tt, dtype):
    x = heavy_tailed(70, 768, seed=31)
    x[4] = 0.0
    if dtype == "f16":
        x = x.astype(np.float16)
    for k, v in enumerate(_variants(768, 7)):
        _say(f"tensor_err {tt} {dtype} variant {k}")
        want = Po.tensor_err(x, tt, v.get("qw"), perm=v.get("perm"), wvec=v.get("wvec"),
                             rows_sample=v.get("rows_sample"), seed=v.get("seed", 0))
        got = ob.tensor_err(x, tt, v.get("qw"), perm=v.get("perm"), wvec=v.get("wvec"),
                            rows_sample=v.get("rows_sample"), seed=v.get("seed", 0))
        assert got == want, (k, got, want)


def _one_tree(v):
    """Pairwise sum of v as one tree (numpy's order only up to 8192 values)."""
    n = len(v)
    if n <= 128:
        r = list(v[:8])
        i = 8
        while i + 8 <= n:
            r = [r[j] + v[i + j] for j in range(8)]
            i += 8
        s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
        for a in v[i:]:
            s = s + a
        return s
    n2 = n // 2
    n2 -= n2 % 8
    return _one_tree(v[:n2]) + _one_tree(v[n2:])


@pytest.mark.parametrize("tt", ["Q4_K", "Q8_0"])
def test_total_over_more_than_8192_columns(ob, tt):
    """numpy sums the weighted column errors in chunks of 8192 values; with 9216 columns
    a single pairwise tree gives another total on this data, and the GPU gives numpy's."""
    from oracle import kquant_oracle as K
    n = 9216
    x = heavy_tailed(6, n, seed=8)
    rng = np.random.default_rng(14)
    wvec = 10.0 ** rng.uniform(-3, 5, n)
    qw = (10.0 ** rng.uniform(-2, 3, n)).astype(F32)
    rec = K.roundtrip(x, tt, None)
    colerr = ((rec.astype(np.float64) - x.astype(np.float64)) ** 2).sum(0)
    assert _one_tree(list(colerr * wvec)) != float((colerr * wvec).sum())
    for k, v in enumerate([dict(wvec=wvec), dict(qw=qw), dict(qw=qw, perm=rng.permutation(n))]):
        _say(f"tensor_err {tt} n={n} variant {k}")
        want = Po.tensor_err(x, tt, v.get("qw"), perm=v.get("perm"), wvec=v.get("wvec"))
        got = ob.tensor_err(x, tt, v.get("qw"), perm=v.get("perm"), wvec=v.get("wvec"))
        assert got == want, (k, got, want)


def test_batch_equals_single_calls(ob):
    """One pass over mixed types, shapes, dtypes and options equals the single calls."""
    rng = np.random.default_rng(3)
    items = []
    for k, tt in enumerate(["Q4_K", "Q2_K", "Q8_0", "Q6_K", "F16", "Q3_K", "Q5_K", "Q2_K"]):
        n = [256, 512, 96, 1024, 256, 768, 512, 256][k]
        x = heavy_tailed(20 + 7 * k, n, seed=40 + k)
        if k % 2:
            x = x.astype(np.float16)
        it = dict(x=x, ttype=tt)
        if k % 3 == 0:
            it["qw"] = (np.abs(rng.standard_normal(n)) + 0.1).astype(F32)
        if k % 3 == 1:
            it["perm"] = rng.permutation(n)
        if k == 7:
            it["rows_sample"] = 9
        items.append(it)
    got = ob.tensor_err_many(items)
    want = [Po.tensor_err(it["x"], it["ttype"], it.get("qw"), perm=it.get("perm"),
                          rows_sample=it.get("rows_sample")) for it in items]
    assert got == want
    assert got[4] == 0.0


def test_errors_like_the_reference(ob):
    x = heavy_tailed(8, 256, seed=1)
    with pytest.raises(IndexError):
        ob.tensor_err(x, "Q4_K", None, perm=np.arange(256) + 1)
    with pytest.raises(ValueError):
        ob.tensor_err(x, "Q4_K", np.ones(100, F32))
    with pytest.raises(ValueError):
        ob.tensor_err(x, "Q7_K", None)
    with pytest.raises(AssertionError):
        ob.tensor_err(heavy_tailed(2, 288, seed=2), "Q2_K", None)
    assert ob.tensor_err(x, "BF16", None) == 0.0
    # numpy's negative indices
    p = np.arange(256)
    p[:5] -= 256
    assert ob.tensor_err(x, "Q6_K", None, perm=p) == Po.tensor_err(x, "Q6_K", None, perm=p)


def test_out_of_range_index_gives_nan_not_a_fault(ob):
    """The C ABI never dereferences an index outside its range: the tensor's result is NaN."""
    from perm_amd import _lib
    lib = _lib.load()
    x = torch.from_numpy(heavy_tailed(16, 256, seed=3)).cuda()
    perm = torch.arange(256, dtype=torch.int32, device="cuda")
    perm[7] = 999
    rows = torch.tensor([0, 3, 99], dtype=torch.int32, device="cuda")
    ts = [_lib.ErrTensor(_lib.TTYPE["Q4_K"], 0, 16, 256, x.data_ptr(), None, perm.data_ptr(),
                         None, None, 0),
          _lib.ErrTensor(_lib.TTYPE["Q4_K"], 0, 16, 256, x.data_ptr(), None, None, None,
                         rows.data_ptr(), 3),
          _lib.ErrTensor(_lib.TTYPE["Q4_K"], 0, 16, 256, x.data_ptr(), None, None, None, None, 0)]
    arr = (_lib.ErrTensor * 3)(*ts)
    ws = _lib.workspace(lib.cp_tensor_err_ws_bytes(arr, 3))
    out = torch.empty(3, dtype=torch.float64, device="cuda")
    _lib.check(lib.cp_tensor_err_batch(arr, 3, _lib.ptr(ws), ws.numel(), _lib.ptr(out),
                                       _lib.stream_ptr()))
    v = out.cpu().numpy()
    assert np.isnan(v[0]) and np.isnan(v[1])
    assert v[2] == Po.tensor_err(x.cpu().numpy(), "Q4_K", None)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_col_sums_and_log_rms(ob, dtype):
    from perm_amd import _lib
    x = heavy_tailed(1000, 320, seed=9)
    if dtype == "f16":
        x = x.astype(np.float16)
    for step in (32768, 7, 64):
        _say(f"col_log_rms {dtype} row_step={step}")
        assert np.array_equal(ob.col_log_rms(x, step), Po.col_log_rms(x, step))
    # the device-libm variant of the C ABI: within 2 ulp of the host's log
    lib = _lib.load()
    xd, code = ob.weights_dev(x)
    ws = _lib.workspace(lib.cp_col_sums_ws_bytes(1000, 320, 64))
    out = torch.empty(320, dtype=torch.float64, device="cuda")
    _lib.check(lib.cp_col_log_rms(_lib.ptr(xd), code, 1000, 320, 64, _lib.ptr(out),
                                  _lib.ptr(ws), ws.numel(), _lib.stream_ptr()))
    got, want = out.cpu().numpy(), Po.col_log_rms(x, 64)
    ulp = np.abs(got.view(np.int64) - want.view(np.int64))
    assert ulp.max() <= 2


@pytest.mark.parametrize("case", ["q2k-unweighted", "mixed-imatrix", "q2k-scaled-channels"])
def test_optimize_matches_oracle(case):
    """The reference optimizer test's model (test_perm_optimize.py:14-61), and the same
    shapes with channel scales under which every space's sorted candidate matters (one
    layer's value-channel candidate loses): the GPU search picks the oracle's
    permutations with bit-identical objective values."""
    from perm_amd import perm as gp
    w = small_qwen3_model()
    if case == "q2k-scaled-channels":
        from test_oracle_objective import _scaled_qwen3_model
        w, _s = _scaled_qwen3_model()
        ttypes, qws = {n: "Q2_K" for n in w}, {}
    elif case == "q2k-unweighted":
        ttypes, qws = {n: "Q2_K" for n in w}, {}
    else:
        kinds = ["Q4_K", "Q3_K", "Q6_K", "Q5_K", "Q2_K", "Q8_0"]
        ttypes = {n: kinds[i % len(kinds)] for i, n in enumerate(sorted(w))}
        rng = np.random.default_rng(4)
        qws = {n: (np.abs(rng.standard_normal(a.shape[1])) + 0.05).astype(F32)
               for i, (n, a) in enumerate(sorted(w.items())) if i % 3}
    _say(f"optimize {case}")
    want_p, want_r = Po.optimize_qwen3(w, ttypes, qws, OPT_DIMS, rows_sample=300)
    got_p, got_r = gp.optimize(w, ttypes, qws, OPT_DIMS, rows_sample=300, log=lambda *_: None)
    assert np.array_equal(got_p["res"], want_p["res"])
    for l in range(2):
        assert np.array_equal(got_p["ffn"][l], want_p["ffn"][l])
        for h in range(2):
            assert np.array_equal(got_p["vo"][l][h], want_p["vo"][l][h])
    for space in ("res", "ffn", "vo"):
        for k in ("base", "opt", "rel"):
            assert got_r[space][k] == want_r[space][k], (space, k)
        assert got_r[space]["rel"] <= 1e-9
    assert got_r["res"]["key"] == want_r["res"]["key"]


def test_full_size_sampled_embedding(ob):
    """Qwen3-0.6B token_embd shape (151936 x 1024, f16) with the reference's default
    16384-row sample: Q8_0 bit-identical to the oracle on the full-size call, and the
    identity permutation equal to no permutation."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((151936, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    xd = torch.from_numpy(x).cuda()
    _say("full-size Q8_0 sampled")
    got = ob.tensor_err(xd, "Q8_0", None, rows_sample=16384)
    assert got == Po.tensor_err(x, "Q8_0", None, rows_sample=16384)
    qw = (np.abs(rng.standard_normal(1024)) + 0.1).astype(F32)
    _say("full-size Q6_K identity permutation")
    a = ob.tensor_err(xd, "Q6_K", qw, rows_sample=16384)
    b = ob.tensor_err(xd, "Q6_K", qw, perm=np.arange(1024), rows_sample=16384)
    assert a == b and np.isfinite(a) and a > 0
