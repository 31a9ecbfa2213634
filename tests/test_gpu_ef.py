"""GPU EF path parity: act order, the fp64 inverse-Hessian factor, and the EF
sweep (bit-exact against the oracle when both use the same factor; within the
code-agreement and H-weighted-error gates when the GPU computes its own)."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import correlated_hessian, heavy_tailed
from oracle import ef_oracle as E
from oracle import kquant_oracle as K
from perm_amd import _lib

pytestmark = pytest.mark.gpu
F32 = np.float32
TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]


@pytest.fixture(scope="module")
def ef():
    from perm_amd import ef as gef
    return gef


def _say(msg):
    print(msg, flush=True)


def _spectrum_matrix(n, eig, seed=0):
    rng = np.random.default_rng(seed)
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    M = (Q * eig) @ Q.T
    return (M + M.T) / 2


def test_act_order_is_stable_descending(ef):
    rng = np.random.default_rng(0)
    d = rng.standard_normal(1000)
    d[::7] = 0.5                                    # ties
    H = np.diag(d)
    got = ef.act_order_dev(torch.from_numpy(H).cuda()).cpu().numpy()
    assert np.array_equal(got, np.argsort(-d, kind="stable"))


@pytest.mark.parametrize("dtype,n,batch", [
    (torch.float32, 1, 1), (torch.float32, 2, 3), (torch.float32, 1000, 2),
    (torch.float32, 4096, 1), (torch.float32, 4097, 2), (torch.float32, 16384, 1),
    (torch.float32, 16385, 1),                      # past the LDS sort: the rank count
    (torch.float64, 3, 2), (torch.float64, 3072, 2), (torch.float64, 8192, 1),
    (torch.float64, 8193, 1)])
def test_act_order_matches_numpy_argsort(ef, dtype, n, batch):
    """The order is numpy's stable argsort of -diag(H) (NaN last, by index; -0 and +0
    tie) for both the LDS bitonic sort and the rank count past its size limit, with ties,
    signed zeros, infinities and NaN on the diagonal."""
    _say(f"act order {dtype} n={n} batch={batch}")
    rng = np.random.default_rng(n + batch)
    want = []
    H = torch.zeros((batch, n, n), dtype=dtype, device="cuda")
    for b in range(batch):
        d = rng.standard_normal(n)
        d[rng.integers(0, n, n // 5 + 1)] = 0.5               # ties
        d[rng.integers(0, n, n // 50 + 1)] = 0.0
        d[rng.integers(0, n, n // 50 + 1)] = -0.0
        if n > 8:
            d[rng.integers(0, n, 3)] = np.nan
            d[rng.integers(0, n, 2)] = np.inf
            d[rng.integers(0, n, 2)] = -np.inf
        d = d.astype(np.float32 if dtype == torch.float32 else np.float64)
        want.append(np.argsort(-d, kind="stable"))
        H[b].diagonal().copy_(torch.from_numpy(d))
    got = ef.act_order_dev(H).cpu().numpy()
    del H
    for b in range(batch):
        assert np.array_equal(got[b], want[b]), b


@pytest.mark.parametrize("n", [96, 200, 256, 777, 1024, 1500])
def test_factor_matches_closed_form(ef, n):
    _say(f"factor n={n}")
    H = correlated_hessian(n, 4 * n, seed=n)
    U = ef.cholesky_inv_upper(H, 0.01)
    U_ref = E.inv_upper_factor(H, 0.01)
    assert U.dtype == np.float64 and np.array_equal(U, np.triu(U))
    rel = np.abs(U - U_ref).max() / np.abs(U_ref).max()
    assert rel < 1e-11, rel
    Hd = H + (0.01 * np.mean(np.diag(H)) + 1e-8) * np.eye(n)
    assert np.abs(U.T @ U @ Hd - np.eye(n)).max() < 1e-9


@pytest.mark.parametrize("n,N,kind", [(3072, 65536, "student-t"), (4096, 131072, "outliers"),
                                      (14336, 131072, "outliers")])
def test_factor_matches_library_at_config_sizes(ef, n, N, kind):
    """E1 at the benchmark configurations' sizes (the Qwen3-0.6B down_in space, the
    Llama-3-8B spaces with 0.5 % of channels x50): U from the act-ordered Hessian against
    the float64 closed form of coldpress/ef.py:60-78 -- inv, symmetrize, Cholesky -- taken
    from torch.linalg on the device (a library routine, none of this library's kernels).
    The bound is on max |dU| / max |U|; float32, which the sweep consumes, resolves 6e-8."""
    from perm_amd import workloads as wl
    from perm_amd.hessians import xtx_accumulate
    _say(f"factor vs torch.linalg n={n} N={N} {kind}")
    H = xtx_accumulate(wl.family_activations(kind, N, n, seed=n))
    order = ef.act_order_dev(H)
    U, used = ef.factor_dev(H, order, out_dtype=torch.float64)
    assert used == [0.01]
    o = order.long()
    Hp = H.double()[o][:, o]
    lam = 0.01 * float(torch.diagonal(Hp).mean()) + 1e-8
    Hp.diagonal().add_(lam)
    Hinv = torch.linalg.inv(Hp)
    del Hp
    Hinv = (Hinv + Hinv.T) / 2
    Uref = torch.linalg.cholesky(Hinv).T
    del Hinv
    rel = float((U - Uref).abs().max() / Uref.abs().max())
    _say(f"  max |dU| / max |U| = {rel:.2e}")
    assert torch.equal(U, torch.triu(U))
    assert rel < 1e-8


def _np_tree(v):
    """One pairwise tree over all of v (numpy's order only up to 8192 values)."""
    n = len(v)
    if n < 8:
        r = 0.0
        for a in v:
            r = r + a
        return r
    if n <= 128:
        r = list(v[:8])
        i = 8
        while i + 8 <= n:
            for j in range(8):
                r[j] = r[j] + v[i + j]
            i += 8
        s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
        for a in v[i:]:
            s = s + a
        return s
    n2 = n // 2
    n2 -= n2 % 8
    return _np_tree(v[:n2]) + _np_tree(v[n2:])


@pytest.mark.parametrize("n", [100, 1000, 3000, 9000, 14336])
def test_factor_damping_shift_is_numpys_mean(ef, n):
    """Diagonal H: U = diag(1 / sqrt(h + shift)) with correctly rounded sqrt and
    division, so U equals numpy's bit for bit only if the damping shift does,
    i.e. only if the mean of diag(H) is summed in numpy's order (pairwise inside
    chunks of 8192 values, the chunk sums added in order)."""
    _say(f"damping shift n={n}")
    rng = np.random.default_rng(n)
    h = 10.0 ** rng.uniform(-3, 7, n)
    draw = 0
    while n > 8192 and _np_tree(list(h)) == np.add.reduce(h):
        # a draw on which one tree over all n values gives another sum than numpy's
        draw += 1
        h = 10.0 ** np.random.default_rng(n + 1000 * draw).uniform(-3, 7, n)
    H = np.diag(h)
    shift = 0.01 * np.mean(np.diag(H)) + 1e-8
    seq = 0.0
    for v in h:  # the plain left-to-right order: a different shift on this data
        seq += v
    if n > 128:
        assert 0.01 * (seq / n) + 1e-8 != shift
    Hd = torch.from_numpy(H).cuda()
    del H
    U, used = ef.factor_dev(Hd, None, 0.01, out_dtype=torch.float64)
    del Hd
    assert used == [0.01]
    diag = torch.diagonal(U).cpu().numpy()
    assert int(torch.count_nonzero(U)) == n
    del U
    assert np.array_equal(diag, 1.0 / np.sqrt(h + shift))


def test_factor_with_order_and_f32_output(ef):
    n = 512
    H = correlated_hessian(n, 2048, seed=3)
    Hd = torch.from_numpy(H).cuda()
    order = ef.act_order_dev(Hd)
    U, used = ef.factor_dev(Hd, order, 0.01)
    o = order.cpu().numpy()
    U_ref = E.inv_upper_factor(H[np.ix_(o, o)], 0.01).astype(F32)
    assert used == [0.01]
    Ug = U.cpu().numpy()
    assert (Ug != U_ref).mean() < 0.01                      # f32 cast: rare 1-ulp differences
    assert np.abs(Ug - U_ref).max() <= 4 * np.spacing(np.abs(U_ref).max())


def test_factor_batched_equals_single(ef):
    Hs = [correlated_hessian(256, 1024, seed=s) for s in range(3)]
    Hb = torch.from_numpy(np.stack(Hs)).cuda()
    order = ef.act_order_dev(Hb)
    Ub, _ = ef.factor_dev(Hb, order, 0.01)
    for i in range(3):
        Ui, _ = ef.factor_dev(Hb[i].contiguous(), order[i], 0.01)
        assert torch.equal(Ub[i], Ui)


def test_factor_escalates_like_reference(ef, capfd):
    n = 256
    eig = np.linspace(1.0, 100.0, n)
    eig[0] = -2.0
    H = _spectrum_matrix(n, eig, seed=1)
    Hd = torch.from_numpy(H).cuda()
    U, used = ef.factor_dev(Hd, None, 0.01, out_dtype=torch.float64)
    U = U.cpu().numpy()
    assert used[0] > 0.01 and np.all(np.isfinite(U)) and np.array_equal(U, np.triu(U))
    # the oracle escalates to the same damp and lands on the same factor
    U_ref = E.inv_upper_factor(H, 0.01, log=False)
    assert np.abs(U - U_ref).max() / np.abs(U_ref).max() < 1e-9


def test_nan_diagonal_orders_last_and_raises_linalg_error(ef):
    """numpy's argsort puts NaN last, and LAPACK's Cholesky fails on a NaN pivot at every
    damping, so the reference raises LinAlgError. The GPU order is a permutation with the
    NaN columns last (by index), and the factor raises the same error."""
    n = 256
    H = correlated_hessian(n, 1024, seed=12)
    H[5, 5] = np.nan
    H[77, 77] = np.nan
    Hd = torch.from_numpy(H).cuda()
    order = ef.act_order_dev(Hd).cpu().numpy()
    assert np.array_equal(order, np.argsort(-np.diag(H), kind="stable"))
    assert order[-2:].tolist() == [5, 77]
    with pytest.raises(np.linalg.LinAlgError):
        ef.factor_dev(Hd, torch.from_numpy(order).cuda(), 0.01)
    with pytest.raises(np.linalg.LinAlgError):
        ef.ef_encode(heavy_tailed(4, n, seed=1), "Q2_K", None, H)


def test_factor_flags_an_order_that_is_not_a_permutation(ef):
    """Called through the C ABI with a bad order (no host check in between), the factor
    clamps every read of it and reports CP_ERR_INDEX; the async form sets bit 1 of the
    matrix's flag and leaves the other matrix alone."""
    from perm_amd import _lib
    lib = _lib.load()
    n = 128
    Hs = np.stack([correlated_hessian(n, 512, seed=s) for s in (1, 2)])
    Hb = torch.from_numpy(Hs).cuda()
    order = torch.arange(n, dtype=torch.int32, device="cuda").repeat(2, 1)
    order[1, 3] = 1000      # out of range
    order[1, 9] = -4        # out of range
    ws = _lib.workspace(lib.cp_chol_ws_bytes(n, 2))
    U = torch.empty(2, n, n, device="cuda")
    st = lib.cp_chol_inv_upper(_lib.ptr(Hb), 1, n, 2, _lib.ptr(order), 0.01, 6, _lib.ptr(U), 0,
                               None, _lib.ptr(ws), ws.numel(), _lib.stream_ptr())
    assert st == _lib.CP_ERR_INDEX
    with pytest.raises(IndexError):
        _lib.check(st)
    order[1, 3], order[1, 9] = 3, 3  # in range, repeated
    flags = torch.full((2,), 7, dtype=torch.int32, device="cuda")
    _lib.check(lib.cp_chol_inv_upper_async(_lib.ptr(Hb), 1, n, 2, _lib.ptr(order), 0.01,
                                           _lib.ptr(U), 0, _lib.ptr(flags), _lib.ptr(ws),
                                           ws.numel(), _lib.stream_ptr()))
    assert flags.cpu().tolist() == [0, 2]
    U0 = E.inv_upper_factor(Hs[0], 0.01).astype(F32)
    assert np.abs(U[0].cpu().numpy() - U0).max() <= 4 * np.spacing(np.abs(U0).max())


def test_factor_gives_up(ef):
    H = -np.eye(64) * 1e6
    H[0, 0] = 1.0
    with pytest.raises(np.linalg.LinAlgError, match="not positive definite"):
        ef.cholesky_inv_upper(H, 0.01, _max_tries=3)


def _run_exact(ef, W, tt, qw, H, n_iter=2, mode="exact"):
    """GPU EF with the oracle's own float32 factor and order: must be bit-exact."""
    order = E.act_order(H, stable=True)
    U = E.inv_upper_factor(H[np.ix_(order, order)], 0.01).astype(F32)
    want_raw, want_rec = E.ef_encode(W, tt, qw, H, n_iter=n_iter, U=U, stable_order=True)
    item = {"ttype": tt, "x": torch.from_numpy(W).cuda(),
            "qw": torch.from_numpy(qw).cuda() if qw is not None else None,
            "U": torch.from_numpy(U).cuda(), "order": torch.from_numpy(order.astype(np.int32)).cuda()}
    (raw, rec), = ef.ef_encode_dev([item], n_iter, ef.MODES[mode])
    return raw.cpu().numpy(), rec.cpu().numpy(), want_raw, want_rec


@pytest.mark.parametrize("mode", ["exact", "exact_valu"])
@pytest.mark.parametrize("tt", TYPES)
@pytest.mark.parametrize("weighted", [False, True])
def test_sweep_bit_exact_vs_oracle(ef, tt, weighted, mode):
    nrow, n = 70, 512                                   # 70 rows: a partial stripe
    _say(f"exact sweep {mode} {tt} weighted={weighted}")
    W = heavy_tailed(nrow, n, seed=17)
    W[5] = 0.0                                          # an all-zero row
    W[9, ::3] = -0.0                                    # signed zeros
    H = correlated_hessian(n, 4096, seed=5)
    qw = (np.diag(H) / 4096).astype(F32) if weighted else None
    raw, rec, want_raw, want_rec = _run_exact(ef, W, tt, qw, H, mode=mode)
    bad = np.nonzero((raw != want_raw).any(1))[0]
    assert bad.size == 0, f"rows {bad[:10]} differ"
    assert np.array_equal(rec, want_rec)


@pytest.mark.parametrize("n_iter", [1, 3])
def test_sweep_bit_exact_iterations(ef, n_iter):
    W = heavy_tailed(64, 768, seed=3)
    H = correlated_hessian(768, 2048, seed=6)
    qw = (np.diag(H) / 2048).astype(F32)
    raw, _, want_raw, _ = _run_exact(ef, W, "Q2_K", qw, H, n_iter=n_iter)
    assert np.array_equal(raw, want_raw)


@pytest.mark.parametrize("rows", ["16", "32"])
@pytest.mark.parametrize("waves", ["1", "2", "4", "8"])
def test_sweep_waves_per_stripe_bit_exact(ef, rows, waves, monkeypatch):
    """Calls with few stripes spread each stripe over 2, 4 or 8 waves (blocks taken in
    rounds, the round's blocks swept in order); every stripe height and wave count gives
    the oracle's bytes, including tensors with fewer blocks than waves, a partial last
    round and rows that do not fill the last stripe."""
    monkeypatch.setenv("CP_EF_SWEEP_ROWS", rows)
    monkeypatch.setenv("CP_EF_SWEEP_WAVES", waves)
    specs = [(40, 1024, "Q2_K", 61), (17, 768, "Q4_K", 62), (33, 256, "Q6_K", 63)]
    for W, tt, qw, H, order, U in _oracle_items(specs):
        _say(f"waves {waves}: {tt} {W.shape}")
        want_raw, want_rec = E.ef_encode(W, tt, qw, H, n_iter=2, U=U, order=order)
        item = {"ttype": tt, "x": torch.from_numpy(W).cuda(), "qw": torch.from_numpy(qw).cuda(),
                "U": torch.from_numpy(U).cuda(),
                "order": torch.from_numpy(order.astype(np.int32)).cuda()}
        (raw, rec), = ef.ef_encode_dev([item], 2)
        assert np.array_equal(raw.cpu().numpy(), want_raw)
        assert np.array_equal(rec.cpu().numpy(), want_rec)
        # the launch the library reports: the requested stripe height and waves, the waves
        # capped at the tensor's 64-column blocks (a power of two)
        rs, wv = (ctypes.c_int * 1)(), (ctypes.c_int * 1)()
        mode = _lib.load().cp_ef_last_sweep(ctypes.cast(rs, ctypes.c_void_p),
                                            ctypes.cast(wv, ctypes.c_void_p))
        want_w = int(waves)
        while want_w > W.shape[1] // 64:
            want_w //= 2
        assert (mode, rs[0], wv[0]) == (_lib.CP_EF_EXACT, int(rows), want_w)


def _codes(tt, raw, nrow, n):
    return K.stored_codes(tt, raw).reshape(nrow, n)


@pytest.mark.parametrize("tt", TYPES)
def test_full_gpu_path_within_gates(ef, tt):
    """GPU order + fp64 factor + sweep against the reference-equivalent oracle:
    >= 99.9 % identical codes, tr(dW H dW^T) within 1e-3 relative."""
    from perm_amd.workloads import single_linear
    _say(f"full path {tt}")
    W, _X, H = single_linear(seed=0, nrow=192, n=1024, n_act=8192)
    qw = np.diag(H).astype(F32)
    raw, rec = ef.ef_encode(W, tt, qw, H)
    want_raw, want_rec = E.ef_encode(W, tt, qw, H, stable_order=True)
    agree = (_codes(tt, raw, *W.shape) == _codes(tt, want_raw, *W.shape)).mean()
    e_gpu, e_ref = E.h_weighted_err(W, rec, H), E.h_weighted_err(W, want_rec, H)
    _say(f"  codes agree {agree:.6f}, err rel diff {abs(e_gpu - e_ref) / e_ref:.2e}")
    assert agree >= 0.999
    assert abs(e_gpu - e_ref) / e_ref < 1e-3


def test_fp16_stored_rank_deficient_hessian(ef, tmp_path):
    """The reference's faithful-path case (test_ef_cholesky_robust.py:67-79): a rank-
    deficient X^T X (128 rows for n = 512, four rows x60) through the fp16 Hessian storage
    (here the GPU pack / expand of perm_amd.hessians). The GPU factor takes the oracle's
    damping step, agrees with its factor within 1e-9 relative, and the EF encode on it
    stays inside the gates."""
    from perm_amd import hessians as hs
    n = 512
    rng = np.random.default_rng(2)
    A = rng.standard_normal((n // 4, n))
    A[:4] *= 60.0
    H = (A.T @ A).astype(np.float32)
    hs.save_hessians({"blk.0.ffn_down.weight": {"H": H, "n": 4096}}, str(tmp_path))
    H_rt, _ = hs.load_hessian(str(tmp_path), "blk.0.ffn_down.weight")
    assert H_rt.dtype == np.float64
    Hd = torch.from_numpy(H_rt).cuda()
    U, used = ef.factor_dev(Hd, None, 0.01, out_dtype=torch.float64)
    U_ref = E.inv_upper_factor(H_rt, 0.01, log=False)
    assert used == [0.01]
    U = U.cpu().numpy()
    assert np.abs(U - U_ref).max() / np.abs(U_ref).max() < 1e-9
    W = heavy_tailed(96, n, seed=4)
    qw = (np.diag(H_rt) / 4096).astype(F32)
    raw, rec = ef.ef_encode(W, "Q2_K", qw, H_rt)
    want_raw, want_rec = E.ef_encode(W, "Q2_K", qw, H_rt, stable_order=True)
    agree = (_codes("Q2_K", raw, *W.shape) == _codes("Q2_K", want_raw, *W.shape)).mean()
    e_gpu, e_ref = E.h_weighted_err(W, rec, H_rt), E.h_weighted_err(W, want_rec, H_rt)
    _say(f"  rank-deficient fp16 H: codes agree {agree:.6f}, err rel diff "
         f"{abs(e_gpu - e_ref) / e_ref:.2e}")
    assert agree >= 0.999 and abs(e_gpu - e_ref) / e_ref < 1e-3


def _damped_near_singular(n, rel, seed):
    """H with eigenvalues linspace(1, 100) except the smallest, placed so that the damped
    matrix H + (0.01 mean(diag H) + 1e-8) I has smallest eigenvalue rel x the shift
    (negative rel: not positive definite at the first damping)."""
    eig = np.linspace(1.0, 100.0, n)
    S, c = eig[1:].sum(), 0.01 / n
    eig[0] = -(c * S + 1e-8) * (1 - rel) / (1 + c * (1 - rel))
    return _spectrum_matrix(n, eig, seed)


@pytest.mark.parametrize("rel", [1e-2, 1e-6, 1e-11, -1e-11, -1e-6, -1e-2, -30.0])
def test_near_singular_damped_hessian_escalates_like_reference(ef, rel):
    """Damped matrices close to singular on both sides: the GPU takes the reference's
    escalation step every time (ef.py:60-84: LAPACK inverse, then Cholesky of it; here the
    Cholesky of the reversed damped H). The two criteria part only where the damped
    matrix's condition number reaches about 1e16 (smallest eigenvalue within ~1e-14 of
    the shift), where the reference's own LAPACK inverse is decided by rounding; the
    cases here stay 1000x clear of that band. Where the factor is well conditioned it
    agrees with the oracle's within 1e-9 relative."""
    n = 256
    H = _damped_near_singular(n, rel, seed=3)
    U_ref = E.inv_upper_factor(H, 0.01, log=False)
    d_ref = None
    for k in range(6):  # the oracle's damping step, read back from its closed form
        Hd = H + (0.01 * 10 ** k * np.mean(np.diag(H)) + 1e-8) * np.eye(n)
        try:
            Hi = np.linalg.inv(Hd)
            if np.array_equal(np.linalg.cholesky((Hi + Hi.T) / 2).T, U_ref):
                d_ref = 0.01 * 10 ** k
                break
        except np.linalg.LinAlgError:
            continue
    assert d_ref is not None
    U, used = ef.factor_dev(torch.from_numpy(H).cuda(), None, 0.01, out_dtype=torch.float64)
    assert np.isclose(used[0], d_ref, rtol=1e-12), (used, d_ref)
    U = U.cpu().numpy()
    assert np.all(np.isfinite(U)) and np.array_equal(U, np.triu(U))
    if used[0] > 0.01 or rel >= 1e-2:  # well conditioned after the shift
        assert np.abs(U - U_ref).max() / np.abs(U_ref).max() < 1e-9


def test_ef_beats_rtn_on_gpu(ef):
    """test_ef_synthetic.py:30-46 on the GPU path."""
    n, nrow, T = 512, 24, 4096
    rng = np.random.default_rng(101)
    W = (rng.standard_normal((nrow, n)) ** 3).astype(F32)
    H = correlated_hessian(n, T, seed=0)
    qw = (np.diag(H) / T).astype(F32)
    rtn = K.roundtrip(W, "Q2_K", qw)
    _, rec = ef.ef_encode(W, "Q2_K", qw, H)
    assert E.h_weighted_err(W, rec, H) < 0.97 * E.h_weighted_err(W, rtn, H)


def test_many_shares_factor_and_matches_single(ef):
    n = 512
    H = torch.from_numpy(correlated_hessian(n, 2048, seed=9)).cuda()
    qw = torch.diagonal(H).float().contiguous() / 2048
    ws = {nm: torch.from_numpy(heavy_tailed(r, n, seed=i)).cuda()
          for i, (nm, r) in enumerate([("a", 64), ("b", 128), ("c", 96)])}
    tens = [{"name": nm, "ttype": "Q2_K", "x": x, "qw": qw, "H": H} for nm, x in ws.items()]
    out = ef.ef_encode_many(tens)
    for nm, x in ws.items():
        raw1, rec1 = ef.ef_encode(x, "Q2_K", qw, H)
        assert torch.equal(out[nm][0], raw1) and torch.equal(out[nm][1], rec1)


def _oracle_items(specs):
    """(W, tt, qw, H, order, U) per spec (nrow, n, tt, seed), with the oracle's own
    float32 factor and order, so the GPU sweep must reproduce the oracle bit for bit."""
    out = []
    for nrow, n, tt, seed in specs:
        W = heavy_tailed(nrow, n, seed=seed)
        H = correlated_hessian(n, 4 * n, seed=seed + 100)
        qw = (np.diag(H) / (4 * n)).astype(F32)
        order = E.act_order(H, stable=True)
        U = E.inv_upper_factor(H[np.ix_(order, order)], 0.01).astype(F32)
        out.append((W, tt, qw, H, order, U))
    return out


@pytest.mark.parametrize("specs", [
    # one size: the sweep hands each XCD a contiguous run of stripes; uneven row
    # counts and partial stripes put task boundaries anywhere in those runs
    [(70, 512, "Q2_K", 1), (200, 512, "Q3_K", 2), (33, 512, "Q2_K", 3), (129, 512, "Q6_K", 4)],
    # mixed sizes in one call: stripes in the table's longest-first order
    [(96, 768, "Q2_K", 5), (70, 512, "Q4_K", 6), (40, 1024, "Q5_K", 7), (64, 256, "Q2_K", 8)],
], ids=["same_n", "mixed_n"])
def test_batched_sweep_bit_exact_vs_oracle(ef, specs):
    """Several tensors in one EF call: every tensor's bytes equal the oracle's."""
    _say(f"batched sweep {[s[:3] for s in specs]}")
    data = _oracle_items(specs)
    items = [{"ttype": tt, "x": torch.from_numpy(W).cuda(), "qw": torch.from_numpy(qw).cuda(),
              "U": torch.from_numpy(U).cuda(), "order": torch.from_numpy(order.astype(np.int32)).cuda()}
             for W, tt, qw, _, order, U in data]
    got = ef.ef_encode_dev(items, 2, ef.MODES["exact"])
    for (W, tt, qw, H, _, U), (raw, rec) in zip(data, got):
        want_raw, want_rec = E.ef_encode(W, tt, qw, H, n_iter=2, U=U, stable_order=True)
        assert np.array_equal(raw.cpu().numpy(), want_raw), tt
        assert np.array_equal(rec.cpu().numpy(), want_rec), tt


def test_factor_async_equals_blocking(ef):
    Hs = [correlated_hessian(320, 1280, seed=s) for s in range(3)]
    Hb = torch.from_numpy(np.stack(Hs)).cuda()
    order = ef.act_order_dev(Hb)
    Ua, flags = ef.factor_dev_async(Hb, order, 0.01)
    Ub, _ = ef.factor_dev(Hb, order, 0.01)
    assert flags.cpu().tolist() == [0, 0, 0]
    assert torch.equal(Ua, Ub)


@pytest.mark.parametrize("n,batch", [(3072, 4), (1000, 3)])
def test_factor_compact_tiles_give_the_same_factor(ef, n, batch):
    """cp_chol_compact_tiles(1) (every fp64 GEMM on 64 x 64 tiles, as the concurrent
    size-class driver queues them) gives bit-identical U: each output element sums its K
    range in the same order whatever the tile."""
    lib = _lib.load()
    _say(f"compact tiles n={n} batch={batch}")
    Hb = torch.from_numpy(np.stack([correlated_hessian(n, 2 * n, seed=40 + s)
                                    for s in range(batch)])).cuda()
    order = ef.act_order_dev(Hb)
    Ua, _ = ef.factor_dev(Hb, order, 0.01)
    lib.cp_chol_compact_tiles(1)
    try:
        Ub, flags = ef.factor_dev_async(Hb, order, 0.01)
    finally:
        lib.cp_chol_compact_tiles(0)
    assert flags.cpu().tolist() == [0] * batch
    assert torch.equal(Ua, Ub)


def test_factor_chunked_outer_updates_do_not_depend_on_the_schedule(ef):
    """From n = 8192 the outer updates sum K in 1024-column chunks. A single matrix has
    too few row tiles to fill the GPU, so each outer update computes all its chunk
    products at once and subtracts them in order afterwards; in a batch of eight most
    outer updates run one GEMM per chunk instead. Both must give the same U bit for bit,
    and U must invert H + lambda I."""
    from perm_amd.hessians import xtx_accumulate_many
    from perm_amd import workloads as wl
    n, batch = 8448, 8
    _say(f"chunked outer updates n={n} batch={batch}")
    Hb = torch.zeros(batch, n, n, device="cuda")
    for z in range(batch):
        xtx_accumulate_many([wl.student_t_activations(2 * n, n, seed=70 + z)], [Hb[z]])
    order = ef.act_order_dev(Hb)
    Ub, used = ef.factor_dev(Hb, order, 0.01, out_dtype=torch.float64)
    assert used == [0.01] * batch
    for z in (0, 5):
        Uz, _ = ef.factor_dev(Hb[z].contiguous(), order[z], 0.01, out_dtype=torch.float64)
        assert torch.equal(Ub[z], Uz)
    o = order[0].long()
    Hp = Hb[0].double()[o][:, o]
    lam = 0.01 * float(torch.diagonal(Hp).mean()) + 1e-8
    v = torch.randn((n, 4), device="cuda", dtype=torch.float64)
    r = Ub[0].T @ (Ub[0] @ (Hp @ v + lam * v))
    assert float((r - v).abs().max() / v.abs().max()) < 1e-8


def test_factor_on_many_streams_gives_one_factor(ef):
    """A factorization of a small batch runs its look-ahead updates on a second stream kept
    per calling stream, for up to 64 calling streams; past that it queues them on the
    calling stream. U must be the same bit for bit on every stream: 70 raw HIP streams
    here (torch's pool would hand out only 32 distinct ones), so the last ones take the
    in-place path."""
    n = 1280
    _say(f"factor on 70 streams n={n}")
    hip = ctypes.CDLL(_lib.LIB_PATH)  # resolves the HIP runtime the library links
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    H = torch.from_numpy(correlated_hessian(n, 2 * n, seed=17)).cuda()
    order = ef.act_order_dev(H)
    U0, _ = ef.factor_dev(H, order, 0.01)
    raw = []
    try:
        for _ in range(70):
            h = ctypes.c_void_p()
            assert hip.hipStreamCreate(ctypes.byref(h)) == 0
            raw.append(h)
        outs = []
        for h in raw:
            s = torch.cuda.ExternalStream(h.value)
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs.append(ef.factor_dev_async(H, order, 0.01))
        torch.cuda.synchronize()
        for U, flags in outs:
            assert int(flags.sum()) == 0
            assert torch.equal(U, U0)
    finally:
        torch.cuda.synchronize()
        outs = None
        torch.cuda.empty_cache()  # no cached block stays tied to a stream destroyed below
        for h in raw:
            hip.hipStreamDestroy(h)


def test_factor_async_flags_a_failed_matrix(ef):
    n = 256
    eig = np.linspace(1.0, 100.0, n)
    eig[0] = -2.0
    bad = _spectrum_matrix(n, eig, seed=1)
    good = correlated_hessian(n, 1024, seed=2)
    Hb = torch.from_numpy(np.stack([good, bad])).cuda()
    _, flags = ef.factor_dev_async(Hb, None, 0.01)
    assert flags.cpu().tolist() == [0, 1]


def test_many_redoes_a_class_that_needs_escalation(ef, capfd):
    """A size class whose factorization fails at the first damp is factorized
    again with escalation and re-encoded; the other class is untouched."""
    n1, n2 = 256, 512
    eig = np.linspace(1.0, 100.0, n1)
    eig[0] = -2.0
    Hbad = torch.from_numpy(_spectrum_matrix(n1, eig, seed=1)).cuda()
    Hgood = torch.from_numpy(correlated_hessian(n2, 2048, seed=3)).cuda()
    xa = torch.from_numpy(heavy_tailed(64, n1, seed=5)).cuda()
    xb = torch.from_numpy(heavy_tailed(96, n2, seed=6)).cuda()
    tens = [{"name": "a", "ttype": "Q2_K", "x": xa, "qw": None, "H": Hbad},
            {"name": "b", "ttype": "Q4_K", "x": xb, "qw": None, "H": Hgood}]
    out = ef.ef_encode_many(tens)
    for t in tens:
        raw1, rec1 = ef.ef_encode(t["x"], t["ttype"], None, t["H"])
        assert torch.equal(out[t["name"]][0], raw1) and torch.equal(out[t["name"]][1], rec1)
    assert "damp escalated" in capfd.readouterr().err


@pytest.fixture(scope="module")
def single_linear_ref():
    """Oracle EF of the single-Linear workload (1024 x 1024, H from 8192 rows with
    1 % outlier channels x20), for qw = diag(H) and qw = None."""
    from perm_amd.workloads import single_linear
    W, _X, H = single_linear(seed=0)
    out = {}
    for tag, qw in (("imat", np.diag(H).astype(F32)), ("ref", None)):
        out[tag] = (qw, *E.ef_encode(W, "Q2_K", qw, H, stable_order=True))
    return W, H, out


@pytest.mark.parametrize("mode", ["exact", "exact_valu", "mfma"])
def test_single_linear_workload_gates(ef, single_linear_ref, mode):
    """Exact modes: every byte identical. MFMA-accumulated mode: within the
    code-agreement and H-weighted-error gates on the imatrix path (the
    unweighted path is reported, not gated: near-tie flips cascade there)."""
    W, H, ref = single_linear_ref
    for tag, (qw, want_raw, want_rec) in ref.items():
        raw, rec = ef.ef_encode(W, "Q2_K", qw, H, mode=mode)
        agree = (_codes("Q2_K", raw, *W.shape) == _codes("Q2_K", want_raw, *W.shape)).mean()
        e_gpu, e_ref = E.h_weighted_err(W, rec, H), E.h_weighted_err(W, want_rec, H)
        _say(f"single-linear {mode}/{tag}: codes agree {agree:.6f}, rows identical "
             f"{(raw == want_raw).all(1).mean():.4f}, err rel diff {abs(e_gpu - e_ref) / e_ref:.2e}")
        if mode.startswith("exact"):
            assert np.array_equal(raw, want_raw) and np.array_equal(rec, want_rec)
        elif tag == "imat":
            assert agree >= 0.999
            assert abs(e_gpu - e_ref) / e_ref < 1e-3


@pytest.mark.parametrize("tt", TYPES)
def test_mfma_accumulate_mode_bounds(ef, tt):
    """The opt-in MFMA-accumulated mode is not bit-exact: a near-tie code flip
    cascades along its row. Its bound here is >= 99 % identical codes (98 % for
    Q5_K, whose 32-level affine grid has the most near-ties: 98.4 % measured) and
    the H-weighted error within 5e-3 of the reference (the exact modes carry the
    99.9 % / 1e-3 gates with 100 % / 0)."""
    from perm_amd.workloads import single_linear
    W, _X, H = single_linear(seed=3, nrow=160, n=1536, n_act=6144)
    qw = np.diag(H).astype(F32)
    raw, rec = ef.ef_encode(W, tt, qw, H, mode="mfma")
    want_raw, want_rec = E.ef_encode(W, tt, qw, H, stable_order=True)
    agree = (_codes(tt, raw, *W.shape) == _codes(tt, want_raw, *W.shape)).mean()
    e_gpu, e_ref = E.h_weighted_err(W, rec, H), E.h_weighted_err(W, want_rec, H)
    _say(f"mfma {tt}: codes agree {agree:.6f}, err rel diff {abs(e_gpu - e_ref) / e_ref:.2e}")
    assert agree >= (0.98 if tt == "Q5_K" else 0.99)
    assert abs(e_gpu - e_ref) / e_ref < 5e-3


@pytest.mark.parametrize("n,batch", [(1000, 3), (3072, 2), (4096, 1)])
def test_factor_reads_no_workspace_it_did_not_write(ef, n, batch):
    """The factorization clears its inverse workspace only where a 128 x 128 GEMM tile can
    read an entry nothing wrote (n > 4096). Below that every entry it reads is written
    first, so a workspace full of NaN must give the same U, bit for bit, as a zeroed one."""
    from perm_amd import _lib
    lib = _lib.load()
    _say(f"factor on a NaN workspace n={n} batch={batch}")
    Hb = torch.stack([torch.from_numpy(correlated_hessian(n, 2 * n, seed=40 + z)) for z in range(batch)]
                     ).float().cuda()
    order = ef.act_order_dev(Hb)
    nbytes = lib.cp_chol_ws_bytes(n, batch)
    outs = []
    for fill in (0.0, float("nan")):
        ws = torch.full(((nbytes + 7) // 8,), fill, dtype=torch.float64, device="cuda")
        U = torch.empty((batch, n, n), dtype=torch.float64, device="cuda")
        used = (ctypes.c_double * batch)()
        st = lib.cp_chol_inv_upper(_lib.ptr(Hb), 0, n, batch, _lib.ptr(order), 0.01, 6,
                                   _lib.ptr(U), 1, ctypes.cast(used, ctypes.c_void_p), _lib.ptr(ws),
                                   ws.numel() * 8, _lib.stream_ptr())
        assert st == 0, lib.cp_last_error()
        assert list(used) == [0.01] * batch
        outs.append(U)
    assert torch.isfinite(outs[1]).all()
    assert torch.equal(outs[0], outs[1])
