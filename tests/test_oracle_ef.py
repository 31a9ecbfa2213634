"""Pins for the EF oracle (oracle/ef_oracle.py) -- the reference's ef.py cannot be
imported here (it needs the absent pip ``gguf``), so each function is pinned by a
closed form, an independent re-derivation, or the reference's own invariants."""
import numpy as np
import pytest

from conftest import correlated_hessian, heavy_tailed
from oracle import ef_oracle as E
from oracle import kquant_oracle as K

F32 = np.float32


def _spectrum_matrix(n, eig, seed=0):
    rng = np.random.default_rng(seed)
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    M = (Q * eig) @ Q.T
    return (M + M.T) / 2


def test_factor_closed_form_first_attempt():
    """First attempt == chol((inv(H+lI) + inv(H+lI)^T)/2)^T (test_ef_cholesky_robust.py:51-64)."""
    n = 128
    rng = np.random.default_rng(5)
    M = rng.standard_normal((n, n))
    H = M @ M.T + n * np.eye(n)
    Hd = H.copy()
    Hd[np.diag_indices(n)] += 0.01 * float(np.mean(np.diag(Hd))) + 1e-8
    Hinv = np.linalg.inv(Hd)
    U_ref = np.linalg.cholesky((Hinv + Hinv.T) / 2).T
    assert np.array_equal(E.inv_upper_factor(H, 0.01), U_ref)


def test_factor_is_upper_inverse_factor():
    """U upper with U^T U = inv(H + lI): a transposed or lower factor fails this."""
    H = correlated_hessian(96, 512, seed=1)
    U = E.inv_upper_factor(H, 0.01)
    assert np.array_equal(U, np.triu(U)) and np.all(np.diag(U) > 0)
    Hd = H + (0.01 * np.mean(np.diag(H)) + 1e-8) * np.eye(96)
    assert np.allclose(U.T @ U @ Hd, np.eye(96), atol=1e-9)


def test_factor_escalates_on_negative_eigenvalue(capsys):
    """Exact spectrum with eig -2 breaks the fixed damp; escalation recovers
    (test_ef_cholesky_robust.py:36-48)."""
    n = 256
    eig = np.linspace(1.0, 100.0, n)
    eig[0] = -2.0
    H = _spectrum_matrix(n, eig, seed=1)
    U = E.inv_upper_factor(H, 0.01)
    assert np.all(np.isfinite(U)) and np.array_equal(U, np.triu(U))
    assert "escalated" in capsys.readouterr().err


def test_factor_gives_up_after_max_tries():
    H = -np.eye(8) * 1e6
    H[0, 0] = 1.0          # mean diag negative -> base 1, shift can never win
    with pytest.raises(np.linalg.LinAlgError, match="not positive definite"):
        E.inv_upper_factor(H, 0.01, max_tries=3)


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_grid_and_repack_against_golden(golden, tt):
    """Decoding the committed grid reproduces the reference decoder; re-packing the
    decoded codes reproduces the golden bytes."""
    x = golden["x/heavy"]
    raw = golden[f"raw/heavy/imat/{tt}"]
    nrow, n = x.shape
    dl, ml, lo, hi, sub = E.committed_grid(tt, raw, nrow, n)
    rec = golden[f"rec/heavy/imat/{tt}"]
    # recover the signed codes from the reference reconstruction where dl != 0
    dle = np.repeat(dl, sub, 1)
    mle = np.repeat(ml, sub, 1) if ml is not None else np.zeros_like(dle)
    nz = dle != 0
    codes = np.where(nz, np.rint((rec + mle) / np.where(nz, dle, 1)), 0).astype(np.int32)
    assert codes.min() >= lo and codes.max() <= hi
    assert np.array_equal(np.where(nz, dle * codes.astype(F32) - mle, rec), rec)
    # where dl == 0 the code cannot be read back from rec; take it from the bytes
    packed = K.stored_codes(tt, raw).reshape(nrow, n)
    codes = np.where(nz, codes, packed)
    assert np.array_equal(E.write_codes(tt, raw, codes, nrow, n), raw)


def _scalar_sweep(xp, U, dl, ml, lo, hi, sub, order):
    """Per-row scalar GPTQ recurrence: an independent restatement of the sweep."""
    nrow, n = xp.shape
    codes = np.zeros((nrow, n), np.int32)
    for r in range(nrow):
        t = [F32(v) for v in xp[r]]
        for jj in range(n):
            j = order[jj]
            d = F32(dl[r, j // sub])
            m = F32(ml[r, j // sub]) if ml is not None else F32(0)
            if d == 0:
                q, e = 0, F32(0)
            else:
                q = int(K.rint_magic(np.array([F32(F32(t[jj] + m) / d)]))[0])
                q = min(max(q, lo), hi)
                e = F32(F32(t[jj] - F32(F32(d * F32(q)) - m)) / F32(U[jj, jj]))
            codes[r, j] = q
            for k in range(jj + 1, n):
                t[k] = F32(t[k] - F32(e * U[jj, k]))
    return codes


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_sweep_matches_scalar_recurrence(tt):
    n, nrow = 256, 3
    W = heavy_tailed(nrow, n, seed=7)
    H = correlated_hessian(n, 1024, seed=2)
    order = E.act_order(H)
    U = E.inv_upper_factor(H[np.ix_(order, order)]).astype(F32)
    raw = K.QUANTIZE[tt](W, (np.diag(H) / 1024).astype(F32))
    dl, ml, lo, hi, sub = E.committed_grid(tt, raw, nrow, n)
    xp = W[:, order].copy()
    got = E.sweep(xp.copy(), U, dl, ml, lo, hi, sub, order)
    want = _scalar_sweep(xp, U, dl, ml, lo, hi, sub, order)
    assert np.array_equal(got, want)


def _row_grid(tt, raw_row, n):
    """One row's committed grid, read sub-block by sub-block from its container bytes
    with the golden-pinned field readers: (steps dl[n/sub], offsets ml or None)."""
    sub = K.SUB_W[tt]
    bp = K.BYTES_PER_SB[tt]
    dl, ml = [], []
    for sb in range(n // 256):
        b = raw_row[sb * bp:(sb + 1) * bp][None]
        if tt == "Q2_K":
            d, m = K._half_field(b, 80)[0], K._half_field(b, 82)[0]
            sc = [(int(v) & 0xF, int(v) >> 4) for v in b[0, 0:16]]
        elif tt == "Q3_K":
            d, m = K._half_field(b, 108)[0], None
            sc = [(int(v) - 32, 0) for v in K.unpack_scales_q3(b[:, 96:108])[0]]
        elif tt in ("Q4_K", "Q5_K"):
            d, m = K._half_field(b, 0)[0], K._half_field(b, 2)[0]
            s_, m_ = K.unpack_scales_k4(b[:, 4:16])
            sc = list(zip((int(v) for v in s_[0]), (int(v) for v in m_[0])))
        else:
            d, m = K._half_field(b, 208)[0], None
            sc = [(int(v), 0) for v in b[0, 192:208].view(np.int8)]
        for s_k, m_k in sc:
            dl.append(F32(d * F32(s_k)))
            if m is not None:
                ml.append(F32(m * F32(m_k)))
    return dl, (ml if ml else None)


def _row_ef(x_row, tt, qw, U, order, n_iter, restart_from="x", commit_on="targets"):
    """ef_encode (ef.py:179-218) for ONE row, written from the GPTQ recurrence alone:
    each iteration commits the codec (K.QUANTIZE, golden-pinned) on the current targets,
    reads the row's grid from those bytes, sweeps the visiting order starting again from
    the original weights, and scatters the compensated targets back into storage order.
    Returns (final codes in storage order, the targets the last commit saw).
    ``restart_from`` / ``commit_on`` select the two planted mistakes a test must catch:
    sweeping from the current targets instead of x, and committing every pass on x."""
    n = x_row.size
    sub = K.SUB_W[tt]
    lo, hi = E.GRID[tt][1], E.GRID[tt][2]
    targets = x_row.astype(F32).copy()
    codes = np.zeros(n, np.int64)
    committed_on = None
    for _ in range(n_iter):
        committed_on = (targets if commit_on == "targets" else x_row).astype(F32).copy()
        raw = K.QUANTIZE[tt](committed_on[None], qw)[0]
        dl, ml = _row_grid(tt, raw, n)
        start = x_row if restart_from == "x" else targets
        t = np.array([start[order[jj]] for jj in range(n)], F32)  # visiting order
        for jj in range(n):
            j = order[jj]
            d = dl[j // sub]
            m = ml[j // sub] if ml is not None else F32(0)
            if d == 0:
                q, e = 0, F32(0)
            else:
                q = int(K.rint_magic(np.array([F32(F32(t[jj] + m) / d)]))[0])
                q = min(max(q, lo), hi)
                e = F32(F32(t[jj] - F32(F32(d * F32(q)) - m)) / U[jj, jj])
            codes[j] = q
            # fl(t - fl(e * u)) elementwise: numpy float32 arithmetic, no fused terms
            t[jj + 1:] = t[jj + 1:] - (e * U[jj, jj + 1:]).astype(F32)
        targets = np.empty(n, F32)
        for jj in range(n):
            targets[order[jj]] = t[jj]
    return codes, committed_on


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_ef_loop_matches_row_restatement(tt):
    """The oracle's whole ef_encode loop equals the per-row restatement for n_iter 1-3:
    the codes (read back with the golden-pinned code readers) and the scale fields (the
    codec's own bytes on the targets of the last commit). The two planted mistakes give
    other bytes on the same inputs, so an oracle carrying either one fails this test."""
    n, nrow = (256, 3) if tt in ("Q3_K", "Q6_K") else (512, 2)
    W = heavy_tailed(nrow, n, seed=21)
    H = correlated_hessian(n, 2048, seed=22)
    qw = (np.diag(H) / 2048).astype(F32) if tt != "Q6_K" else None
    order = E.act_order(H, stable=True)
    U = E.inv_upper_factor(H[np.ix_(order, order)]).astype(F32)
    for n_iter in (1, 2, 3):
        raw, rec = E.ef_encode(W, tt, qw, H, n_iter=n_iter, U=U, order=order)
        codes = K.stored_codes(tt, raw).reshape(nrow, n).astype(np.int64)  # signed codes
        for r in range(nrow):
            want, seen = _row_ef(W[r], tt, qw, U, order, n_iter)
            assert np.array_equal(codes[r], want), (n_iter, r)
            commit = K.QUANTIZE[tt](seen[None], qw)[0]
            assert np.array_equal(E.write_codes(tt, commit[None], want[None], 1, n)[0], raw[r])
        assert np.array_equal(rec, K.DEQUANTIZE[tt](raw, n))
        if n_iter == 1:
            continue
        for mistake in ({"restart_from": "targets"}, {"commit_on": "x"}):
            planted = [_row_ef(W[r], tt, qw, U, order, n_iter, **mistake)[0] for r in range(nrow)]
            assert not np.array_equal(codes, np.stack(planted)), (n_iter, mistake)


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_diagonal_hessian_reduces_to_codec(tt):
    """With a diagonal H nothing propagates: every superblock whose sub-block steps are
    all non-zero gets exactly the codec's own requantized bytes."""
    nrow, n = 6, 512
    W = heavy_tailed(nrow, n, seed=11)
    rng = np.random.default_rng(3)
    H = np.diag(rng.uniform(0.5, 4.0, n))
    qw = np.diag(H).astype(F32)
    raw, _ = E.ef_encode(W, tt, qw, H)
    ref = K.QUANTIZE[tt](W, qw)
    dl, *_ = E.committed_grid(tt, ref, nrow, n)
    full = (dl.reshape(nrow * n // 256, -1) != 0).all(1)
    bp = K.BYTES_PER_SB[tt]
    assert full.mean() > 0.9
    assert np.array_equal(raw.reshape(-1, bp)[full], ref.reshape(-1, bp)[full])


@pytest.mark.parametrize("tt", ["Q2_K", "Q3_K", "Q4_K"])
def test_ef_beats_weighted_rtn(tt):
    """test_ef_synthetic.py:30-46: >= 3 % lower tr(dW H dW^T) than weighted RTN."""
    n, nrow, T = 512, 24, 4096
    rng = np.random.default_rng({"Q2_K": 101, "Q3_K": 202, "Q4_K": 303}[tt])
    W = (rng.standard_normal((nrow, n)) ** 3).astype(F32)
    H = correlated_hessian(n, T, seed=0)
    qw = (np.diag(H) / T).astype(F32)
    rtn = K.roundtrip(W, tt, qw)
    _, rec = E.ef_encode(W, tt, qw, H)
    assert E.h_weighted_err(W, rec, H) < 0.97 * E.h_weighted_err(W, rtn, H)


@pytest.mark.parametrize("tt", ["Q2_K", "Q4_K"])
def test_act_order_beats_storage_order(tt):
    """test_ef_synthetic.py:49-68: importance rising with the column index."""
    n, nrow, T = 512, 24, 8192
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((nrow, n)) ** 3).astype(F32)
    var = 1.0 + 8.0 * np.arange(n) / n
    Z = rng.standard_normal((T, n)) * np.sqrt(var)
    Z += 0.4 * Z[:, [0]]
    H = Z.T @ Z
    qw = (np.diag(H) / T).astype(F32)
    _, rec_a = E.ef_encode(W, tt, qw, H, act_order_on=True)
    _, rec_s = E.ef_encode(W, tt, qw, H, act_order_on=False)
    assert E.h_weighted_err(W, rec_a, H) < E.h_weighted_err(W, rec_s, H)


def test_rows_are_independent():
    n, nrow = 512, 8
    W = heavy_tailed(nrow, n, seed=5)
    H = correlated_hessian(n, 2048, seed=4)
    qw = (np.diag(H) / 2048).astype(F32)
    raw, _ = E.ef_encode(W, "Q2_K", qw, H)
    p = np.random.default_rng(0).permutation(nrow)
    raw_p, _ = E.ef_encode(W[p], "Q2_K", qw, H)
    assert np.array_equal(raw_p, raw[p])


def test_hessian_oracle_closed_form():
    import torch
    from oracle import hess_oracle as Ho
    rng = np.random.default_rng(0)
    X = (rng.standard_normal((2048, 96)) * np.exp(rng.standard_normal(96))).astype(np.float32)
    H64 = Ho.xtx(X)
    assert np.array_equal(H64, H64.T)
    Ht = (torch.from_numpy(X).T @ torch.from_numpy(X)).numpy()
    assert Ho.rel_fro(Ht, H64) < 1e-6
    Hb, cnt = Ho.accumulate([X[:1000], X[1000:]])
    assert cnt == 2048 and Ho.rel_fro(Hb, H64) < 1e-12


@pytest.mark.parametrize("shape", [(1, 4), (1, 7), (3, 40), (5, 333), (3, 1000), (2, 4096),
                                   (7, 3072), (100, 256), (9, 8192), (2, 10000), (3, 24581),
                                   (517, 1024), (1024, 3072)])
def test_sq_err_sum_is_numpys_sum(shape):
    """The err-vs-stock statistic's order (coldpress/ef.py:299-300): the oracle's chunked
    pairwise model against numpy's own float32 .sum() of the same terms, bit for bit, for
    totals under one 8192-term chunk, exact multiples, partial last chunks and rows that
    are not multiples of a 128-term leaf; plain left-to-right or one tree over all terms
    gives other bits on some of these."""
    rng = np.random.default_rng(shape[0] * 7919 + shape[1])
    x = (rng.standard_normal(shape) ** 3).astype(np.float32)
    r = (x + rng.standard_normal(shape).astype(np.float32) * 0.1).astype(np.float32)
    w = np.abs(rng.standard_normal(shape[1])).astype(np.float32)
    for ww in (w, None):
        want = (((r - x) ** 2) * (ww if ww is not None else np.ones(shape[1], np.float32))).sum()
        got = E.sq_err_sum(r, x, ww)
        assert np.float32(got).tobytes() == want.tobytes(), (shape, got, want)


def test_sq_err_sum_order_is_not_a_plain_sum():
    """A planted mistake the model must not admit: summing the chunks' terms in one
    sequential pass (or one pairwise tree over everything) differs from numpy's result
    on this input, so the test above distinguishes the orders."""
    rng = np.random.default_rng(5)
    t = (rng.standard_normal(3 * 8192 + 1000) ** 3).astype(np.float32)
    want = t.sum()
    seq = np.float32(0.0)
    for v in t:
        seq = np.float32(seq + v)
    assert seq.tobytes() != want.tobytes()
    assert np.float32(E.pairwise_f32(t)).tobytes() != want.tobytes()
    assert np.float32(E.full_sum_f32(t)).tobytes() == want.tobytes()


def test_single_linear_bytes_do_not_follow_the_factors_last_bits():
    """The GPU factor's float64 U differs from LAPACK's (another algorithm, other roundings)
    by a few ulps; what reaches the sweep is U cast to float32. On the single-Linear workload
    (1024 x 1024 Q2_K, qw = diag H), relative noise of 1e-13 on the oracle's float64 U moves
    at most a handful of float32 entries and leaves every EF byte as it was, which is why
    the byte-exact GPU test of that workload holds with the GPU's own factor."""
    from perm_amd.workloads import single_linear
    W, _X, H = single_linear(seed=0)
    qw = np.diag(H).astype(np.float32)
    order = E.act_order(H, stable=True)
    U64 = E.inv_upper_factor(H[np.ix_(order, order)], 0.01, log=False)
    raw0, _ = E.ef_encode(W, "Q2_K", qw, H, n_iter=2, U=U64.astype(np.float32), order=order)
    rng = np.random.default_rng(5)
    Up = np.triu(U64 * (1 + 1e-13 * rng.standard_normal(U64.shape))).astype(np.float32)
    assert int((Up != U64.astype(np.float32)).sum()) <= 8
    raw, _ = E.ef_encode(W, "Q2_K", qw, H, n_iter=2, U=Up, order=order)
    assert np.array_equal(raw, raw0)
