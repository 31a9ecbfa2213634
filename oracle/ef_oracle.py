"""EF encoder oracle (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates the encoder core of coldpress/ef.py:46-218: the damped inverse-Hessian
upper Cholesky factor, decoding committed container bytes into the per-sub-block
grid, writing integer codes back into the bytes, and the GPTQ column sweep with
act_order. The float32 arithmetic of the sweep follows the reference op for op
(per column: divide, magic-add rounding, clip, f32 multiply then subtract for
every later column), so it reproduces the reference's codes exactly.

Pinning (no byte vectors of the reference's ef.py exist -- its module needs the
absent pip ``gguf`` package, so it is never imported):
* ``inv_upper_factor`` makes the same numpy calls as the reference and is
  pinned by the closed form chol(inv(H + lambda I))^T (the reference's own
  test_ef_cholesky_robust.py:51-64 known answer) and by U^T U = inv(H + lambda I);
* ``committed_grid`` / ``write_codes`` are pinned by the golden container bytes
  (decode of the committed grid equals the reference decoder, repack of the
  decoded codes reproduces the golden bytes);
* ``ef_encode`` is pinned by a scalar, per-row re-derivation of the GPTQ
  recurrence on small inputs, by the closed form for a diagonal H (no error
  propagates, so the codes are the plain nearest codes on the committed grid),
  and by the reference's invariants (EF beats weighted RTN in tr(dW H dW^T) by
  >= 3 %, act_order beats storage order when importance grows with the index).
"""
import sys

import numpy as np

from . import kquant_oracle as kq

F32 = np.float32

# (sub-block width, lowest code, highest code, has a min term) -- ef.py:87-127
GRID = {"Q2_K": (16, 0, 3, True), "Q3_K": (16, -4, 3, False), "Q4_K": (32, 0, 15, True),
        "Q5_K": (32, 0, 31, True), "Q6_K": (16, -32, 31, False)}


class NotPositiveDefinite(np.linalg.LinAlgError):
    pass


def damp_shift(H, damp):
    """Diagonal load added on each attempt: damp * mean(diag H) + 1e-8, with the mean
    replaced by 1 when it is not positive (ef.py:64-69)."""
    mean_diag = float(np.mean(np.diag(H)))
    base = mean_diag if mean_diag > 0.0 else 1.0
    return damp * base + 1e-8


def inv_upper_factor(H, damp=0.01, max_tries=6, log=True):
    """Upper U with U^T U = inv(H + lambda I), float64 (ef.py:46-84).

    lambda = damp * mean(diag H) + 1e-8; on a failed factorization damp is
    multiplied by 10, up to ``max_tries`` attempts, then LinAlgError."""
    n = H.shape[0]
    H = H.astype(np.float64).copy()
    d = damp
    for attempt in range(max_tries):
        Hd = H.copy()
        Hd[np.diag_indices(n)] += damp_shift(H, d)
        try:
            Hinv = np.linalg.inv(Hd)
            Hinv = (Hinv + Hinv.T) / 2
            U = np.linalg.cholesky(Hinv).T
        except np.linalg.LinAlgError:
            d *= 10.0
            continue
        if attempt and log:
            print(f"[ef] inverse factor: damp escalated {damp:g} -> {d:g} in {attempt} "
                  f"step(s) (n={n})", file=sys.stderr, flush=True)
        return np.ascontiguousarray(U)
    raise np.linalg.LinAlgError(
        f"cholesky_inv_upper: inv(H) not positive definite even after escalating damp to "
        f"{d / 10.0:g} (n={n}); Hessian appears degenerate")


def committed_grid(tt, raw, nrow, n):
    """Per (row, sub-block) step dl and offset ml (None for the symmetric types) of the
    committed container (ef.py:87-127). Returns (dl, ml, lo, hi, width)."""
    sub, lo, hi, affine = GRID[tt]
    bp = kq.BYTES_PER_SB[tt]
    b = raw.reshape(-1, bp)
    if tt == "Q2_K":
        d, dm = kq._half_field(b, 80), kq._half_field(b, 82)
        s, m = (b[:, 0:16] & 0xF).astype(F32), (b[:, 0:16] >> 4).astype(F32)
    elif tt == "Q3_K":
        d, dm = kq._half_field(b, 108), None
        s, m = (kq.unpack_scales_q3(b[:, 96:108]) - 32).astype(F32), None
    elif tt in ("Q4_K", "Q5_K"):
        d, dm = kq._half_field(b, 0), kq._half_field(b, 2)
        si, mi = kq.unpack_scales_k4(b[:, 4:16])
        s, m = si.astype(F32), mi.astype(F32)
    elif tt == "Q6_K":
        d, dm = kq._half_field(b, 208), None
        s, m = b[:, 192:208].copy().view(np.int8).astype(F32), None
    else:
        raise ValueError(tt)
    dl = (d[:, None] * s).reshape(nrow, -1)
    ml = (dm[:, None] * m).reshape(nrow, -1) if affine else None
    return dl, ml, lo, hi, sub


def write_codes(tt, raw, codes, nrow, n):
    """Container bytes with the integer codes replaced, scales untouched (ef.py:130-176).
    ``codes`` are the signed sweep codes (lo..hi)."""
    bp = kq.BYTES_PER_SB[tt]
    b = raw.reshape(-1, bp).copy()
    L = codes.reshape(-1, kq.QK_K).astype(np.int32)
    if tt == "Q2_K":
        b[:, 16:80] = kq.pack_2bit(L)
    elif tt == "Q3_K":
        b[:, 0:32], b[:, 32:96] = kq.pack_q3_codes(L + 4)
    elif tt == "Q4_K":
        b[:, 16:144] = kq.pack_nibbles(L)
    elif tt == "Q5_K":
        b[:, 16:48], b[:, 48:176] = kq.pack_q5_codes(L)
    elif tt == "Q6_K":
        b[:, 0:128], b[:, 128:192] = kq.pack_q6_codes(L + 32)
    else:
        raise ValueError(tt)
    return b.reshape(nrow, -1)


def act_order(H, enabled=True, stable=False):
    """Column visiting order: descending diag(H) (ef.py:187). The reference uses
    numpy's default (unstable) argsort; ``stable`` breaks ties by index instead,
    which is what the GPU path does."""
    n = H.shape[0]
    if not enabled:
        return np.arange(n)
    return np.argsort(-np.diag(H), kind="stable" if stable else None)


def sweep(xp, U, dl, ml, lo, hi, sub, order):
    """One GPTQ pass over the act-ordered columns (ef.py:197-213).

    xp: [nrow, n] f32 weights already in visiting order (modified in place into the
    error-compensated targets). Returns the codes [nrow, n] int32 in STORAGE order."""
    nrow, n = xp.shape
    L = np.zeros((nrow, n), np.int32)
    diag = np.diag(U).copy()
    for jj in range(n):
        j = order[jj]
        dlj = dl[:, j // sub]
        mlj = ml[:, j // sub] if ml is not None else F32(0)
        nz = dlj != 0
        with np.errstate(divide="ignore", invalid="ignore"):
            q = kq.rint_magic((xp[:, jj] + mlj) / np.where(nz, dlj, F32(1)))
        q = np.where(nz, np.clip(q, lo, hi), 0)
        L[:, j] = q
        r = xp[:, jj] - (dlj * q.astype(F32) - mlj)
        e = np.where(nz, r / diag[jj], F32(0)).astype(F32)
        if jj + 1 < n:
            xp[:, jj + 1:] -= np.outer(e, U[jj, jj + 1:])
    return L


def ef_encode(x, ttype, qw, H, n_iter=2, damp=0.01, act_order_on=True, U=None,
              stable_order=False, order=None):
    """GPTQ error feedback into committed k-quant containers (ef.py:179-218).

    Returns (raw bytes [nrow, row_bytes], recon [nrow, n] f32). ``U`` lets a test
    supply the float32 factor directly (in visiting order), ``order`` the
    visiting order (then H is not read)."""
    nrow, n = x.shape
    if order is None:
        order = act_order(H, act_order_on, stable_order)
    if U is None:
        U = inv_upper_factor(H[np.ix_(order, order)], damp).astype(F32)
    w_cur = x.astype(F32).copy()
    raw = None
    for _ in range(n_iter):
        raw = kq.QUANTIZE[ttype](w_cur, qw)
        dl, ml, lo, hi, sub = committed_grid(ttype, raw, nrow, n)
        xp = x.astype(F32)[:, order].copy()
        L = sweep(xp, U, dl, ml, lo, hi, sub, order)
        raw = write_codes(ttype, raw, L, nrow, n)
        w_cur = np.empty_like(xp)
        w_cur[:, order] = xp
    return raw, kq.DEQUANTIZE[ttype](raw, n)


def h_weighted_err(W, What, H):
    """tr((What - W) H (What - W)^T) in float64 (tests/test_ef_synthetic.py:20-22)."""
    D = (What - W).astype(np.float64)
    return float(np.einsum("ri,ij,rj->", D, H, D))


# ---------------------------------------------------------------- err-vs-stock statistic

NP_CHUNK = 8192  # elements per inner-loop call of numpy's full reduction of a contiguous array


def pairwise_f32(a):
    """numpy's float32 pairwise sum of a 1-D array (its pairwise_sum: under 8 values left
    to right, up to 128 values eight interleaved accumulators and their tree plus the
    remainder, above that split at n/2 rounded down to a multiple of 8)."""
    n = len(a)
    if n < 8:
        s = F32(-0.0)
        for v in a:
            s = F32(s + v)
        return s
    if n <= 128:
        r = a[:8].astype(F32).copy()
        m = n - n % 8
        for i in range(8, m, 8):
            r = (r + a[i:i + 8]).astype(F32)
        s = F32(F32(F32(r[0] + r[1]) + F32(r[2] + r[3])) + F32(F32(r[4] + r[5]) + F32(r[6] + r[7])))
        for i in range(m, n):
            s = F32(s + a[i])
        return s
    n2 = n // 2
    n2 -= n2 % 8
    return F32(pairwise_f32(a[:n2]) + pairwise_f32(a[n2:]))


def full_sum_f32(a):
    """``a.sum()`` of a contiguous float32 array with no axis, in numpy's order: the
    flattened array in chunks of 8192 elements, each summed pairwise, the chunk sums
    added left to right from 0.0. Full chunks are evaluated vectorized (64 leaves of 128,
    eight interleaved accumulators each, then a balanced tree)."""
    f = np.ascontiguousarray(a, dtype=F32).reshape(-1)
    nfull = len(f) // NP_CHUNK
    total = F32(0.0)
    if nfull:
        leaves = f[:nfull * NP_CHUNK].reshape(nfull, 64, 16, 8)
        r = leaves[:, :, 0, :].copy()
        for k in range(1, 16):
            r = (r + leaves[:, :, k, :]).astype(F32)
        s = ((r[..., 0] + r[..., 1]) + (r[..., 2] + r[..., 3])) + \
            ((r[..., 4] + r[..., 5]) + (r[..., 6] + r[..., 7]))
        while s.shape[1] > 1:
            s = (s[:, 0::2] + s[:, 1::2]).astype(F32)
        for v in s[:, 0]:
            total = F32(total + v)
    if len(f) % NP_CHUNK:
        total = F32(total + pairwise_f32(f[nfull * NP_CHUNK:]))
    return total


def sq_err_sum(recon, x, w):
    """(((recon - x) ** 2) * w).sum() of coldpress/ef.py:299-300 (float32 terms, numpy's
    summation order); w [n] broadcast over rows, None for ones."""
    d = (np.asarray(recon, F32) - np.asarray(x, F32)).astype(F32)
    t = (d * d).astype(F32)
    if w is not None:
        t = (t * np.asarray(w, F32)).astype(F32)
    return full_sum_f32(t)
