"""Hessian X^T X oracle. TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

coldpress/hessians.py:137-154 accumulates, per hooked Linear and per batch,
``x.float().T @ x`` into a float32 [d, d] accumulator, and counts rows. The
oracle is the float64 closed form of the same sum (the parity gate is 1e-5
relative Frobenius, which float32 accumulation of any order meets by a wide
margin at the batch sizes used here).

h2_pack / h2_expand restate the storage arithmetic of hessians.py:163-243. Pins: the
expectations of the reference's own storage tests (test_hessian_fp16.py: exact diagonal,
off-diagonal equal to float16(float32(H)) when unscaled and within float16 epsilon, finite
storage of a Hessian far above the float16 range, the float32-only format unchanged), which
tests/test_gguf.py (test_h2_oracle_*) restates.
"""
import numpy as np


def xtx(X):
    """sum_t x_t x_t^T in float64 for X [N, d] (any float dtype; bf16 arrives as float32)."""
    X = np.asarray(X, dtype=np.float64)
    return X.T @ X


def accumulate(batches):
    """(H float64, row count) over an iterable of [N_i, d] batches (hessians.py:147-153)."""
    H, cnt = None, 0
    for X in batches:
        X = np.asarray(X).reshape(-1, np.asarray(X).shape[-1])
        h = xtx(X)
        H = h if H is None else H + h
        cnt += X.shape[0]
    return H, cnt


def rel_fro(A, B):
    """||A - B||_F / ||B||_F in float64."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    return float(np.linalg.norm(A - B) / np.linalg.norm(B))


# ------------------------------------------------------------------ H2 storage
# hessians.py:163-243: float16 off-diagonal over a per-matrix scale, exact float32 diagonal.

FP16_SAFE_MAX = 32768.0


def h2_pack(H):
    """(H16, diag32, hscale) of the stored form (hessians.py:180-194)."""
    H = np.asarray(H, dtype=np.float32)
    diag32 = np.ascontiguousarray(np.diag(H)).astype(np.float32)
    amax = float(np.max(np.abs(H))) if H.size else 0.0
    hscale = amax / FP16_SAFE_MAX if amax > FP16_SAFE_MAX else 1.0
    H16 = (H / np.float32(hscale)).astype(np.float16)
    return H16, diag32, np.float32(hscale)


def h2_expand(H16, hscale=None, diag32=None):
    """float64 H from the stored form (hessians.py:234-241); hscale / diag32 None for the
    older formats."""
    H = np.asarray(H16).astype(np.float64)
    if hscale is not None:
        H *= float(hscale)
    if diag32 is not None:
        np.fill_diagonal(H, np.asarray(diag32).astype(np.float64))
    return H
