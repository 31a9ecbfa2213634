"""Hessian X^T X oracle. TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

coldpress/hessians.py:137-154 accumulates, per hooked Linear and per batch,
``x.float().T @ x`` into a float32 [d, d] accumulator, and counts rows. The
oracle is the float64 closed form of the same sum (the parity gate is 1e-5
relative Frobenius, which float32 accumulation of any order meets by a wide
margin at the batch sizes used here).
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
