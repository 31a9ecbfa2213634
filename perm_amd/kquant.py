"""GGUF container codec (k-quants and Q8_0) on the GPU, with the API of
coldpress/kquant.py.

``QUANTIZE[tt](x, qw)`` and ``DEQUANTIZE[tt](raw, n)`` keep the reference's
signatures and results (coldpress/kquant.py:732-741): bit-identical container
bytes and reconstructions. Inputs may be numpy arrays (results come back as
numpy) or torch tensors (results stay on the device).

x: [nrow, n] float32, n % 256 == 0 (n % 32 == 0 for Q8_0); qw: [n] float32
importance (imatrix means) or None, ignored by Q8_0. The same qw applies to
every row.
"""
import torch

from . import _lib

QK_K = 256
# k-quant superblocks: 256 weights each
BYTES_PER_SB = {"Q2_K": 84, "Q3_K": 110, "Q4_K": 144, "Q5_K": 176, "Q6_K": 210}
SUB_W = {"Q2_K": 16, "Q3_K": 16, "Q4_K": 32, "Q5_K": 32, "Q6_K": 16}
# every container: (weights, bytes) per block
BLOCK = {**{tt: (QK_K, b) for tt, b in BYTES_PER_SB.items()}, "Q8_0": (32, 34)}


def row_bytes(ttype, n):
    """Container bytes of one row of n weights."""
    w, b = BLOCK[ttype]
    return (n // w) * b


def quantize_dev(ttype, x, qw=None, out=None):
    """Device-side encode: x, qw (or None) contiguous float32 CUDA tensors; returns
    (or fills) a uint8 CUDA tensor [nrow, row_bytes(ttype, n)]."""
    lib = _lib.load()
    nrow, n = x.shape
    if out is None:
        out = torch.empty((nrow, row_bytes(ttype, n)), dtype=torch.uint8, device=x.device)
    st = lib.cp_kq_quantize(_lib.TTYPE[ttype], _lib.ptr(x), nrow, n, _lib.ptr(qw),
                            _lib.ptr(out), _lib.stream_ptr())
    _lib.check(st, AssertionError if ttype == "Q2_K" else ValueError)
    return out


def dequantize_dev(ttype, raw, n, out=None):
    lib = _lib.load()
    nrow = raw.shape[0]
    if out is None:
        out = torch.empty((nrow, n), dtype=torch.float32, device=raw.device)
    st = lib.cp_kq_dequantize(_lib.TTYPE[ttype], _lib.ptr(raw), nrow, n, _lib.ptr(out),
                              _lib.stream_ptr())
    _lib.check(st)
    return out


def _quantizer(ttype):
    def quantize(x, qw=None):
        xd, host = _lib.to_device(x, torch.float32)
        if xd.dim() != 2:
            raise ValueError("x must be [nrow, n_per_row]")
        if xd.shape[0] == 0:  # the reference's out.reshape(nrow, -1) fails on zero rows
            raise ValueError("cannot encode an empty tensor (zero rows)")
        qd = None
        if qw is not None and ttype != "Q8_0":  # Q8_0 has no weighted path (kquant.py:706)
            qd, _ = _lib.to_device(qw, torch.float32)
            qd = qd.reshape(-1)
            if qd.numel() != xd.shape[1]:
                raise ValueError(f"qw has {qd.numel()} entries for rows of {xd.shape[1]}")
        out = quantize_dev(ttype, xd, qd)
        return _lib.to_host(out) if host else out
    quantize.__name__ = f"quantize_{ttype.lower()}"
    return quantize


def _dequantizer(ttype):
    def dequantize(raw, n_per_row):
        rd, host = _lib.to_device(raw, torch.uint8)
        rd = rd.reshape(rd.shape[0], -1) if rd.numel() else rd.reshape(rd.shape[0], 0)
        y = dequantize_dev(ttype, rd, int(n_per_row))
        return _lib.to_host(y) if host else y
    dequantize.__name__ = f"dequantize_{ttype.lower()}"
    return dequantize


QUANTIZE = {tt: _quantizer(tt) for tt in BLOCK}
DEQUANTIZE = {tt: _dequantizer(tt) for tt in BLOCK}


def roundtrip(x, ttype, qw=None):
    """quantize then dequantize; returns the reconstruction (coldpress/kquant.py:738-741)."""
    raw = QUANTIZE[ttype](x, qw)
    n = x.shape[1]
    return DEQUANTIZE[ttype](raw, n)
