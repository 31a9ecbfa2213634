"""ctypes binding to libcoldpress_hip.so plus tensor plumbing.

The library is loaded after ``import torch`` so that it binds to the HIP runtime
torch already loaded (same soname), and device pointers from torch's allocator
are valid in it. Nothing here computes on the CPU: a missing library or a
missing GPU raises.
"""
import ctypes
import os

import numpy as np
import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcoldpress_hip.so")

CP_OK, CP_ERR_SHAPE, CP_ERR_TTYPE, CP_ERR_NOT_PD = 0, -1, -2, -3
CP_ERR_HIP, CP_ERR_ARG, CP_ERR_ALIGN, CP_ERR_WORKSPACE, CP_ERR_INDEX = -4, -5, -6, -7, -8
CP_ERR_TIMEOUT = -9

TTYPE = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}

_i64, _i32, _vp, _f64 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_double
_sz = ctypes.c_size_t

CP_EF_EXACT = 0
CP_EF_MFMA = 1
CP_EF_EXACT_VALU = 2


class EfTensor(ctypes.Structure):
    """struct cp_ef_tensor (include/coldpress_hip.h)."""
    _fields_ = [("ttype", ctypes.c_int), ("nrow", ctypes.c_int64), ("n", ctypes.c_int64),
                ("x", _vp), ("qw", _vp), ("U", _vp), ("order", _vp), ("raw", _vp),
                ("recon", _vp)]


_ef_p = ctypes.POINTER(EfTensor)


class ErrTensor(ctypes.Structure):
    """struct cp_err_tensor (include/coldpress_hip.h)."""
    _fields_ = [("ttype", ctypes.c_int), ("x_dtype", ctypes.c_int), ("nrow", ctypes.c_int64),
                ("n", ctypes.c_int64), ("x", _vp), ("qw", _vp), ("perm", _vp), ("wvec", _vp),
                ("rows", _vp), ("rows_used", ctypes.c_int64)]


_err_p = ctypes.POINTER(ErrTensor)


class ColTensor(ctypes.Structure):
    """struct cp_col_tensor (include/coldpress_hip.h)."""
    _fields_ = [("x", _vp), ("x_dtype", ctypes.c_int), ("nrow", ctypes.c_int64),
                ("n", ctypes.c_int64), ("out", _vp)]


_col_p = ctypes.POINTER(ColTensor)

# name -> (restype, argtypes); every symbol include/coldpress_hip.h declares
SIGNATURES = {
    "cp_last_error": (ctypes.c_char_p, []),
    "cp_kq_block_bytes": (_i32, [_i32]),
    "cp_kq_quantize": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _vp]),
    "cp_kq_dequantize": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp]),
    "cp_act_order": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp]),
    "cp_chol_ws_bytes": (_sz, [_i64, _i32]),
    "cp_chol_inv_upper": (_i32, [_vp, _i32, _i64, _i32, _vp, _f64, _i32, _vp, _i32, _vp, _vp,
                                 _sz, _vp]),
    "cp_chol_inv_upper_async": (_i32, [_vp, _i32, _i64, _i32, _vp, _f64, _vp, _i32, _vp, _vp,
                                       _sz, _vp]),
    "cp_ef_ws_bytes": (_sz, [_ef_p, _i32]),
    "cp_ef_encode_batch": (_i32, [_ef_p, _i32, _i32, _i32, _vp, _sz, _vp]),
    "cp_ef_encode": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _sz,
                            _vp]),
    "cp_ef_encode_noalloc": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _vp, _i32, _vp, _vp,
                                    _vp]),
    "cp_ef_noalloc_max_ws_bytes": (_sz, []),
    "cp_ef_read_status": (_i32, [_vp, _vp]),
    "cp_ef_wait_limit": (None, [_i32]),
    "cp_hess_accum": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp]),
    "cp_hess_accum_batch": (_i32, [_vp, _vp, _i32, _i32, _i64, _i64, _vp]),
    "cp_hess_ws_bytes": (_sz, [_i32, _i32, _i64, _i64]),
    "cp_hess_accum_batch_ws": (_i32, [_vp, _vp, _i32, _i32, _i64, _i64, _vp, _sz, _vp]),
    "cp_ef_profile": (None, [_i32]),
    "cp_ef_phase_ms": (_i32, [_vp, _i32]),
    "cp_ef_last_sweep": (_i32, [_vp, _vp]),
    "cp_chol_compact_tiles": (None, [_i32]),
    "cp_chol_wait_limit": (None, [_i32]),
    "cp_permute_gather": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "cp_lin_extract": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _vp]),
    "cp_lin_reconstruct": (_i32, [_i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "cp_lin_reconstruct_grad": (_i32, [_i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "cp_lin_write_back": (_i32, [_i32, _vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "cp_h2_pack": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "cp_h2_expand": (_i32, [_vp, _i32, _i64, _f64, _vp, _vp, _vp]),
    "cp_tensor_err_ws_bytes": (_sz, [_err_p, _i32]),
    "cp_tensor_err_batch": (_i32, [_err_p, _i32, _vp, _sz, _vp, _vp]),
    "cp_err_profile": (None, [_i32]),
    "cp_err_phase_ms": (_i32, [_vp, _i32]),
    "cp_col_sums_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "cp_col_sums_batch_ws_bytes": (_sz, [_col_p, _i32, _i64]),
    "cp_col_sq_sums_batch": (_i32, [_col_p, _i32, _i64, _i32, _vp, _sz, _vp]),
    "cp_col_sq_sums": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "cp_col_log_rms": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "cp_check_division": (_i32, [_i64, ctypes.c_uint64, _vp, _vp]),
    "cp_sq_err_ws_bytes": (_sz, [_i64, _i64]),
    "cp_sq_err_sum": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
}


def workspace(nbytes, device="cuda"):
    """A 256-byte aligned device workspace (torch's caching allocator aligns to 512)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)

_lib = None


class HipError(RuntimeError):
    """A HIP runtime failure reported by the library."""


class WaitTimeout(RuntimeError):
    """A device-side bounded wait gave up: that call's results are not valid."""


class SweepTimeout(WaitTimeout):
    """An EF sweep wave gave up a bounded wait: that call's bytes are not valid."""


class FactorTimeout(WaitTimeout):
    """A factorization chain step gave up waiting for its diagonal block: that U is not valid."""


def load(require_gpu=True):
    """The loaded library. Raises if it is not built, or (by default) if no GPU is visible."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m perm_amd.build` "
                               f"(there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    if require_gpu and not torch.cuda.is_available():
        raise RuntimeError("perm_amd needs a HIP device (torch.cuda.is_available() is False)")
    return _lib


def check(status, exc_for_shape=ValueError, exc_for_timeout=SweepTimeout):
    """Map a cp_status to the exception the reference raises for the same condition."""
    if status >= 0:
        return status
    msg = (_lib.cp_last_error() or b"").decode(errors="replace")
    if status == CP_ERR_NOT_PD:
        raise np.linalg.LinAlgError(msg)
    if status == CP_ERR_SHAPE:
        raise exc_for_shape(msg)
    if status == CP_ERR_TTYPE:
        raise KeyError(msg)
    if status == CP_ERR_HIP:
        raise HipError(msg)
    if status == CP_ERR_INDEX:
        raise IndexError(msg)
    if status == CP_ERR_TIMEOUT:
        raise exc_for_timeout(msg)
    raise ValueError(f"{msg} (status {status})")


def check_index(p, size, what="index", permutation=False):
    """An index array checked on the host before anything is launched with it.

    numpy's rules for an index into an axis of ``size``: every entry lies in
    [-size, size) and negative entries count from the end (IndexError otherwise, as
    numpy's fancy indexing raises). With ``permutation`` every position must occur
    exactly once, as an act order or a channel permutation must (IndexError
    otherwise). ``p``: a numpy array, a sequence or a torch tensor; a CUDA tensor is
    checked with device reductions and one synchronization. Returns an int32 array
    (or tensor, on p's device) with negative entries resolved; the shape is kept."""
    if isinstance(p, torch.Tensor):
        if (p.is_floating_point() or p.is_complex() or p.dtype == torch.bool) and p.numel():
            raise IndexError(f"{what}: indices must be integers, got {p.dtype}")
        t = p.to(torch.int64)
        if t.numel():
            lo, hi = (int(v) for v in torch.stack([t.min(), t.max()]).cpu())
            if lo < -size or hi >= size:
                raise IndexError(f"{what}: index {lo if lo < -size else hi} is out of bounds "
                                 f"for axis 0 with size {size}")
        t = torch.where(t < 0, t + size, t)
        if permutation and t.numel():
            rows = t.reshape(-1, t.shape[-1]) if t.dim() else t.reshape(1, 1)
            ok = rows.shape[-1] == size and bool(
                torch.equal(torch.sort(rows, dim=-1).values,
                            torch.arange(size, device=t.device).expand_as(rows)))
            if not ok:
                raise IndexError(f"{what} is not a permutation of {size}")
        return t.to(torch.int32)
    a = np.asarray(p)
    if a.dtype.kind not in "iu" and a.size:
        raise IndexError(f"{what}: indices must be integers, got {a.dtype}")
    a = a.astype(np.int64)
    if a.size and (int(a.min()) < -size or int(a.max()) >= size):
        bad = int(a.min()) if int(a.min()) < -size else int(a.max())
        raise IndexError(f"{what}: index {bad} is out of bounds for axis 0 with size {size}")
    a = np.where(a < 0, a + size, a)
    if permutation and a.size:
        rows = a.reshape(-1, a.shape[-1]) if a.ndim else a.reshape(1, 1)
        if rows.shape[-1] != size or not np.array_equal(np.sort(rows, axis=-1),
                                                        np.broadcast_to(np.arange(size), rows.shape)):
            raise IndexError(f"{what} is not a permutation of {size}")
    return a.astype(np.int32)


def stream_ptr():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def to_device(a, dtype):
    """(contiguous device tensor of ``dtype``, True if ``a`` came from the host)."""
    if isinstance(a, torch.Tensor):
        host = not a.is_cuda
        t = a.to(device="cuda", dtype=dtype, non_blocking=False)
        return t.contiguous(), host
    arr = np.ascontiguousarray(np.asarray(a))
    return torch.from_numpy(arr).to(device="cuda", dtype=dtype).contiguous(), True


def to_host(t):
    return t.cpu().numpy()
