"""The PERM container objective on the GPU, with the API of coldpress/perm/objective.py.

  tensor_err(x, ttype, qw, perm=None, wvec=None, rows_sample=None, seed=0)
      objective.py:17-39: the (weighted) squared reconstruction error of x[:, perm]
      at container ttype; bit-identical to the reference.
  col_log_rms(x, row_step=32768)
      objective.py:42-49: per-column log-RMS; bit-identical to the reference.

plus ``tensor_err_many``, which evaluates many tensors in one GPU pass (the form the
space-map optimizer uses: one pass per candidate permutation).

x may be a numpy array or a torch tensor, float16 (GGUF F16 weights) or float32;
device tensors are used in place. The row sample is drawn on the host with numpy's
Generator exactly as the reference draws it; everything of size nrow x n runs on the
GPU (gather, codec, column sums, weighted total).
"""
import numpy as np
import torch

from . import _lib
from .kquant import BLOCK

PASSTHROUGH = ("F16", "F32", "BF16")


def sample_rows(nrow, rows_sample, seed=0):
    """The sorted row sample of objective.py:21-24, or None when every row is used."""
    if rows_sample and nrow > rows_sample:
        rng = np.random.default_rng(seed)
        return np.sort(rng.choice(nrow, rows_sample, replace=False))
    return None


_SAMPLES = {}


def _sample_dev(nrow, rows_sample, seed, device):
    """Device int32 copy of sample_rows (drawn once per (nrow, rows_sample, seed))."""
    if not (rows_sample and nrow > rows_sample):
        return None
    key = (int(nrow), int(rows_sample), int(seed), str(device))
    t = _SAMPLES.get(key)
    if t is None:
        if len(_SAMPLES) > 64:
            _SAMPLES.clear()
        idx = sample_rows(nrow, rows_sample, seed)
        t = _SAMPLES[key] = torch.from_numpy(idx.astype(np.int32)).to(device)
    return t


def weights_dev(x):
    """(contiguous device tensor of float16 or float32, x_dtype code 1 / 0)."""
    if isinstance(x, torch.Tensor):
        t = x if x.is_cuda else x.cuda()
        if t.dtype not in (torch.float16, torch.float32):
            t = t.to(torch.float32)
        return t.contiguous(), 1 if t.dtype == torch.float16 else 0
    a = np.asarray(x)
    if a.dtype not in (np.float16, np.float32):
        a = a.astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda(), 1 if a.dtype == np.float16 else 0


def index_dev(p, n, what="perm"):
    """A column index as a device int32 tensor. Host arrays are range-checked here
    (IndexError, as numpy's fancy indexing raises); device tensors are checked by the
    kernels, which never dereference an index out of range and report it (the
    result comes back NaN and tensor_err_many raises IndexError). Negative indices
    count from the end in both cases."""
    if isinstance(p, torch.Tensor):
        t = p.reshape(-1)
        if not (t.is_cuda and t.dtype == torch.int32):
            t = t.to(device="cuda", dtype=torch.int32)
    else:
        a = np.asarray(p).reshape(-1)
        if a.size and (int(a.min()) < -n or int(a.max()) >= n):
            raise IndexError(f"{what} index out of range for {n} columns")
        t = torch.from_numpy(a.astype(np.int32)).cuda()
    if t.numel() != n:
        raise ValueError(f"{what} has {t.numel()} entries for {n} columns")
    return t.contiguous()


def _vec_dev(v, n, dtype, what):
    t = v.to(device="cuda", dtype=dtype) if isinstance(v, torch.Tensor) else \
        torch.from_numpy(np.ascontiguousarray(np.asarray(v, dtype=np.float64 if dtype == torch.float64
                                                          else np.float32))).cuda()
    t = t.reshape(-1).contiguous()
    if t.numel() != n:
        raise ValueError(f"{what} has {t.numel()} entries for {n} columns")
    return t


def tensor_err_many(items):
    """tensor_err for every item (a dict of tensor_err's keyword arguments: x, ttype,
    qw, perm, wvec, rows_sample, seed) in one GPU pass. Returns a list of floats."""
    lib = _lib.load()
    out_vals = [0.0] * len(items)
    structs, keep, slots = [], [], []
    for k, it in enumerate(items):
        tt = it["ttype"]
        if tt in PASSTHROUGH:
            continue
        if tt not in BLOCK:
            raise ValueError(f"no encoder for {tt}")
        xd, code = weights_dev(it["x"])
        if xd.dim() != 2:
            raise ValueError("x must be [nrow, n]")
        nrow, n = xd.shape
        bw = BLOCK[tt][0]
        if n % bw:
            exc = AssertionError if tt == "Q2_K" else ValueError
            raise exc(f"row length {n} is not a multiple of {bw}")
        rows = _sample_dev(nrow, it.get("rows_sample"), it.get("seed", 0), xd.device)
        perm = index_dev(it["perm"], n, "perm") if it.get("perm") is not None else None
        qw = it.get("qw")
        # Q8_0's codec ignores qw; the error is still weighted by it (objective.py:37-38)
        qd = _vec_dev(qw, n, torch.float32, "qw") if qw is not None else None
        wv = it.get("wvec")
        if wv is None and qw is not None and str(getattr(qw, "dtype", "")) not in (
                "float32", "torch.float32"):
            wv = qw  # the codec reads qw as float32; the error weights keep its own precision
        wd = _vec_dev(wv, n, torch.float64, "wvec") if wv is not None else None
        keep += [xd, rows, perm, qd, wd]
        structs.append(_lib.ErrTensor(_lib.TTYPE[tt], code, nrow, n, xd.data_ptr(),
                                      qd.data_ptr() if qd is not None else None,
                                      perm.data_ptr() if perm is not None else None,
                                      wd.data_ptr() if wd is not None else None,
                                      rows.data_ptr() if rows is not None else None,
                                      rows.numel() if rows is not None else 0))
        slots.append(k)
    if not structs:
        return out_vals
    arr = (_lib.ErrTensor * len(structs))(*structs)
    nbytes = lib.cp_tensor_err_ws_bytes(arr, len(structs))
    ws = _lib.workspace(nbytes, keep[0].device)
    out = torch.empty(len(structs), dtype=torch.float64, device=keep[0].device)
    st = lib.cp_tensor_err_batch(arr, len(structs), _lib.ptr(ws), ws.numel(), _lib.ptr(out),
                                 _lib.stream_ptr())
    _lib.check(st)
    vals = out.cpu().tolist()
    for k, v in zip(slots, vals):
        if v != v:
            raise IndexError(f"item {k}: an index fell outside its range")
        out_vals[k] = float(v)
    return out_vals


def tensor_err(x, ttype, qw, perm=None, wvec=None, rows_sample=None, seed=0):
    """Weighted quant error of x under permutation ``perm`` at container ``ttype``
    (coldpress/perm/objective.py:17-39)."""
    return tensor_err_many([dict(x=x, ttype=ttype, qw=qw, perm=perm, wvec=wvec,
                                 rows_sample=rows_sample, seed=seed)])[0]


def col_sq_sums_many(xs, row_step=32768):
    """Device float64 [n] per tensor: per-column sums of squares in row chunks of
    row_step (objective.py:44-48), bit-identical to the reference's accumulator,
    all tensors in one pass."""
    lib = _lib.load()
    devs = [weights_dev(x) for x in xs]
    outs = [torch.empty(xd.shape[1], dtype=torch.float64, device=xd.device) for xd, _ in devs]
    structs = [_lib.ColTensor(xd.data_ptr(), code, xd.shape[0], xd.shape[1], o.data_ptr())
               for (xd, code), o in zip(devs, outs)]
    arr = (_lib.ColTensor * len(structs))(*structs)
    ws = _lib.workspace(lib.cp_col_sums_batch_ws_bytes(arr, len(structs), row_step),
                        devs[0][0].device)
    _lib.check(lib.cp_col_sq_sums_batch(arr, len(structs), row_step, 0, _lib.ptr(ws), ws.numel(),
                                        _lib.stream_ptr()))
    return outs


def col_sq_sums(x, row_step=32768):
    return col_sq_sums_many([x], row_step)[0]


def col_log_rms_many(xs, row_step=32768):
    """col_log_rms of every tensor, the sums in one GPU pass (numpy arrays out)."""
    accs = col_sq_sums_many(xs, row_step)
    flat = torch.cat(accs).cpu().numpy()
    out, o = [], 0
    for x, a in zip(xs, accs):
        acc = flat[o:o + a.numel()]
        o += a.numel()
        out.append(np.log(np.sqrt(acc / x.shape[0]) + 1e-12))
    return out


def col_log_rms(x, row_step=32768):
    """Per-column log-RMS profile (coldpress/perm/objective.py:42-49), a numpy float64
    array. The O(nrow x n) sums run on the GPU; the final n-element
    log(sqrt(acc / nrow) + 1e-12) is the host libm's, as in the reference, so the
    profile (a sort key) is bit-identical."""
    return col_log_rms_many([x], row_step)[0]
