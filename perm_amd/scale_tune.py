"""The linear form of a k-quant tensor on the GPU, with the API of coldpress/scale_tune.py.

With the integer codes fixed, dequantization is linear in the per-superblock fp16 scales:

    W[r, c] = d[r, c // 256] * A[r, c] - dmin[r, c // 256] * B[r, c]

(A = integer sub-block scale x signed code, B = integer sub-block min; no min side for
Q3_K and Q6_K). The form in float32 equals the container's decode bit for bit.

  extract_linear(raw, ttype, n_per_row)            scale_tune.py:67-159
  reconstruct_np(lin)                              scale_tune.py:162-173
  write_back(raw, ttype, d_new, dmin_new=None)     scale_tune.py:176-203
  build_torch_params(gguf_path)                    scale_tune.py:206-242
  reconstruct(entry, dtype=None)                   scale_tune.py:245-269

Every array of nrow x n entries is produced on the GPU (cp_lin_*); ``reconstruct`` is a
torch autograd function whose forward and backward are the library's kernels, so the
distill stage's scale parameters train on the device.
"""
import numpy as np
import torch

from . import _lib

SUPPORTED = ("Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K")
_HAS_MIN = {"Q2_K": True, "Q3_K": False, "Q4_K": True, "Q5_K": True, "Q6_K": False}


def _raw_dev(raw):
    if isinstance(raw, torch.Tensor):
        return raw.to(device="cuda", dtype=torch.uint8).contiguous(), False
    return torch.from_numpy(np.ascontiguousarray(raw, dtype=np.uint8)).cuda(), True


def extract_linear_dev(raw, ttype, n_per_row, ab_dtype=torch.int16):
    """Device form of extract_linear: d, dmin float32 [nrow, n_sb]; A, B [nrow, n] of
    ``ab_dtype`` (int16 or float32). dmin and B are None for Q3_K / Q6_K."""
    if ttype not in SUPPORTED:
        raise ValueError(f"unsupported ttype {ttype!r}; supported: {SUPPORTED}")
    lib = _lib.load()
    rd, _ = _raw_dev(raw)
    nrow = rd.shape[0]
    n_sb = n_per_row // 256
    dev = rd.device
    d = torch.empty((nrow, n_sb), dtype=torch.float32, device=dev)
    A = torch.empty((nrow, n_per_row), dtype=ab_dtype, device=dev)
    dmin = B = None
    if _HAS_MIN[ttype]:
        dmin = torch.empty((nrow, n_sb), dtype=torch.float32, device=dev)
        B = torch.empty((nrow, n_per_row), dtype=ab_dtype, device=dev)
    _lib.check(lib.cp_lin_extract(_lib.TTYPE[ttype], _lib.ptr(rd), nrow, n_per_row, _lib.ptr(d),
                                  _lib.ptr(dmin), _lib.ptr(A), _lib.ptr(B),
                                  1 if ab_dtype == torch.float32 else 0, _lib.stream_ptr()))
    return {"d": d, "dmin": dmin, "A": A, "B": B, "ttype": ttype, "shape": (nrow, n_per_row)}


def extract_linear(raw_bytes_2d, ttype, n_per_row):
    """{d, dmin, A, B, ttype, shape} with float32 arrays, as the reference returns them
    (numpy for numpy input, CUDA tensors for a tensor input)."""
    host = not isinstance(raw_bytes_2d, torch.Tensor)
    lin = extract_linear_dev(raw_bytes_2d, ttype, n_per_row, ab_dtype=torch.float32)
    if host:
        for k in ("d", "dmin", "A", "B"):
            if lin[k] is not None:
                lin[k] = lin[k].cpu().numpy()
    return lin


def _as_dev(v, dtype):
    if v is None:
        return None
    if isinstance(v, torch.Tensor):
        return v.to(device="cuda", dtype=dtype).contiguous()
    return torch.from_numpy(np.ascontiguousarray(v)).to(device="cuda", dtype=dtype)


def _reconstruct_dev(d, dmin, A16, B16, shape):
    lib = _lib.load()
    nrow, n = shape
    W = torch.empty((nrow, n), dtype=torch.float32, device=d.device)
    _lib.check(lib.cp_lin_reconstruct(nrow, n, _lib.ptr(d), _lib.ptr(dmin), _lib.ptr(A16),
                                      _lib.ptr(B16), _lib.ptr(W), _lib.stream_ptr()))
    return W


def reconstruct_np(lin):
    """float32 reconstruction from an extract_linear dict (equals DEQUANTIZE exactly)."""
    shape = lin["shape"]
    host = isinstance(lin["d"], np.ndarray)
    d = _as_dev(lin["d"], torch.float32)
    A = _as_dev(lin["A"], torch.int16)   # integer products: exact in int16
    dmin = _as_dev(lin["dmin"], torch.float32)
    B = _as_dev(lin["B"], torch.int16)
    W = _reconstruct_dev(d, dmin, A, B, shape)
    return W.cpu().numpy() if host else W


def write_back(raw_bytes_2d, ttype, d_new_f32, dmin_new_f32=None):
    """Container bytes with only the fp16 d / dmin fields replaced (float32 -> float16,
    round to nearest even); every other byte unchanged."""
    if ttype not in SUPPORTED:
        raise ValueError(f"unsupported ttype {ttype!r}")
    if _HAS_MIN[ttype] and dmin_new_f32 is None:
        raise ValueError(f"{ttype} has a dmin field; dmin_new_f32 required")
    lib = _lib.load()
    rd, host = _raw_dev(raw_bytes_2d)
    nrow = rd.shape[0]
    bp = {"Q2_K": 84, "Q3_K": 110, "Q4_K": 144, "Q5_K": 176, "Q6_K": 210}[ttype]
    row_bytes = rd.shape[1] if rd.dim() == 2 else rd.reshape(nrow, -1).shape[1]
    n = row_bytes // bp * 256
    d = _as_dev(d_new_f32, torch.float32)
    dmin = _as_dev(dmin_new_f32, torch.float32) if _HAS_MIN[ttype] else None
    if d.numel() != nrow * (n // 256) or (dmin is not None and dmin.numel() != d.numel()):
        raise ValueError("one d (and dmin) per superblock")
    out = torch.empty_like(rd)
    _lib.check(lib.cp_lin_write_back(_lib.TTYPE[ttype], _lib.ptr(rd), nrow, n, _lib.ptr(d),
                                     _lib.ptr(dmin), _lib.ptr(out), _lib.stream_ptr()))
    out = out.reshape(nrow, row_bytes)
    return out.cpu().numpy() if host else out


class _Reconstruct(torch.autograd.Function):
    """W = d (x) A - dmin (x) B; gradients to d and dmin by the library's kernels."""

    @staticmethod
    def forward(ctx, d, dmin, A16, B16, shape):
        dd = d.detach().to(device=A16.device, dtype=torch.float32).contiguous()
        dm = dmin.detach().to(device=A16.device, dtype=torch.float32).contiguous() \
            if dmin is not None else None
        ctx.save_for_backward(A16, B16 if B16 is not None else torch.empty(0))
        ctx.shape, ctx.has_min = shape, dmin is not None
        ctx.devices = (d.device, dmin.device if dmin is not None else None)
        return _reconstruct_dev(dd, dm, A16, B16, shape)

    @staticmethod
    def backward(ctx, gW):
        lib = _lib.load()
        A16, B16 = ctx.saved_tensors
        nrow, n = ctx.shape
        gW = gW.contiguous().to(torch.float32)
        gd = torch.empty((nrow, n // 256), dtype=torch.float32, device=gW.device)
        gdmin = torch.empty_like(gd) if ctx.has_min else None
        _lib.check(lib.cp_lin_reconstruct_grad(nrow, n, _lib.ptr(gW), _lib.ptr(A16),
                                               _lib.ptr(B16) if ctx.has_min else None,
                                               _lib.ptr(gd), _lib.ptr(gdmin), _lib.stream_ptr()))
        # parameters kept on the host get their gradients there
        return gd.to(ctx.devices[0]), (gdmin.to(ctx.devices[1]) if gdmin is not None else None), \
            None, None, None


def reconstruct(entry, dtype=None):
    """float32 weight [nrow, n] = d (x) A - dmin (x) B (differentiable in d and dmin),
    cast to ``dtype`` last when given (scale_tune.py:245-269). The result lives on the
    GPU; d and dmin may live on the host or the GPU and get their gradients where they
    live."""
    d, dmin = entry["d"], entry["dmin"]
    A16 = _as_dev(entry["A"], torch.int16)
    B16 = _as_dev(entry["B"], torch.int16) if dmin is not None else None
    W = _Reconstruct.apply(d, dmin, A16, B16, tuple(entry["shape"]))
    if dtype is not None and dtype != torch.float32:
        W = W.to(dtype)
    return W


def build_torch_params(gguf_path):
    """{name: {d, dmin (nn.Parameter float32 on the GPU or None), A, B (int16 CUDA
    constants), ttype, shape}} for every Q2_K..Q6_K tensor of a GGUF file."""
    from .ggufio import GGUFReader
    out = {}
    for t in GGUFReader(gguf_path).tensors:
        tt = t.tensor_type.name
        if tt not in SUPPORTED:
            continue
        n_per_row = int(t.shape[0])
        nrow = int(t.n_elements) // n_per_row
        raw = np.array(t.data).reshape(nrow, -1)
        lin = extract_linear_dev(raw, tt, n_per_row)
        out[t.name] = {"d": torch.nn.Parameter(lin["d"]),
                       "dmin": torch.nn.Parameter(lin["dmin"]) if lin["dmin"] is not None else None,
                       "A": lin["A"], "B": lin["B"], "ttype": tt, "shape": lin["shape"]}
    return out
