"""Input-Hessian accumulation on the GPU (coldpress/hessians.py).

The reference's forward hook computes ``x.float().T @ x`` per batch on the
activation's device, copies the [d, d] result to the host and adds it into a
CPU float32 accumulator (coldpress/hessians.py:137-154). Here the accumulator
stays on the device and each batch is added by one MFMA kernel launch
(cp_hess_accum), bf16 activations going straight into bf16 MFMA with float32
accumulation -- no upcast copy, no device-to-host copy per batch.

Module -> GGUF tensor naming: the reference asks gguf's TensorNameMap (pip ``gguf``,
absent here); ``build_name_map`` carries the map for the HF decoder layout of the dense
llama-family architectures (llama, mistral, qwen2, qwen3), and ``collect_hessians`` also
takes a caller's map.

Storage (coldpress/hessians.py:163-243): ``save_hessians`` writes the reference's npz
format (float16 H over a per-matrix ``hscale``, exact float32 ``diag32``, ``n``, ``name``),
with the packing arithmetic on the GPU (cp_h2_pack); ``load_hessian`` reads the same files
(and the older float32-only ones) and rebuilds the float64 matrix on the GPU (cp_h2_expand).
"""
import os

import numpy as np
import torch

from . import _lib

FP16_SAFE_MAX = 32768.0

# old family-keyed file layout (hessians.py:39-44, 209-222)
_FAMILY_FALLBACK = {"attn_q": "qkv_in", "attn_k": "qkv_in", "attn_v": "qkv_in",
                    "attn_output": "o_in", "ffn_gate": "gateup_in", "ffn_up": "gateup_in",
                    "ffn_down": "down_in"}


def _on_device(X, H):
    """Both operands must live on one CUDA device: their addresses go to a kernel."""
    if not X.is_cuda or (H is not None and (not H.is_cuda or H.device != X.device)):
        raise ValueError(f"X ({X.device}) and H ({None if H is None else H.device}) must be "
                         f"tensors on one CUDA device")


def xtx_accumulate(X, H=None):
    """H += X^T X on the device. X: [..., d] bf16 or float32 CUDA tensor (leading
    dims are flattened into rows, like the hook's reshape(-1, d)); H: [d, d]
    float32 CUDA tensor or None (a zero one is allocated). Returns H."""
    _on_device(X, H)
    lib = _lib.load()
    d = X.shape[-1]
    X2 = X.reshape(-1, d)
    if X2.dtype not in (torch.bfloat16, torch.float32):
        X2 = X2.float()
    X2 = X2.contiguous()
    if H is None:
        H = torch.zeros((d, d), dtype=torch.float32, device=X2.device)
    if H.shape != (d, d) or H.dtype != torch.float32 or not H.is_contiguous():
        raise ValueError("H must be a contiguous float32 [d, d] tensor")
    st = lib.cp_hess_accum(_lib.ptr(X2), 1 if X2.dtype == torch.bfloat16 else 0, X2.shape[0], d,
                           _lib.ptr(H), _lib.stream_ptr())
    _lib.check(st)
    return H


def xtx_accumulate_many(Xs, Hs):
    """Hs[z] += Xs[z]^T Xs[z] for many (X, H) pairs, batched by (rows, d, dtype) into as
    few launches as fit. X: [..., d] bf16 or float32 CUDA tensors; H: contiguous float32
    [d, d] CUDA tensors (updated in place)."""
    import ctypes
    lib = _lib.load()
    groups = {}
    for X, H in zip(Xs, Hs):
        _on_device(X, H)
        d = X.shape[-1]
        X2 = X.reshape(-1, d)
        if X2.dtype not in (torch.bfloat16, torch.float32):
            X2 = X2.float()
        X2 = X2.contiguous()
        if H.shape != (d, d) or H.dtype != torch.float32 or not H.is_contiguous():
            raise ValueError("H must be a contiguous float32 [d, d] tensor")
        groups.setdefault((X2.shape[0], d, X2.dtype), []).append((X2, H))
    for (N, d, dt), jobs in groups.items():
        xs = (ctypes.c_void_p * len(jobs))(*[x.data_ptr() for x, _ in jobs])
        hs = (ctypes.c_void_p * len(jobs))(*[h.data_ptr() for _, h in jobs])
        st = lib.cp_hess_accum_batch(ctypes.cast(xs, ctypes.c_void_p), ctypes.cast(hs, ctypes.c_void_p),
                                     len(jobs), 1 if dt == torch.bfloat16 else 0, N, d,
                                     _lib.stream_ptr())
        _lib.check(st)
    return Hs


class HessianAccumulator:
    """Device-resident float32 X^T X accumulator with a row count (the hook state
    of coldpress/hessians.py:148-153)."""

    def __init__(self, d, device="cuda"):
        self.H = torch.zeros((d, d), dtype=torch.float32, device=device)
        self.n = 0

    def add(self, X):
        xtx_accumulate(X, self.H)
        self.n += X.reshape(-1, X.shape[-1]).shape[0]
        return self


# HF module names of the dense llama-family decoders (llama, mistral, qwen2, qwen3) and
# the GGUF tensor each maps to -- the entries gguf's TensorNameMap gives these modules.
NAME_MAP_ARCHES = ("llama", "mistral", "qwen2", "qwen3")
_PREFIXES = ("model.", "model.language_model.", "language_model.model.")
_LAYER_KINDS = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k",
                "self_attn.v_proj": "attn_v", "self_attn.o_proj": "attn_output",
                "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up", "mlp.down_proj": "ffn_down"}


def _gguf_base(module_name, n_layers):
    """GGUF base name (no ".weight") of an HF module name, or None."""
    if module_name in ("lm_head", "language_model.lm_head"):
        return "output"
    for pre in _PREFIXES:
        if not module_name.startswith(pre):
            continue
        rest = module_name[len(pre):]
        if rest == "embed_tokens":
            return "token_embd"
        head, _, tail = rest.partition(".")
        layer, _, kind = tail.partition(".")
        if head == "layers" and layer.isdigit() and int(layer) < n_layers and kind in _LAYER_KINDS:
            return f"blk.{int(layer)}.{_LAYER_KINDS[kind]}"
    return None


def build_name_map(model, arch, n_layers):
    """{module name: GGUF base name (no ".weight")} for every nn.Linear / nn.Embedding
    of ``model`` that maps (coldpress/hessians.py:64-82). Raises ValueError for an
    architecture without a built-in map."""
    import torch.nn as nn
    if arch not in NAME_MAP_ARCHES:
        raise ValueError(f"arch {arch!r} has no built-in module -> GGUF name map "
                         f"(have {', '.join(NAME_MAP_ARCHES)}); pass name_map")
    out = {}
    for name, mod in model.named_modules():
        if isinstance(mod, (nn.Linear, nn.Embedding)):
            base = _gguf_base(name, n_layers)
            if base is not None:
                out[name] = base
    return out


def _block_of(gguf_name):
    """Decoder block of a GGUF tensor name, -1 for the non-block tensors."""
    parts = gguf_name.split(".")
    return int(parts[1]) if parts[0] == "blk" and len(parts) > 1 and parts[1].isdigit() else -1


def collect_hessians(model, batches, gguf_ne0, arch, n_layers, layer_lo=0, layer_hi=None,
                     progress_every=16, log=print, name_map=None, keep_on_device=False):
    """Accumulate X^T X on the GPU for every hooked matmul of the layer shard
    [layer_lo, layer_hi) over ``batches`` (coldpress/hessians.py:85-179).

    gguf_ne0: {GGUF tensor name (with .weight): ne0} of the target artifact; a module whose
    GGUF name is absent is unmapped, one whose in_features differs is refused with
    ValueError before any hook is registered. Non-block tensors (output) belong to the
    shard that starts at layer 0. ``name_map`` ({module name: GGUF base name}) replaces the
    built-in map of ``arch``. Modules that read one input tensor (q/k/v, gate/up) share one
    accumulator, formed once per batch. Returns ({GGUF name: {"H": float32 [d, d], "n":
    rows}}, unmapped module names); H is a host array, as the reference returns it, or
    with ``keep_on_device`` the CUDA tensor (tensors sharing an input share one object)."""
    import torch.nn as nn
    if layer_hi is None:
        layer_hi = n_layers
    if name_map is None:
        name_map = build_name_map(model, arch, n_layers)
    plan, unmapped, mismatched = [], [], []
    for mname, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue  # an embedding lookup has no input Hessian
        base = name_map.get(mname)
        if base is None:
            unmapped.append(mname)
            continue
        g = base + ".weight"
        if g not in gguf_ne0:
            unmapped.append(f"{mname} (-> {g}, absent from the GGUF)")
            continue
        blk = _block_of(g)
        if not (layer_lo <= blk < layer_hi if blk >= 0 else layer_lo == 0):
            continue
        if mod.in_features != gguf_ne0[g]:
            mismatched.append((mname, g, mod.in_features, gguf_ne0[g]))
            continue
        plan.append((mod, g))
    if mismatched:
        for mname, g, inf, ne0 in mismatched:
            log(f"  SHAPE MISMATCH {mname} -> {g}: in_features={inf} ne0={ne0}")
        raise ValueError(f"{len(mismatched)} module(s) map to a GGUF tensor with a different "
                         f"ne[0]; refusing to mis-key a Hessian")
    acc = {}
    # input identity of the current forward pass -> (its accumulator, the input). Holding
    # the input keeps its memory from being reused by a later input of the same pass, so
    # the address identifies one tensor until the pass ends.
    seen = {}
    dev = torch.device("cuda", torch.cuda.current_device())

    def make_hook(g):
        def fn(mod, inp, out):
            x = inp[0]
            if not torch.is_floating_point(x):
                return
            # q/k/v (and gate/up) read one and the same input tensor: accumulate it once and
            # share the accumulator (the reference forms the identical X^T X per module)
            key = (x.device, x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype)
            hit = seen.get(key)
            if hit is None:
                a = acc.get(g)
                if a is None:
                    a = HessianAccumulator(x.shape[-1], x.device if x.is_cuda else dev)
                a.add(x.detach().to(a.H.device))  # a host activation crosses once per batch
                seen[key] = (a, x)
            else:
                a = hit[0]
            if g in acc and acc[g] is not a:
                raise RuntimeError(f"{g}: shares its input with another module in one batch "
                                   f"but not in another")
            acc[g] = a
        return fn

    handles = [mod.register_forward_hook(make_hook(g)) for mod, g in plan]
    log(f"hooked {len(handles)} matmuls in layers [{layer_lo},{layer_hi}); "
        f"{len(unmapped)} module(s) unmapped/skipped")
    try:
        with torch.inference_mode():
            for c, ids in enumerate(batches):
                seen.clear()
                model(ids.unsqueeze(0) if ids.dim() == 1 else ids)
                if progress_every and (c + 1) % progress_every == 0:
                    log(f"  chunk {c + 1}")
    finally:
        for h in handles:
            h.remove()
    host = {}
    out = {}
    for g, a in acc.items():
        if a.H.shape[0] != gguf_ne0[g]:
            raise ValueError(f"{g}: collected H.shape[0]={a.H.shape[0]} != ne0={gguf_ne0[g]}")
        if not keep_on_device and id(a) not in host:
            host[id(a)] = a.H.cpu().numpy()
        out[g] = {"H": a.H if keep_on_device else host[id(a)], "n": a.n}
    return out, unmapped


# ---------------------------------------------------------------- storage

def _path(outdir, gguf_name):
    return os.path.join(outdir, gguf_name.replace(".", "_") + ".npz")


def pack_hessian(H):
    """(H16 float16 [d, d], diag32 float32 [d], hscale float32) of a float32 Hessian, the
    stored form of save_hessians, computed on the GPU. H: numpy or torch [d, d]."""
    lib = _lib.load()
    Hd = H if isinstance(H, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(H))
    Hd = Hd.to(device="cuda", dtype=torch.float32).contiguous()
    d = Hd.shape[0]
    if Hd.shape != (d, d):
        raise ValueError("H must be square")
    H16 = torch.empty((d, d), dtype=torch.float16, device=Hd.device)
    diag = torch.empty(d, dtype=torch.float32, device=Hd.device)
    hs = torch.empty(1, dtype=torch.float32, device=Hd.device)
    ws = _lib.workspace(256, Hd.device)
    _lib.check(lib.cp_h2_pack(_lib.ptr(Hd), d, _lib.ptr(H16), _lib.ptr(diag), _lib.ptr(hs),
                              _lib.ptr(ws), ws.numel(), _lib.stream_ptr()))
    return H16, diag, hs


def save_hessians(hessians, outdir):
    """Write each {gguf_name: {"H": [d, d], "n": rows}} as the reference's npz
    (hessians.py:166-194): H float16 over hscale, diag32, hscale, n, name."""
    os.makedirs(outdir, exist_ok=True)
    for gname, h in hessians.items():
        H16, diag, hs = pack_hessian(h["H"])
        np.savez_compressed(_path(outdir, gname), H=H16.cpu().numpy(), diag32=diag.cpu().numpy(),
                            hscale=np.float32(hs.item()), n=h["n"], name=gname)


def _fallback_key(gguf_name):
    """Old family key: blk.3.attn_q.weight -> blk.3.qkv_in, output.weight -> lmhead_in."""
    if gguf_name == "output.weight":
        return "lmhead_in"
    if not gguf_name.startswith("blk."):
        return None
    parts = gguf_name.split(".")
    if len(parts) < 3:
        return None
    fam = _FAMILY_FALLBACK.get(parts[2])
    return f"blk.{parts[1]}.{fam}" if fam else None


def hessian_path(hessdir, gguf_name):
    """The file load_hessian reads for this tensor (per-tensor first, then the family
    file), or None."""
    cand = [_path(hessdir, gguf_name)]
    fk = _fallback_key(gguf_name)
    if fk is not None:
        cand.append(_path(hessdir, fk))
    for p in cand:
        if os.path.exists(p):
            return p
    return None


def has_hessian(hessdir, gguf_name):
    return hessian_path(hessdir, gguf_name) is not None


def read_stored(path):
    """Host arrays of one stored Hessian file: (H16 or older float32 H, hscale, diag32 or
    None, n). Plain arrays only: no pickled object is read."""
    with np.load(path) as z:
        Hs = np.ascontiguousarray(z["H"])
        hscale = float(z["hscale"]) if "hscale" in z.files else 1.0
        diag = np.ascontiguousarray(z["diag32"], dtype=np.float32) if "diag32" in z.files else None
        n = int(z["n"])
    if Hs.dtype not in (np.float16, np.float32):
        Hs = Hs.astype(np.float32)
    return Hs, hscale, diag, n


def expand_stored(stored, device=None):
    """(float64 H on the device, n) from read_stored's arrays: float16 H times hscale with
    the float32 diagonal written back, or an older float32 H widened (cp_h2_expand)."""
    Hs, hscale, diag, n = stored
    lib = _lib.load()
    dev = torch.device(device) if device is not None else torch.device("cuda")
    Hd = torch.from_numpy(Hs).to(dev)
    dd = torch.from_numpy(diag).to(dev) if diag is not None else None
    d = Hs.shape[0]
    out = torch.empty((d, d), dtype=torch.float64, device=dev)
    _lib.check(lib.cp_h2_expand(_lib.ptr(Hd), 1 if Hs.dtype == np.float16 else 0, d, hscale,
                                _lib.ptr(dd), _lib.ptr(out), _lib.stream_ptr()))
    return out, n


def stored_digest(path):
    """Content key of a stored Hessian file, computed without decompressing it: SHA-1 over
    the stored bytes (and compression method) of every member except the tensor name.
    Equal keys mean equal stored bytes, hence equal arrays; equal arrays written by
    different compressors may hash apart, which only forgoes sharing them."""
    import hashlib
    import struct
    import zipfile
    h = hashlib.sha1()
    with zipfile.ZipFile(path) as zf, open(path, "rb") as f:
        for info in sorted(zf.infolist(), key=lambda i: i.filename):
            if info.filename == "name.npy":
                continue
            f.seek(info.header_offset)
            hdr = f.read(30)  # local file header; name and extra-field lengths at 26 and 28
            if len(hdr) != 30 or hdr[:4] != b"PK\x03\x04":
                raise ValueError(f"{path}: damaged member header for {info.filename}")
            nlen, elen = struct.unpack("<HH", hdr[26:30])
            f.seek(info.header_offset + 30 + nlen + elen)
            h.update(info.filename.encode())
            h.update(struct.pack("<IQ", info.compress_type, info.file_size))
            h.update(f.read(info.compress_size))
    return h.hexdigest()


def load_hessian(hessdir, gguf_name, device=None):
    """(H float64 [d, d], n) for a GGUF tensor name (hessians.py:225-243): float16 H times
    hscale with the float32 diagonal written back, or an older float32 H widened. The
    matrix is rebuilt on the GPU; it is returned there when ``device`` is given, as numpy
    otherwise. Raises FileNotFoundError when neither file exists."""
    path = hessian_path(hessdir, gguf_name)
    if path is None:
        raise FileNotFoundError(f"no Hessian for {gguf_name} in {hessdir}")
    out, n = expand_stored(read_stored(path), device)
    return (out if device is not None else out.cpu().numpy()), n
