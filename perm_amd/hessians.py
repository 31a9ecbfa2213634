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
import contextlib
import os
from typing import NamedTuple

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


def _prepared(X, H):
    """(X as a contiguous [rows, d] bf16 / float32 tensor, d), with H checked."""
    _on_device(X, H)
    d = X.shape[-1]
    X2 = X.reshape(-1, d)
    if X2.dtype not in (torch.bfloat16, torch.float32):
        X2 = X2.float()
    X2 = X2.contiguous()
    if H is not None and (H.shape != (d, d) or H.dtype != torch.float32 or not H.is_contiguous()):
        raise ValueError("H must be a contiguous float32 [d, d] tensor")
    return X2, d


def _accumulate_group(lib, xs, hs, N, d, dt):
    """One cp_hess_accum_batch_ws call for jobs of one (rows, d, dtype), its row-split
    workspace from torch's allocator on the current stream."""
    import ctypes
    xdt = 1 if dt == torch.bfloat16 else 0
    xa = (ctypes.c_void_p * len(xs))(*[x.data_ptr() for x in xs])
    ha = (ctypes.c_void_p * len(hs))(*[h.data_ptr() for h in hs])
    nbytes = lib.cp_hess_ws_bytes(len(xs), xdt, N, d)
    ws = _lib.workspace(nbytes, xs[0].device) if nbytes else None
    _lib.check(lib.cp_hess_accum_batch_ws(ctypes.cast(xa, ctypes.c_void_p),
                                          ctypes.cast(ha, ctypes.c_void_p), len(xs), xdt, N, d,
                                          _lib.ptr(ws), nbytes, _lib.stream_ptr()))


def xtx_accumulate(X, H=None):
    """H += X^T X on the device. X: [..., d] bf16 or float32 CUDA tensor (leading
    dims are flattened into rows, like the hook's reshape(-1, d)); H: [d, d]
    float32 CUDA tensor or None (a zero one is allocated). Returns H. The same X and
    H give the same result bit for bit (the row summation order is fixed)."""
    lib = _lib.load()
    X2, d = _prepared(X, H)
    if H is None:
        H = torch.zeros((d, d), dtype=torch.float32, device=X2.device)
    if X2.shape[0]:
        _accumulate_group(lib, [X2], [H], X2.shape[0], d, X2.dtype)
    return H


def xtx_accumulate_many(Xs, Hs):
    """Hs[z] += Xs[z]^T Xs[z] for many (X, H) pairs, batched by (rows, d, dtype) into as
    few launches as fit. X: [..., d] bf16 or float32 CUDA tensors; H: contiguous float32
    [d, d] CUDA tensors (updated in place)."""
    lib = _lib.load()
    groups = {}
    for X, H in zip(Xs, Hs):
        X2, d = _prepared(X, H)
        groups.setdefault((X2.shape[0], d, X2.dtype), []).append((X2, H))
    for (N, d, dt), jobs in groups.items():
        if N:
            _accumulate_group(lib, [x for x, _ in jobs], [h for _, h in jobs], N, d, dt)
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


class HookTarget(NamedTuple):
    """A module whose input Hessian is collected and the GGUF tensor it is keyed by."""
    module_name: str
    module: object
    gguf_name: str   # with ".weight"
    width: int       # the module's in_features, equal to the tensor's ne[0]


def _in_shard(gguf_name, layer_lo, layer_hi):
    """Blocks [layer_lo, layer_hi) own their tensors; a tensor outside the blocks (output)
    belongs to the shard that starts at block 0."""
    blk = _block_of(gguf_name)
    return layer_lo <= blk < layer_hi if blk >= 0 else layer_lo == 0


def plan_targets(model, name_map, gguf_ne0, layer_lo, layer_hi):
    """Sort the Linear / Embedding modules of ``model`` into this shard's hook targets and
    the unmapped ones, with the classification of coldpress/hessians.py:108-135: a module
    without a GGUF name, or whose tensor is not in ``gguf_ne0``, is unmapped; a tensor of
    another shard, or a token lookup (integer input, so no Hessian), is left alone.
    Returns ([HookTarget], [unmapped description]). Raises ValueError naming every module
    whose in_features disagrees with its tensor's ne[0]; nothing is hooked before that
    check, so a refused call leaves the model untouched."""
    import torch.nn as nn
    targets, unmapped, conflicts = [], [], []
    for mname, mod in model.named_modules():
        if not isinstance(mod, (nn.Linear, nn.Embedding)):
            continue
        base = name_map.get(mname)
        gguf = None if base is None else base + ".weight"
        if gguf is None:
            unmapped.append(mname)
        elif gguf not in gguf_ne0:
            unmapped.append(f"{mname} (-> {gguf}, not in the GGUF)")
        elif isinstance(mod, nn.Embedding) or not _in_shard(gguf, layer_lo, layer_hi):
            continue
        elif mod.in_features != gguf_ne0[gguf]:
            conflicts.append(f"{mname} -> {gguf} (in_features {mod.in_features}, "
                             f"ne[0] {gguf_ne0[gguf]})")
        else:
            targets.append(HookTarget(mname, mod, gguf, mod.in_features))
    if conflicts:
        raise ValueError(f"refusing to mis-key Hessians: in_features differs from the GGUF "
                         f"ne[0] for {'; '.join(conflicts)}")
    return targets, unmapped


class _InputHessians:
    """The accumulators of one collection, keyed by GGUF name. Modules that read one and
    the same input tensor within a forward pass (q/k/v, gate/up) share one accumulator,
    and the product is formed once per pass (the reference forms it per module)."""

    def __init__(self, device):
        self.by_name = {}
        self._device = device
        # input identity -> (accumulator, the input) for the current pass; holding the
        # input keeps its memory from being reused by a later input of the same pass, so
        # an address names one tensor until the pass ends
        self._inputs = {}

    def new_pass(self):
        self._inputs.clear()

    def observe(self, gguf_name, x):
        if not torch.is_floating_point(x):
            return
        ident = (x.device, x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype)
        known = self._inputs.get(ident)
        if known is None:
            acc = self.by_name.get(gguf_name)
            if acc is None:
                acc = HessianAccumulator(x.shape[-1], x.device if x.is_cuda else self._device)
            acc.add(x.detach().to(acc.H.device))  # a host activation crosses once per pass
            known = self._inputs[ident] = (acc, x)
        if self.by_name.setdefault(gguf_name, known[0]) is not known[0]:
            raise RuntimeError(f"{gguf_name}: shares its input with another module in one "
                               f"batch but not in another")

    @contextlib.contextmanager
    def hooked(self, targets):
        handles = [t.module.register_forward_hook(
            lambda _mod, inp, _out, g=t.gguf_name: self.observe(g, inp[0])) for t in targets]
        try:
            yield
        finally:
            for h in handles:
                h.remove()

    def results(self, gguf_ne0, keep_on_device):
        out = {}
        for gguf_name, acc in self.by_name.items():
            if acc.H.shape[0] != gguf_ne0[gguf_name]:
                raise ValueError(f"{gguf_name}: the collected Hessian is {acc.H.shape[0]} wide "
                                 f"but the GGUF ne[0] is {gguf_ne0[gguf_name]}")
            # host results: one array per name, as the reference returns them
            out[gguf_name] = {"H": acc.H if keep_on_device else acc.H.cpu().numpy(), "n": acc.n}
        return out


def collect_hessians(model, batches, gguf_ne0, arch, n_layers, layer_lo=0, layer_hi=None,
                     progress_every=16, log=print, name_map=None, keep_on_device=False):
    """Accumulate X^T X on the GPU for every hooked matmul of the layer shard
    [layer_lo, layer_hi) over ``batches`` (the interface of coldpress/hessians.py:85-179).

    gguf_ne0: {GGUF tensor name (with .weight): ne0} of the target artifact (plan_targets
    says which modules are hooked, unmapped or refused). ``name_map`` ({module name: GGUF
    base name}) replaces the built-in map of ``arch``. Returns ({GGUF name: {"H": float32
    [d, d], "n": rows}}, unmapped module names). H is a host array of its own per name, as
    the reference returns it; with ``keep_on_device`` it is the CUDA accumulator, and the
    names whose modules read one input (q/k/v, gate/up) share that one tensor."""
    if layer_hi is None:
        layer_hi = n_layers
    if name_map is None:
        name_map = build_name_map(model, arch, n_layers)
    targets, unmapped = plan_targets(model, name_map, gguf_ne0, layer_lo, layer_hi)
    sink = _InputHessians(torch.device("cuda", torch.cuda.current_device()))
    log(f"hessians: hooking {len(targets)} module inputs of blocks {layer_lo}..{layer_hi - 1}; "
        f"{len(unmapped)} unmapped")
    with sink.hooked(targets), torch.inference_mode():
        for k, ids in enumerate(batches, 1):
            sink.new_pass()
            model(ids if ids.dim() > 1 else ids[None])
            if progress_every and k % progress_every == 0:
                log(f"hessians: {k} batches in")
    return sink.results(gguf_ne0, keep_on_device), unmapped


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


def _member_table(path):
    """(filename, compression, size, stored size, CRC-32) of every member of a stored
    Hessian file except the tensor name, from the zip directory alone (no member data is
    read)."""
    import zipfile
    with zipfile.ZipFile(path) as zf:
        return tuple(sorted((i.filename, i.compress_type, i.file_size, i.compress_size, i.CRC)
                            for i in zf.infolist() if i.filename != "name.npy"))


def stored_keys(paths):
    """{path: content key} for a set of stored Hessian files: equal keys exactly for files
    whose members other than the tensor name have equal stored bytes (as stored_digest),
    so equal keys mean equal arrays. Files with the same stored bytes have the same member
    table (sizes and CRC-32s from the zip directory); only files whose tables coincide are
    hashed (stored_digest) to tell them apart. A set of distinct files reads no member
    data at all."""
    table = {p: _member_table(p) for p in set(paths)}
    by_table = {}
    for p, t in table.items():
        by_table.setdefault(t, []).append(p)
    keys = {}
    for t, ps in by_table.items():
        for p in ps:
            keys[p] = (t, stored_digest(p) if len(ps) > 1 else None)
    return keys


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
