"""Input-Hessian accumulation on the GPU (coldpress/hessians.py).

The reference's forward hook computes ``x.float().T @ x`` per batch on the
activation's device, copies the [d, d] result to the host and adds it into a
CPU float32 accumulator (coldpress/hessians.py:137-154). Here the accumulator
stays on the device and each batch is added by one MFMA kernel launch
(cp_hess_accum), bf16 activations going straight into bf16 MFMA with float32
accumulation -- no upcast copy, no device-to-host copy per batch.

Module -> GGUF tensor naming (the reference uses gguf's TensorNameMap, a package
not present here) is supplied by the caller as ``name_map``.
"""
import torch

from . import _lib


def xtx_accumulate(X, H=None):
    """H += X^T X on the device. X: [..., d] bf16 or float32 CUDA tensor (leading
    dims are flattened into rows, like the hook's reshape(-1, d)); H: [d, d]
    float32 CUDA tensor or None (a zero one is allocated). Returns H."""
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


def collect_hessians(model, batches, name_map, gguf_ne0=None, progress_every=16, log=print):
    """Accumulate X^T X for every nn.Linear named in ``name_map`` ({module name:
    GGUF tensor name}) over ``batches`` (coldpress/hessians.py:85-179).

    A module whose in_features differs from gguf_ne0[gguf name] is refused before
    any hook is registered (hessians.py:126-135). Returns
    ({gguf name: {"H": float32 [d, d] CUDA tensor, "n": rows}}, unmapped)."""
    import torch.nn as nn
    plan, unmapped, mismatched = [], [], []
    for mname, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        g = name_map.get(mname)
        if g is None:
            unmapped.append(mname)
            continue
        if gguf_ne0 is not None and g in gguf_ne0 and mod.in_features != gguf_ne0[g]:
            mismatched.append((mname, g, mod.in_features, gguf_ne0[g]))
            continue
        plan.append((mod, g))
    if mismatched:
        for mname, g, inf, ne0 in mismatched:
            log(f"  SHAPE MISMATCH {mname} -> {g}: in_features={inf} ne0={ne0}")
        raise ValueError(f"{len(mismatched)} module(s) map to a GGUF tensor with a different "
                         f"ne[0]; refusing to mis-key a Hessian")
    acc = {}

    def make_hook(g):
        def fn(mod, inp, out):
            x = inp[0]
            if not torch.is_floating_point(x):
                return
            if g not in acc:
                acc[g] = HessianAccumulator(x.shape[-1], x.device)
            acc[g].add(x.detach())
        return fn

    handles = [mod.register_forward_hook(make_hook(g)) for mod, g in plan]
    try:
        with torch.inference_mode():
            for c, ids in enumerate(batches):
                model(ids)
                if progress_every and (c + 1) % progress_every == 0:
                    log(f"  chunk {c + 1}")
    finally:
        for h in handles:
            h.remove()
    return {g: {"H": a.H, "n": a.n} for g, a in acc.items()}, unmapped
