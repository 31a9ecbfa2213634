"""GPTQ-style error feedback into committed k-quant containers, on the GPU.

Mirrors the encoder core of coldpress/ef.py (the reference's numpy backend):

  cholesky_inv_upper(H, damp=0.01, _max_tries=6)      coldpress/ef.py:46-84
  ef_encode(x, ttype, qw, H, n_iter=2, damp=0.01,
            act_order=True)                            coldpress/ef.py:179-218

plus the batched form the encode stage uses to run every tensor of a model in
one pass (``ef_encode_many``): tensors that share an input Hessian (q/k/v,
gate/up) share one factorization.

numpy inputs give numpy outputs; torch CUDA inputs keep everything on the device.
"""
import contextlib
import ctypes
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _lib
from .kquant import BYTES_PER_SB, QK_K


def _h_dtype(t):
    if t.dtype == torch.float64:
        return 1
    if t.dtype == torch.float32:
        return 0
    raise TypeError(f"H must be float32 or float64, got {t.dtype}")


def act_order_dev(H, enabled=True):
    """Visiting order of the columns: descending diag(H), ties by index (ef.py:187).
    H: [n, n] or [batch, n, n] float32/float64 CUDA tensor. Returns int32 [.., n]."""
    lib = _lib.load()
    batch = 1 if H.dim() == 2 else H.shape[0]
    n = H.shape[-1]
    if not enabled:
        o = torch.arange(n, dtype=torch.int32, device=H.device)
        return o if H.dim() == 2 else o.expand(batch, n).contiguous()
    order = torch.empty(H.shape[:-1], dtype=torch.int32, device=H.device)
    _lib.check(lib.cp_act_order(_lib.ptr(H), _h_dtype(H), n, batch, _lib.ptr(order),
                                _lib.stream_ptr()))
    return order


def _order_dev(order, batch, n, device, checked):
    """The visiting order as a device int32 [batch, n] tensor. A caller's order is
    checked first (every row a permutation of n; negative entries count from the end,
    as numpy's): IndexError before anything is launched. ``checked``: the order comes
    from act_order_dev, which always gives a permutation."""
    if order is None:
        return None
    if not checked:
        if int(np.prod(np.shape(order))) != batch * n:
            raise ValueError(f"order has shape {tuple(np.shape(order))}, expected {batch} x {n}")
        order = _lib.check_index(order, n, "order", permutation=True)
    if not isinstance(order, torch.Tensor):
        order = torch.from_numpy(np.ascontiguousarray(order))
    return order.to(device=device, dtype=torch.int32).reshape(batch, n).contiguous()


def factor_dev(H, order=None, damp=0.01, max_tries=6, out_dtype=torch.float32, checked=False):
    """Upper U with U^T U = inv(Hp + lambda I), Hp = H[order][:, order], on the device.

    H: [n, n] or [batch, n, n] CUDA tensor (float32/float64, contiguous). ``order``
    (numpy array or tensor) must be a permutation per matrix: IndexError otherwise,
    before any launch (``checked`` skips the check for orders from act_order_dev).
    Returns (U [.., n, n] of out_dtype, damp actually used per matrix)."""
    squeeze = H.dim() == 2
    Hb = H.unsqueeze(0) if squeeze else H
    batch, n = Hb.shape[0], Hb.shape[-1]
    order = _order_dev(order, batch, n, H.device, checked)
    lib = _lib.load()
    U = torch.empty((batch, n, n), dtype=out_dtype, device=H.device)
    ws = _lib.workspace(lib.cp_chol_ws_bytes(n, batch), H.device)
    used = (ctypes.c_double * batch)()
    st = lib.cp_chol_inv_upper(_lib.ptr(Hb), _h_dtype(Hb), n, batch, _lib.ptr(order), float(damp),
                               int(max_tries), _lib.ptr(U), 1 if out_dtype == torch.float64 else 0,
                               ctypes.cast(used, ctypes.c_void_p), _lib.ptr(ws), ws.numel(),
                               _lib.stream_ptr())
    _lib.check(st, exc_for_timeout=_lib.FactorTimeout)
    return (U[0] if squeeze else U), list(used)


def factor_dev_async(H, order=None, damp=0.01, out_dtype=torch.float32, checked=False):
    """One attempt of ``factor_dev`` at ``damp``, queued on the current stream
    without waiting on it. Returns (U, flags): flags is an int32 device tensor
    [batch] whose set entries mark matrices that met a non-positive pivot or whose
    chain step gave up a bounded wait (their U is meaningless and ``factor_dev``
    must redo them: with escalation, or raising FactorTimeout if the wait gives up
    again)."""
    squeeze = H.dim() == 2
    Hb = H.unsqueeze(0) if squeeze else H
    batch, n = Hb.shape[0], Hb.shape[-1]
    order = _order_dev(order, batch, n, H.device, checked)
    lib = _lib.load()
    U = torch.empty((batch, n, n), dtype=out_dtype, device=H.device)
    flags = torch.empty(batch, dtype=torch.int32, device=H.device)
    ws = _lib.workspace(lib.cp_chol_ws_bytes(n, batch), H.device)
    st = lib.cp_chol_inv_upper_async(_lib.ptr(Hb), _h_dtype(Hb), n, batch, _lib.ptr(order),
                                     float(damp), _lib.ptr(U),
                                     1 if out_dtype == torch.float64 else 0, _lib.ptr(flags),
                                     _lib.ptr(ws), ws.numel(), _lib.stream_ptr())
    _lib.check(st)
    return (U[0] if squeeze else U), flags


def cholesky_inv_upper(H, damp=0.01, _max_tries=6):
    """U = chol(inv(H + lambda I), upper), float64 (coldpress/ef.py:46-84).

    lambda = damp * mean(diag H) + 1e-8; escalates damp x10 on failure, up to
    _max_tries attempts, then raises np.linalg.LinAlgError."""
    Hd, host = _lib.to_device(H, torch.float64)
    U, _ = factor_dev(Hd, None, damp, _max_tries, out_dtype=torch.float64)
    return np.ascontiguousarray(_lib.to_host(U)) if host else U


def _ws_for(tensors):
    lib = _lib.load()
    arr = (_lib.EfTensor * len(tensors))(*tensors)
    return arr, lib.cp_ef_ws_bytes(arr, len(tensors))


def ef_encode_dev(items, n_iter=2, mode=_lib.CP_EF_EXACT, checked=False, out_stream=None,
                  status=None):
    """Batched EF on device tensors.

    items: list of dicts with keys ttype, x [nrow, n] f32, qw [n] f32 or None,
    U [n, n] f32 (visiting order), order [n] int32 (a permutation: IndexError
    otherwise, before any launch; ``checked`` skips that for orders from
    act_order_dev), and optional ``recon`` flag.
    out_stream: the stream the outputs are allocated on (default: the current one).
    The caller must order that stream after this call's work before using or freeing
    them, and the current stream must already be ordered after out_stream's earlier
    work (as a class stream that waited on the caller's stream is).
    status: None checks the call's status word before returning (one synchronization;
    SweepTimeout when a sweep wave gave up a bounded wait); a list receives a device
    copy of the word instead, for check_status once the caller next synchronizes.
    Returns a list of (raw uint8 [nrow, row_bytes], recon f32 or None)."""
    if not checked:
        items = [dict(it, order=_order_dev(it["order"], 1, it["x"].shape[1], it["x"].device,
                                           False).reshape(-1)) for it in items]
    lib = _lib.load()
    keep, structs, outs = [], [], []
    alloc = torch.cuda.stream(out_stream) if out_stream is not None else contextlib.nullcontext()
    for it in items:
        tt = it["ttype"]
        x = it["x"]
        nrow, n = x.shape
        with alloc:
            raw = torch.empty((nrow, (n // QK_K) * BYTES_PER_SB[tt]), dtype=torch.uint8,
                              device=x.device)
            rec = (torch.empty((nrow, n), dtype=torch.float32, device=x.device)
                   if it.get("recon", True) else None)
        qw = it.get("qw")
        keep += [x, qw, it["U"], it["order"], raw, rec]
        structs.append(_lib.EfTensor(_lib.TTYPE[tt], nrow, n, x.data_ptr(),
                                     qw.data_ptr() if qw is not None else None,
                                     it["U"].data_ptr(), it["order"].data_ptr(), raw.data_ptr(),
                                     rec.data_ptr() if rec is not None else None))
        outs.append((raw, rec))
    arr, nbytes = _ws_for(structs)
    ws = _lib.workspace(nbytes, items[0]["x"].device)
    st = lib.cp_ef_encode_batch(arr, len(structs), int(n_iter), int(mode), _lib.ptr(ws), ws.numel(),
                                _lib.stream_ptr())
    _lib.check(st)
    if status is None:
        _lib.check(lib.cp_ef_read_status(_lib.ptr(ws), _lib.stream_ptr()))
    else:
        status.append(ws[:4].view(torch.int32).clone())  # the word; ws itself is released
    return outs


def status_failed(words):
    """Whether any status word ef_encode_dev(status=...) collected has its give-up bit
    (device int32 tensors of one element; reading them synchronizes)."""
    return bool(words) and bool(int(torch.cat([w.reshape(1) for w in words]).bitwise_and(1).max()))


def check_status(words):
    """Raise SweepTimeout when a collected status word says a sweep wave gave up a bounded
    wait (that call's bytes are not valid)."""
    if status_failed(words):
        raise _lib.SweepTimeout("EF sweep: a wave gave up waiting for an earlier block of its "
                                "stripe (spin bound exhausted); the call's bytes are not valid")


MODES = {"exact": _lib.CP_EF_EXACT, "mfma": _lib.CP_EF_MFMA, "exact_valu": _lib.CP_EF_EXACT_VALU}


def ef_encode(x, ttype, qw, H, n_iter=2, damp=0.01, act_order=True, mode="exact"):
    """GPTQ error feedback into committed k-quant containers (coldpress/ef.py:179-218).

    x: [nrow, n] f32; qw: imatrix means [n] or None; H: [n, n] (X^T X).
    mode "exact" propagates errors in the reference's sequential float32 order
    (bit-identical codes); "mfma" applies the cross-block propagation as
    float32-accumulated MFMA GEMMs.
    Returns (raw bytes [nrow, row_bytes], recon [nrow, n])."""
    if ttype not in BYTES_PER_SB:
        raise ValueError(ttype)
    xd, host = _lib.to_device(x, torch.float32)
    Hd, _ = _lib.to_device(H, torch.float64 if (isinstance(H, np.ndarray) and H.dtype == np.float64)
                           or (isinstance(H, torch.Tensor) and H.dtype == torch.float64)
                           else torch.float32)
    qd = _lib.to_device(qw, torch.float32)[0].reshape(-1) if qw is not None else None
    order = act_order_dev(Hd, act_order)
    U, _ = factor_dev(Hd, order, damp, checked=True)
    (raw, rec), = ef_encode_dev([{"ttype": ttype, "x": xd, "qw": qd, "U": U, "order": order}],
                                n_iter, MODES[mode], checked=True)
    if host:
        return _lib.to_host(raw), _lib.to_host(rec)
    return raw, rec


_STREAMS = {}


def _class_stream(k):
    dev = torch.cuda.current_device()
    s = _STREAMS.get((dev, k))
    if s is None:
        s = _STREAMS[(dev, k)] = torch.cuda.Stream()  # default priority
    return s


def encode_size_classes(classes, n_iter=2, mode="exact", damp=0.01, act_order=True):
    """EF of several Hessian size classes, overlapped on the device.

    classes: list of (Hb [batch, n, n] CUDA float32/float64, build) where
    build(U, order) returns the ef_encode_dev items of that class (U [batch, n, n],
    order [batch, n]). Every class gets its own stream; from this one host thread
    the act orders and one factorization attempt of every class are queued first (in
    the given order: largest first keeps the longest chain in front), then every
    class's EF, smallest matrices first, so one class's factorization overlaps
    another's sweep. Then the factorization flags are read (the only wait), and a class
    with a failed matrix is factorized again with escalation and re-encoded.
    The caller's current stream ends up ordered after all of it.
    Returns one ef_encode_dev result list per class."""
    cur = torch.cuda.current_stream()
    streams = [_class_stream(k) for k in range(len(classes))]
    facs = []
    # with several classes the factorizations share the GPU with other classes' EF: their
    # GEMMs then take the 64 x 64 tiles that fit beside the sweep's workgroups (the same
    # results; measured 77.7 -> 73.8 ms on the 28-layer Qwen3-0.6B-shaped step)
    lib = _lib.load()
    lib.cp_chol_compact_tiles(1 if len(classes) > 1 else 0)
    try:
        for (Hb, _), s in zip(classes, streams):
            s.wait_stream(cur)
            with torch.cuda.stream(s):
                order = act_order_dev(Hb, act_order)
                U, flags = factor_dev_async(Hb, order, damp, checked=True)
            facs.append((order, U, flags))
    finally:
        lib.cp_chol_compact_tiles(0)
    # EFs are queued smallest matrices first: their factorizations end first, and the
    # host time spent queueing the others would otherwise delay them
    # the outputs are allocated on the caller's stream: every class stream waited on it
    # before its first launch, and it waits on every class stream below, so no output
    # needs record_stream (whose per-tensor events cost ~1.8 ms of host time at release
    # for the 392 outputs of the 28-layer Qwen3-0.6B-shaped set)
    outs = [None] * len(classes)
    words = [None] * len(classes)
    for k in sorted(range(len(classes)), key=lambda k: classes[k][0].shape[-1]):
        (_, build), s, (order, U, _) = classes[k], streams[k], facs[k]
        got = []
        with torch.cuda.stream(s):
            outs[k] = ef_encode_dev(build(U, order), n_iter, MODES[mode] if isinstance(mode, str)
                                    else mode, checked=True, out_stream=cur, status=got)
        words[k] = got[0]
    for s in streams:
        cur.wait_stream(s)
    # one read for every class: factorization flags, then EF status words
    seen = torch.stack([f.max() for (_, _, f) in facs] +
                       [w.reshape(()) for w in words]).cpu().tolist()
    failed, gave_up = seen[:len(classes)], seen[len(classes):]
    for k, bad in enumerate(failed):
        if not bad and int(gave_up[k]) & 1:
            check_status([words[k]])  # raises
    for k, bad in enumerate(failed):
        if bad:
            Hb, build = classes[k]
            order = facs[k][0]
            U, _ = factor_dev(Hb, order, damp, checked=True)
            outs[k] = ef_encode_dev(build(U, order), n_iter, MODES[mode] if isinstance(mode, str)
                                    else mode, checked=True)
    return outs


def ef_encode_many(tensors, n_iter=2, damp=0.01, act_order=True, mode="exact"):
    """EF-encode many tensors in one batched pass.

    tensors: list of dicts {name, ttype, x (CUDA f32), qw (CUDA f32 or None),
    H (CUDA f32/f64 [n, n])}. Tensors whose ``H`` is the same object share one
    act order and one factorization (done batched per matrix size). Each size
    class runs on its own stream (``encode_size_classes``).
    Returns {name: (raw, recon)}."""
    hs = {}
    for t in tensors:
        hs.setdefault(id(t["H"]), t["H"])
    by_n = {}
    for key, H in hs.items():
        by_n.setdefault((H.shape[-1], H.dtype), []).append(key)

    classes, members = [], []
    # largest matrices first: their factorization is the longest chain
    for _, keys in sorted(by_n.items(), key=lambda kv: -kv[0][0]):
        slot = {k: i for i, k in enumerate(keys)}
        mine = [t for t in tensors if id(t["H"]) in slot]
        Hb = torch.stack([hs[k] for k in keys]) if len(keys) > 1 else hs[keys[0]].unsqueeze(0)

        def build(U, order, mine=mine, slot=slot):
            return [{"ttype": t["ttype"], "x": t["x"], "qw": t.get("qw"),
                     "U": U[slot[id(t["H"])]], "order": order[slot[id(t["H"])]],
                     "recon": t.get("recon", True)} for t in mine]
        classes.append((Hb.contiguous(), build))
        members.append(mine)
    res = encode_size_classes(classes, n_iter, mode, damp, act_order)
    out = {}
    for mine, r in zip(members, res):
        for t, o in zip(mine, r):
            out[t["name"]] = o
    return {t["name"]: out[t["name"]] for t in tensors}


# ---------------------------------------------------------------- GGUF driver

def _weights_f32(t):
    """A GGUF tensor's data [rows, ne0] as a float32 CUDA tensor (F32 / F16 / BF16)."""
    a = np.array(t.data)  # a private host copy of the mapped file's bytes
    name = t.tensor_type.name
    if name == "F32":
        return torch.from_numpy(a).cuda()
    if name == "F16":
        return torch.from_numpy(a).cuda().to(torch.float32)
    if name == "BF16":  # uint16 bit patterns: the float32 with those high 16 bits
        b = torch.from_numpy(a.astype(np.int32)).cuda()
        return (b << 16).view(torch.float32)
    raise ValueError(f"{t.name}: source weights of type {name} are not float")


def sq_err_sum_dev(recon, x, w=None):
    """(((recon - x) ** 2) * w).sum() of coldpress/ef.py:299-300 as a float32 device
    scalar, bit-identical to numpy's (the same terms, its summation order; cp_sq_err_sum).
    recon, x: contiguous float32 [nrow, n] CUDA tensors; w: float32 [n] or None (ones)."""
    lib = _lib.load()
    nrow, n = x.shape
    out = torch.empty(1, dtype=torch.float32, device=x.device)
    nbytes = lib.cp_sq_err_ws_bytes(nrow, n)
    ws = _lib.workspace(nbytes, x.device) if nbytes else None
    _lib.check(lib.cp_sq_err_sum(_lib.ptr(recon), _lib.ptr(x), _lib.ptr(w), nrow, n, _lib.ptr(out),
                                 _lib.ptr(ws), nbytes, _lib.stream_ptr()))
    return out[0]



def _auto_layers_per_pass(f16, selected, block_of, frac=0.5):
    """Layers per EF pass: the largest count whose estimated device footprint fits in
    ``frac`` of the free device memory. Per weight ~28 B (float32 input and
    reconstruction, the EF workspace of about 18.5 B, the container bytes); per tensor
    40 n^2 B for its Hessian (float64 H, the 3 n^2 float64 factor workspace, the float32
    U), counted per tensor even where tensors share one file, so the estimate errs high."""
    free, _total = torch.cuda.mem_get_info()
    per_layer = {}
    for name, _tt in selected:
        b = block_of(name)
        if b < 0:
            continue
        shape = [int(x) for x in f16[name].shape]
        n = shape[0]  # ne0: the input dimension, the Hessian's size
        nw = int(np.prod(shape))
        per_layer[b] = per_layer.get(b, 0) + 28 * nw + 40 * n * n
    if not per_layer:
        return 1
    return max(1, int(frac * free // max(per_layer.values())))


def encode_gguf(f16_path, target_path, hessdir, out_path, imatrix_path=None, perms=None,
                spacemap=None, dims=None, acknowledge_unreviewed=False, only="all", n_iter=2,
                unsafe_storage_order=False, device="cuda", log=print, layers_per_pass=None):
    """EF-encode every quantized tensor of ``target_path`` (a stock quant artifact) from the
    float weights of ``f16_path`` and the Hessians in ``hessdir``, and write a byte-map
    clone of the target to ``out_path`` (coldpress/ef.py:223-317).

    Per tensor, as the reference: token_embd takes weighted RTN with the layer-0 attention
    input diagonal (diag(H)/n) as column weights; a tensor with a stored Hessian takes EF
    (act order unless ``unsafe_storage_order``); any other takes weighted RTN with its
    imatrix means. With ``perms`` and a ``spacemap`` (an object with the reference's
    ``input_perm(name, perms, dims, ...)``, or "qwen3" for perm_amd.perm), the imatrix
    vectors and Hessians (stored in the original order) are permuted to the already
    permuted weights. Every codec, factorization and sweep runs on the GPU; EF tensors go
    through ef_encode_many ``layers_per_pass`` blocks at a time (None: as many as fit in
    half the free device memory, by a conservative estimate of the EF workspace and the
    fp64 factor buffers per layer), and tensors whose stored Hessians are identical
    (q/k/v, gate/up) share one factorization. Writes the per-tensor
    statistics to ``out_path + ".efstats.json"`` and returns them."""
    import json
    import time
    from . import hessians as hess
    from . import kquant as gkq
    from .ggufio import GGUFReader, load_imatrix_means, reemit

    if device not in ("cuda", "gpu") and not str(device).startswith("cuda"):
        raise ValueError(f"device {device!r}: this backend runs on the GPU only")
    if spacemap == "qwen3":
        from . import perm as spacemap
    imat = load_imatrix_means(imatrix_path) if imatrix_path else {}
    f16 = {t.name: t for t in GGUFReader(f16_path).tensors}
    tr = GGUFReader(target_path)
    targets = [(t.name, t.tensor_type.name, t) for t in tr.tensors
               if t.tensor_type.name in gkq.QUANTIZE]
    unsupported = [(t.name, t.tensor_type.name) for t in tr.tensors
                   if t.tensor_type.name not in gkq.QUANTIZE
                   and t.tensor_type.name not in ("F16", "F32", "BF16")]
    if unsupported:
        raise ValueError(f"target has types we cannot encode: {unsupported}")
    ack = {"acknowledge_unreviewed": acknowledge_unreviewed} if acknowledge_unreviewed else {}

    def input_perm(name):
        if perms is None or spacemap is None:
            return None
        p = spacemap.input_perm(name, perms, dims, **ack)
        return None if p is None else np.asarray(p)

    H_cache = {}

    def read_group_hessians(names, pool):
        """Start reading the stored Hessian of every name that has one: files are shared by
        content (hessians.stored_keys: the zip directory, and a hash of the stored bytes
        only where two files' directories agree), and each distinct file is read once on
        the pool (zlib releases the GIL), while the caller goes on. Returns what
        expand_group_hessians needs."""
        paths = {nm: hess.hessian_path(hessdir, nm) for nm in names}
        paths = {nm: p for nm, p in paths.items() if p is not None}
        keys = hess.stored_keys(paths.values())
        first = {}
        for p in paths.values():
            first.setdefault(keys[p], p)
        return paths, keys, {k: pool.submit(hess.read_stored, p) for k, p in first.items()}

    def expand_group_hessians(pending):
        """{name: (device float64 H, n)}: each distinct file expanded on the GPU once, from
        this thread, as its read completes."""
        paths, keys, reads = pending
        dev = {k: hess.expand_stored(f.result(), "cuda") for k, f in reads.items()}
        return {nm: dev[keys[p]] for nm, p in paths.items()}

    selected = []
    for name, tt, t in targets:
        is_embdout = name in ("token_embd.weight", "output.weight")
        if (only == "blk" and is_embdout) or (only == "embdout" and not is_embdout):
            continue
        if name not in f16:
            raise KeyError(f"{name}: absent from {f16_path}")
        if list(f16[name].shape) != list(t.shape):
            raise ValueError(f"{name}: f16 shape {f16[name].shape} != target {t.shape}")
        selected.append((name, tt))

    def block_of(name):
        return int(name.split(".")[1]) if name.startswith("blk.") else -1

    if layers_per_pass is None:
        layers_per_pass = _auto_layers_per_pass(f16, selected, block_of)
    replace, stats = {}, {}
    t_start = time.time()
    groups = {}
    for name, tt in selected:
        groups.setdefault(max(block_of(name), 0) // max(layers_per_pass, 1), []).append((name, tt))
    done = 0
    for gkey in sorted(groups):
        t0 = time.time()
        ef_items, work = [], []
        names = [nm for nm, _ in groups[gkey]]
        if "token_embd.weight" in names:
            names.append("blk.0.attn_q.weight")  # the embedding's column weights
        # the Hessian files inflate on the pool while this thread moves the weights to the GPU
        with ThreadPoolExecutor(max_workers=16) as pool:
            pending = read_group_hessians(names, pool)
            xs = {name: _weights_f32(f16[name]) for name, _ in groups[gkey]}
            Hg = expand_group_hessians(pending)
        for name, tt in groups[gkey]:
            x = xs.pop(name)
            qw = imat.get(name)
            p = input_perm(name)
            if qw is not None and p is not None:
                qw = qw[p]  # imatrix stats in original order; x is already permuted
            qd = torch.from_numpy(np.ascontiguousarray(qw, dtype=np.float32)).cuda() \
                if qw is not None else None
            if name == "token_embd.weight":
                if "blk.0.attn_q.weight" not in Hg:
                    raise FileNotFoundError(f"no Hessian for blk.0.attn_q.weight in {hessdir}")
                H0, n0 = Hg["blk.0.attn_q.weight"]
                w_embd = (torch.diagonal(H0) / max(n0, 1)).to(torch.float32)
                if p is not None:
                    w_embd = w_embd[torch.from_numpy(p).cuda()]
                w_embd = w_embd.contiguous()
                raw = gkq.quantize_dev(tt, x, w_embd)
                work.append((name, tt, x, qd, raw, gkq.dequantize_dev(tt, raw, x.shape[1]),
                             "wRTN(attn0-diag)"))
            elif name in Hg:
                H, _n = Hg[name]
                if p is not None:
                    from .perm import permute_hessian
                    key = ("perm", id(H), p.tobytes())
                    if key not in H_cache:
                        H_cache[key] = (permute_hessian(H, p), _n)
                    H = H_cache[key][0]
                ef_items.append({"name": name, "ttype": tt, "x": x, "qw": qd, "H": H})
                work.append((name, tt, x, qd, None, None,
                             "EF" if not unsafe_storage_order else "EF(storage-order)"))
            else:
                raw = gkq.quantize_dev(tt, x, qd)
                work.append((name, tt, x, qd, raw, gkq.dequantize_dev(tt, raw, x.shape[1]), "wRTN"))
        res = ef_encode_many(ef_items, n_iter=n_iter, act_order=not unsafe_storage_order) \
            if ef_items else {}
        sec = (time.time() - t0) / max(len(work), 1)
        # the statistics stay on the device until one read-back for the whole group,
        # and the container bytes come back in one copy
        errs, raws = [], []
        for name, tt, x, qd, raw, recon, mode in work:
            if raw is None:
                raw, recon = res[name]
            base = gkq.dequantize_dev(tt, gkq.quantize_dev(tt, x, qd), x.shape[1])
            # w: qw, or the reference's ones (a product by 1.0 changes no term)
            errs.append(torch.stack([sq_err_sum_dev(base, x, qd), sq_err_sum_dev(recon, x, qd)]))
            raws.append(raw.reshape(-1))
        err_host = torch.stack(errs).cpu().tolist() if errs else []
        raw_host = torch.cat(raws).cpu().numpy() if raws else None
        off = 0
        for (name, tt, _x, _qd, _raw, _rec, mode), (e_base, e_ours), r in zip(work, err_host, raws):
            stats[name] = {"type": tt, "mode": mode,
                           "rel_err_vs_stock": e_ours / e_base - 1 if e_base else 0.0,
                           "sec": sec}
            replace[name] = raw_host[off:off + r.numel()]
            off += r.numel()
            done += 1
            if done % 20 == 0 or name in ("token_embd.weight", "output.weight"):
                log(f"[{done}/{len(selected)}] {name} {tt} {mode} "
                    f"err-vs-stock {stats[name]['rel_err_vs_stock'] * 100:+.1f}%")
        H_cache.clear()  # a layer group's Hessians are not read by later groups
        del Hg
    reemit(target_path, out_path, replace=replace, log=log)
    if stats:
        med = float(np.median([s["rel_err_vs_stock"] for s in stats.values()]))
        log(f"median err-vs-stock: {med * 100:+.2f}%; total {(time.time() - t_start) / 60:.1f} min")
    with open(out_path + ".efstats.json", "w") as f:
        json.dump(stats, f, indent=1)
    return stats
