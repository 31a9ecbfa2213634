"""PERM channel permutations on the GPU, Qwen3 dense space map (the index moves of
coldpress/perm/spacemaps/qwen3.py).

Three permutation spaces (qwen3.py module docstring):
  res [d_model]            embedding cols, q/k/v/gate/up input cols, o/down output rows
  ffn [d_ffn] per layer    gate/up output rows, down input cols
  vo  [head_dim] per (layer, kv-head)   v output rows of the kv head, o input cols of
                           its GQA q heads
Every move is a pure index gather (bit-exact); Hessians and importance vectors of
an input space move with the same index (ef.py:274-276, 289-290).

perms: {"res": int [d_model], "ffn": [int [d_ffn]] * n_layers,
        "vo": [[int [head_dim]] * n_kv] * n_layers}  (the reference's container).
dims:  {"d_model", "d_ffn", "n_layers", "n_heads", "n_kv", "head_dim"}.
"""
import numpy as np
import torch

from . import _lib

RES_INPUT_KINDS = ("attn_q", "attn_k", "attn_v", "ffn_gate", "ffn_up")


def identity_perms(dims):
    return {"res": np.arange(dims["d_model"]),
            "ffn": [np.arange(dims["d_ffn"]) for _ in range(dims["n_layers"])],
            "vo": [[np.arange(dims["head_dim"]) for _ in range(dims["n_kv"])]
                   for _ in range(dims["n_layers"])]}


def _check(p, n, what="permutation"):
    """p as an int32 permutation of n, checked before any launch: a wrong length raises
    ValueError, an entry out of range or a repeated one IndexError (numpy's fancy
    indexing raises IndexError for the first; the second is not a permutation)."""
    if np.shape(p) != (n,):
        raise ValueError(f"{what} has shape {np.shape(p)}, expected ({n},)")
    return _lib.check_index(p, n, what, permutation=True)


def v_output_index(perms, layer, dims):
    """Row index of attn_v's output (n_kv * head_dim): kv head h uses vo[layer][h]
    (qwen3.py:163-167)."""
    hd, nkv = dims["head_dim"], dims["n_kv"]
    idx = np.arange(nkv * hd)
    for h in range(nkv):
        idx[h * hd:(h + 1) * hd] = h * hd + _check(perms["vo"][layer][h], hd)
    return idx


def o_input_index(perms, layer, dims):
    """Column index of attn_output's input (n_heads * head_dim): q head q uses
    vo[layer][q // group] (qwen3.py:94-103)."""
    hd, nh = dims["head_dim"], dims["n_heads"]
    group = nh // dims["n_kv"]
    idx = np.arange(nh * hd)
    for q in range(nh):
        idx[q * hd:(q + 1) * hd] = q * hd + _check(perms["vo"][layer][q // group], hd)
    return idx


def input_perm(gguf_name, perms, dims):
    """Permutation of a tensor's input axis (GGUF ne[0]) or None (qwen3.py:106-123).
    Each returned permutation is checked (length, range, uniqueness) before it is used
    to move weights, importance vectors or Hessians."""
    if gguf_name in ("token_embd.weight", "output.weight"):
        return _check(perms["res"], dims["d_model"], "res permutation")
    if not gguf_name.startswith("blk."):
        return None
    parts = gguf_name.split(".")
    layer, kind = int(parts[1]), parts[2]
    if kind in RES_INPUT_KINDS:
        return _check(perms["res"], dims["d_model"], "res permutation")
    if kind == "ffn_down":
        return _check(perms["ffn"][layer], dims["d_ffn"], f"ffn permutation of layer {layer}")
    if kind == "attn_output":
        return o_input_index(perms, layer, dims)
    return None


def inverse(p):
    p = np.asarray(p)
    inv = np.empty_like(p)
    inv[p] = np.arange(p.size)
    return inv


def _dev_index(p, size, device, what):
    """A row or column index checked on the host (numpy's rules, negative entries from
    the end; IndexError before any launch) as a device int32 tensor."""
    if p is None:
        return None
    if np.shape(p) != (size,):
        raise ValueError(f"{what} has shape {tuple(np.shape(p))}, the axis has {size} entries")
    p = _lib.check_index(p, size, what)
    if isinstance(p, torch.Tensor):
        return p.to(device=device).contiguous()
    return torch.from_numpy(np.ascontiguousarray(p)).to(device)


def gather(t, rows=None, cols=None):
    """t[rows][:, cols] on the device (None = all), as numpy's t[np.ix_(rows, cols)].
    t: 2-D CUDA tensor of 1/2/4/8-byte elements; rows / cols have one entry per row /
    column of t. An index out of range raises IndexError before anything is launched."""
    if t.dim() != 2:
        raise ValueError("gather needs a 2-D tensor")
    R, C = t.shape
    rp = _dev_index(rows, R, t.device, "row index")
    cp = _dev_index(cols, C, t.device, "column index")
    lib = _lib.load()
    t = t.contiguous()
    out = torch.empty_like(t)
    st = lib.cp_permute_gather(_lib.ptr(t), _lib.ptr(out), _lib.ptr(rp), _lib.ptr(cp), R, C,
                               t.element_size(), _lib.stream_ptr())
    _lib.check(st)
    return out


def permute_hessian(H, p):
    """H[np.ix_(p, p)] (ef.py:289-290)."""
    return gather(H, p, p)


def _moved(w, rows=None, cols=None):
    """w[rows][:, cols] (a 1-D w: w[rows]) gathered on the GPU, returned on w's device."""
    t = w if w.is_cuda else w.cuda()
    if t.dim() == 1:
        out = gather(t.reshape(1, -1), None, rows).reshape(-1)
    else:
        out = gather(t, rows, cols)
    return out if w.is_cuda else out.to(w.device)


def _hf_moves(perms, dims):
    """{HF parameter suffix: (row index, column index)} of one decoder layer, per layer,
    plus the model-level ones: the moves of qwen3.apply_perms (qwen3.py:141-188). Every
    permutation is checked (IndexError / ValueError) before any of them is used."""
    P = _check(perms["res"], dims["d_model"], "res permutation")
    top = {"model.embed_tokens.weight": (None, P), "lm_head.weight": (None, P),
           "model.norm.weight": (P, None)}
    layers = []
    for l in range(dims["n_layers"]):
        Pf = _check(perms["ffn"][l], dims["d_ffn"], f"ffn permutation of layer {l}")
        v_idx, o_idx = v_output_index(perms, l, dims), o_input_index(perms, l, dims)
        layers.append({"input_layernorm.weight": (P, None),
                       "post_attention_layernorm.weight": (P, None),
                       "self_attn.q_proj.weight": (None, P), "self_attn.k_proj.weight": (None, P),
                       "self_attn.v_proj.weight": (v_idx, P), "self_attn.o_proj.weight": (P, o_idx),
                       "mlp.gate_proj.weight": (Pf, P), "mlp.up_proj.weight": (Pf, P),
                       "mlp.down_proj.weight": (P, Pf)})
    return top, layers


def apply_perms(sd, perms, dims, consume=False, strip_vision=False):
    """A new HF state dict with the permutations applied (qwen3.apply_perms,
    coldpress/perm/spacemaps/qwen3.py:141-188): the embedding (and an untied lm_head) by
    columns, every RMSNorm gain of the residual space, q/k/v/gate/up input columns, o/down
    output rows, v output rows per kv head, o input columns per q head, gate/up rows and
    down columns by the layer's FFN permutation. Every move is one GPU gather (both axes
    in one pass); tensors come back on their own device and dtype, other entries (q_norm /
    k_norm gains) unchanged. ``consume`` pops the moved entries from ``sd`` as they go;
    ``strip_vision`` is accepted for the interface (a text-only architecture)."""
    top, layers = _hf_moves(perms, dims)
    out = dict(sd)

    def move(name, rows, cols, required=True):
        if name not in sd:
            if required:
                raise KeyError(name)
            return
        w = sd.pop(name) if consume else sd[name]
        out[name] = _moved(w, rows, cols)

    for name, (rows, cols) in top.items():
        move(name, rows, cols, required=name != "lm_head.weight")
    for l, moves in enumerate(layers):
        for suffix, (rows, cols) in moves.items():
            move(f"model.layers.{l}.{suffix}", rows, cols)
    return out


def apply_perms_inplace(model, perms, dims):
    """Permute a loaded HF model's parameters in place (qwen3.apply_perms_inplace,
    qwen3.py:191-230). A tied lm_head shares the embedding's storage and is moved once."""
    top, layers = _hf_moves(perms, dims)
    params = dict(model.named_parameters())  # named_parameters lists a tied weight once
    with torch.no_grad():
        for name, (rows, cols) in top.items():
            if name in params:
                params[name].data = _moved(params[name].data, rows, cols)
        for l, moves in enumerate(layers):
            for suffix, (rows, cols) in moves.items():
                p = params[f"model.layers.{l}.{suffix}"]
                p.data = _moved(p.data, rows, cols)


def permute_layer(W, perms, layer, dims):
    """Permuted copies of one decoder layer's linear weights, keyed by GGUF kind
    (attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down), each
    [out_features, in_features] as in the HF state dict (qwen3.py:141-188)."""
    P = _check(perms["res"], dims["d_model"])
    Pf = _check(perms["ffn"][layer], dims["d_ffn"])
    out = {}
    out["attn_q"] = gather(W["attn_q"], None, P)
    out["attn_k"] = gather(W["attn_k"], None, P)
    out["attn_v"] = gather(W["attn_v"], v_output_index(perms, layer, dims), P)
    out["attn_output"] = gather(W["attn_output"], P, o_input_index(perms, layer, dims))
    out["ffn_gate"] = gather(W["ffn_gate"], Pf, P)
    out["ffn_up"] = gather(W["ffn_up"], Pf, P)
    out["ffn_down"] = gather(W["ffn_down"], P, Pf)
    return out


def unpermute_layer(Wp, perms, layer, dims):
    """Inverse of permute_layer (bit-exact)."""
    P = inverse(perms["res"])
    Pf = inverse(perms["ffn"][layer])
    v_idx = inverse(v_output_index(perms, layer, dims))
    o_idx = inverse(o_input_index(perms, layer, dims))
    return {"attn_q": gather(Wp["attn_q"], None, P), "attn_k": gather(Wp["attn_k"], None, P),
            "attn_v": gather(Wp["attn_v"], v_idx, P),
            "attn_output": gather(Wp["attn_output"], P, o_idx),
            "ffn_gate": gather(Wp["ffn_gate"], Pf, P), "ffn_up": gather(Wp["ffn_up"], Pf, P),
            "ffn_down": gather(Wp["ffn_down"], P, Pf)}


# ---------------------------------------------------------------- optimizer

def res_space_tensors(weights, dims):
    """Tensors whose input axis is the residual space, in the reference's order
    (qwen3.py:252-257)."""
    names = ["token_embd.weight", "output.weight"]
    for l in range(dims["n_layers"]):
        for k in RES_INPUT_KINDS:
            names.append(f"blk.{l}.{k}.weight")
    return [n for n in names if n in weights]


def build_res_keys(weights, dims, profiles=None):
    """Candidate residual sort keys from the per-tensor column profiles
    (qwen3.py:269-281)."""
    from .objective import col_log_rms
    keys, profs = {}, []
    for n in res_space_tensors(weights, dims):
        profs.append((n, profiles[n] if profiles is not None else col_log_rms(weights[n])))
    stand = [(p - p.mean()) / (p.std() + 1e-9) for _, p in profs]
    keys["mean-logrms"] = np.mean(stand, axis=0)
    emb = [p for n, p in profs if n == "token_embd.weight"]
    if emb:
        keys["embd-logrms"] = emb[0]
    blk = [s for (n, _), s in zip(profs, stand) if n.startswith("blk.")]
    if blk:
        keys["blk-logrms"] = np.mean(blk, axis=0)
    return keys


def optimize(weights, ttypes, qws, dims, rows_sample=16384, log=print):
    """Choose the res / ffn / vo permutations minimising the container objective
    (coldpress/perm/spacemaps/qwen3.py:284-355), with every objective evaluation on
    the GPU. No candidate depends on another's objective value: the residual keys
    come from column profiles, and the ffn_down / attn_output candidates act on the
    unpermuted weights. So the search takes two device round trips: one for the
    column profiles of every tensor involved, one for every objective item (each
    residual candidate over all residual-space tensors, the ffn_down and attn_output
    baselines and their candidates). The choices are then made in the reference's
    order from those values.

    weights : {gguf_name: [nrow, ne0] float16/float32, numpy or torch}; host arrays are
              uploaded once and stay resident for the whole search
    ttypes  : {gguf_name: target container type}
    qws     : {gguf_name: imatrix means [ne0]} (missing -> unweighted path)
    Returns (perms, report) with the reference's keys (report adds "key", the chosen
    residual candidate)."""
    import time
    from .objective import col_log_rms_many, index_dev, tensor_err_many, weights_dev
    t0 = time.time()
    dev = {n: weights_dev(w)[0] for n, w in weights.items()}
    qdev = {n: torch.from_numpy(np.ascontiguousarray(q, dtype=np.float32)).cuda()
            if str(getattr(q, "dtype", "")) == "float32" else q for n, q in qws.items()}
    res_names = res_space_tensors(dev, dims)
    L = dims["n_layers"]
    hd, nkv, nh = dims["head_dim"], dims["n_kv"], dims["n_heads"]
    group = nh // nkv
    fns = [f"blk.{l}.ffn_down.weight" for l in range(L)]
    ons = [f"blk.{l}.attn_output.weight" for l in range(L)]

    # round trip 1: column profiles of the residual-space tensors and of every
    # ffn_down / attn_output
    profs = col_log_rms_many([dev[n] for n in res_names] + [dev[fn] for fn in fns]
                             + [dev[on] for on in ons])
    profiles = dict(zip(res_names, profs[:len(res_names)]))
    profs = profs[len(res_names):]
    keys = build_res_keys(dev, dims, profiles)
    res_cands = [("identity", None)] + [(k, np.argsort(key, kind="stable")) for k, key in keys.items()]
    fcand = [np.argsort(p, kind="stable") for p in profs[:L]]
    heads_all, ocand = [], []
    for on, prof in zip(ons, profs[L:]):  # column sums are per column: slices share them
        heads = []
        for h in range(nkv):
            key = np.zeros(hd)
            for q in [q for q in range(nh) if q // group == h]:
                key = key + prof[q * hd:(q + 1) * hd]
            heads.append(np.argsort(key, kind="stable"))
        full = np.arange(nh * hd)
        for q in range(nh):
            full[q * hd:(q + 1) * hd] = q * hd + heads[q // group]
        heads_all.append(heads)
        ocand.append(full)

    # round trip 2: every objective item of the search in one batched pass
    items = []
    for _, perm in res_cands:
        pd = index_dev(perm, dims["d_model"]) if perm is not None else None
        items += [dict(x=dev[n], ttype=ttypes[n], qw=qdev.get(n), perm=pd, rows_sample=rows_sample)
                  for n in res_names]
    items += ([dict(x=dev[fn], ttype=ttypes[fn], qw=qdev.get(fn)) for fn in fns]
              + [dict(x=dev[fn], ttype=ttypes[fn], qw=qdev.get(fn), perm=p) for fn, p in zip(fns, fcand)]
              + [dict(x=dev[on], ttype=ttypes[on], qw=qdev.get(on)) for on in ons]
              + [dict(x=dev[on], ttype=ttypes[on], qw=qdev.get(on), perm=p) for on, p in zip(ons, ocand)])
    errs = tensor_err_many(items)
    nr = len(res_names)
    res_vals = [_ordered_sum(errs[k * nr:(k + 1) * nr]) for k in range(len(res_cands))]
    errs = errs[len(res_cands) * nr:]

    base = res_vals[0]
    res_perm, res_val, res_name = np.arange(dims["d_model"]), base, "identity"
    for (kname, perm), val in zip(res_cands[1:], res_vals[1:]):
        if val < res_val:
            res_perm, res_val, res_name = perm, val, kname
    log("residual space: " + ", ".join(
        f"{k} {v / base - 1:+.2%}" for (k, _p), v in zip(res_cands[1:], res_vals[1:]))
        + f" against the identity order; kept {res_name}")

    fb_all, fv_all = errs[0:L], errs[L:2 * L]
    ob_all, ov_all = errs[2 * L:3 * L], errs[3 * L:4 * L]
    ffn_perms, ffn_val, ffn_base = [], 0.0, 0.0
    vo_perms, vo_val, vo_base = [], 0.0, 0.0
    for l in range(L):
        fb, fp, fv = fb_all[l], fcand[l], fv_all[l]
        if fv >= fb:
            fp, fv = np.arange(dims["d_ffn"]), fb
        ffn_perms.append(fp)
        ffn_val += fv
        ffn_base += fb
        ob, heads, ov = ob_all[l], heads_all[l], ov_all[l]
        if ov >= ob:
            heads = [np.arange(hd) for _ in range(nkv)]
            ov = ob
        vo_perms.append(heads)
        vo_val += ov
        vo_base += ob

    def rel(v, b):
        return v / b - 1 if b else 0.0

    perms = {"res": res_perm, "ffn": ffn_perms, "vo": vo_perms}
    report = {"res": {"base": base, "opt": res_val, "rel": rel(res_val, base), "key": res_name},
              "ffn": {"base": ffn_base, "opt": ffn_val, "rel": rel(ffn_val, ffn_base)},
              "vo": {"base": vo_base, "opt": vo_val, "rel": rel(vo_val, vo_base)},
              "rows_sample": rows_sample, "seconds": time.time() - t0}
    return perms, report


def _ordered_sum(vals):
    """The reference's running total: 0.0 + v0 + v1 + ... in order (qwen3.py:260-266)."""
    total = 0.0
    for v in vals:
        total += v
    return total
