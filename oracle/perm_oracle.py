"""PERM oracle (numpy): index moves and the container objective. TEST
INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates the Qwen3 space map's index constructions and moves
(coldpress/perm/spacemaps/qwen3.py:94-123 o_input_index / input_perm, :141-188
apply_perms) as numpy fancy indexing on [out, in] weight matrices, plus the
Hessian move H[np.ix_(p, p)] of ef.py:289-290. Pinned by exact invertibility
and by the reference tests' expectations (test_spacemap.py:53-64 shapes and
permutation validity; test_perm_optimize.py:63-100 movement of res / ffn /
attn_output input statistics).

The objective part (tensor_err, col_log_rms, optimize_qwen3) restates
coldpress/perm/objective.py:17-49 and qwen3.py:252-355 with numpy's own
reductions. Pins: the pairwise and sequential summation orders against numpy
itself (tests/test_oracle_perm.py), tensor_err against an exactly rounded
(math.fsum) evaluation of its formula, the identities of its row sample and
column permutation, col_log_rms against constant-column closed forms, and the
reference optimizer test's expectations (test_perm_optimize.py:45-61: valid
permutations, never worse than identity).
"""
import numpy as np


def o_input_index(perms, layer, dims):
    hd, nh = dims["head_dim"], dims["n_heads"]
    group = nh // dims["n_kv"]
    return np.concatenate([q * hd + np.asarray(perms["vo"][layer][q // group])
                           for q in range(nh)])


def v_output_index(perms, layer, dims):
    hd = dims["head_dim"]
    return np.concatenate([h * hd + np.asarray(perms["vo"][layer][h])
                           for h in range(dims["n_kv"])])


def permute_layer(W, perms, layer, dims):
    P = np.asarray(perms["res"])
    Pf = np.asarray(perms["ffn"][layer])
    return {"attn_q": W["attn_q"][:, P], "attn_k": W["attn_k"][:, P],
            "attn_v": W["attn_v"][:, P][v_output_index(perms, layer, dims)],
            "attn_output": W["attn_output"][P][:, o_input_index(perms, layer, dims)],
            "ffn_gate": W["ffn_gate"][:, P][Pf], "ffn_up": W["ffn_up"][:, P][Pf],
            "ffn_down": W["ffn_down"][P][:, Pf]}


def permute_hessian(H, p):
    return H[np.ix_(p, p)]


# ------------------------------------------------------------------ PERM objective
# coldpress/perm/objective.py:17-49 and the Qwen3 optimizer that calls it
# (coldpress/perm/spacemaps/qwen3.py:252-355). The reductions are numpy's own:
#   * d2.sum(0) over a C-contiguous [R, C] float64 array adds the rows one after
#     another into a zero-initialised row (a sequential chain per column);
#   * a contiguous 1-D float64 .sum() is +0.0 plus numpy's pairwise sum
#     (``pairwise_sum`` below restates it, so a test can pin numpy against it).

from . import kquant_oracle as _K

_PW_BLOCK = 128


def pairwise_sum(a):
    """numpy's pairwise summation of a contiguous 1-D float64 array, in pure Python
    floats: < 8 values sequentially from 0.0; <= 128 values with eight strided
    accumulators then ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) and the remainder
    sequentially; longer runs split at n/2 rounded down to a multiple of 8."""
    a = [float(v) for v in a]

    def pw(lo, n):
        if n < 8:
            r = 0.0
            for i in range(n):
                r += a[lo + i]
            return r
        if n <= _PW_BLOCK:
            r = a[lo:lo + 8]
            i = 8
            while i < n - (n % 8):
                for j in range(8):
                    r[j] += a[lo + i + j]
                i += 8
            s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
            while i < n:
                s += a[lo + i]
                i += 1
            return s
        n2 = n // 2
        n2 -= n2 % 8
        return pw(lo, n2) + pw(lo + n2, n - n2)

    return 0.0 + pw(0, len(a))


def sample_rows(nrow, rows_sample, seed=0):
    """Sorted row sample of objective.py:21-24, or None when every row is used."""
    if rows_sample and nrow > rows_sample:
        rng = np.random.default_rng(seed)
        return np.sort(rng.choice(nrow, rows_sample, replace=False))
    return None


def tensor_err(x, ttype, qw, perm=None, wvec=None, rows_sample=None, seed=0):
    """Weighted quantization error of x[:, perm] at container ttype (objective.py:17-39)."""
    if ttype in ("F16", "F32", "BF16"):
        return 0.0
    idx = sample_rows(x.shape[0], rows_sample, seed)
    if idx is not None:
        x = x[idx]
    x = np.asarray(x, dtype=np.float32)
    if perm is not None:
        x = x[:, perm]
        qw = qw[perm] if qw is not None else None
    if ttype not in _K.QUANTIZE:
        raise ValueError(f"no encoder for {ttype}")
    with np.errstate(all="ignore"):
        recon = _K.roundtrip(np.ascontiguousarray(x), ttype, qw)
    d2 = (recon.astype(np.float64) - x.astype(np.float64)) ** 2
    colerr = d2.sum(0)
    if wvec is not None:
        w = wvec[perm] if perm is not None else wvec
        return float((colerr * w).sum())
    if qw is not None:
        return float((colerr * qw).sum())
    return float(colerr.sum())


def col_log_rms(x, row_step=32768):
    """Per-column log-RMS, float64 sums in chunks of row_step rows (objective.py:42-49)."""
    x = np.asarray(x)
    acc = np.zeros(x.shape[1], np.float64)
    for r0 in range(0, x.shape[0], row_step):
        xc = np.asarray(x[r0:r0 + row_step], dtype=np.float64)
        acc += (xc ** 2).sum(0)
    return np.log(np.sqrt(acc / x.shape[0]) + 1e-12)


RES_TENSORS_PER_LAYER = ["attn_q", "attn_k", "attn_v", "ffn_gate", "ffn_up"]


def res_space_tensors(weights, dims):
    """Tensors whose input axis is the residual space, in the reference's order
    (qwen3.py:252-257)."""
    names = ["token_embd.weight", "output.weight"]
    for l in range(dims["n_layers"]):
        for k in RES_TENSORS_PER_LAYER:
            names.append(f"blk.{l}.{k}.weight")
    return [n for n in names if n in weights]


def build_res_keys(weights, dims):
    """Candidate residual sort keys (qwen3.py:269-281)."""
    keys, profs = {}, []
    for n in res_space_tensors(weights, dims):
        profs.append((n, col_log_rms(weights[n])))
    stand = [(p - p.mean()) / (p.std() + 1e-9) for _, p in profs]
    keys["mean-logrms"] = np.mean(stand, axis=0)
    emb = [p for n, p in profs if n == "token_embd.weight"]
    if emb:
        keys["embd-logrms"] = emb[0]
    blk = [s for (n, _), s in zip(profs, stand) if n.startswith("blk.")]
    if blk:
        keys["blk-logrms"] = np.mean(blk, axis=0)
    return keys


def optimize_qwen3(weights, ttypes, qws, dims, rows_sample=16384, log=lambda *_: None):
    """Choose the res / ffn / vo permutations minimising the container objective
    (qwen3.py:260-266, 284-355). Returns (perms, report) without the wall-clock field."""
    def res_obj(perm):
        total = 0.0
        for n in res_space_tensors(weights, dims):
            total += tensor_err(weights[n], ttypes[n], qws.get(n), perm=perm,
                                rows_sample=rows_sample)
        return total

    base = res_obj(None)
    res_perm, res_val, res_name = np.arange(dims["d_model"]), base, "identity"
    for kname, key in build_res_keys(weights, dims).items():
        perm = np.argsort(key, kind="stable")
        val = res_obj(perm)
        log(f"  res sort[{kname}]: {val:.6g}")
        if val < res_val:
            res_perm, res_val, res_name = perm, val, kname
    ffn_perms, ffn_val, ffn_base = [], 0.0, 0.0
    vo_perms, vo_val, vo_base = [], 0.0, 0.0
    hd, nkv, nh = dims["head_dim"], dims["n_kv"], dims["n_heads"]
    group = nh // nkv
    for l in range(dims["n_layers"]):
        fn = f"blk.{l}.ffn_down.weight"
        fb = tensor_err(weights[fn], ttypes[fn], qws.get(fn))
        fp = np.argsort(col_log_rms(weights[fn]), kind="stable")
        fv = tensor_err(weights[fn], ttypes[fn], qws.get(fn), perm=fp)
        if fv >= fb:
            fp, fv = np.arange(dims["d_ffn"]), fb
        ffn_perms.append(fp)
        ffn_val += fv
        ffn_base += fb
        on = f"blk.{l}.attn_output.weight"
        x = np.asarray(weights[on])
        ob = tensor_err(x, ttypes[on], qws.get(on))
        heads = []
        for h in range(nkv):
            key = np.zeros(hd)
            for q in [q for q in range(nh) if q // group == h]:
                key = key + col_log_rms(x[:, q * hd:(q + 1) * hd])
            heads.append(np.argsort(key, kind="stable"))
        full = np.arange(nh * hd)
        for q in range(nh):
            full[q * hd:(q + 1) * hd] = q * hd + heads[q // group]
        ov = tensor_err(x, ttypes[on], qws.get(on), perm=full)
        if ov >= ob:
            heads = [np.arange(hd) for _ in range(nkv)]
            ov = ob
        vo_perms.append(heads)
        vo_val += ov
        vo_base += ob
    perms = {"res": res_perm, "ffn": ffn_perms, "vo": vo_perms}

    def rel(v, b):
        return v / b - 1 if b else 0.0

    report = {"res": {"base": base, "opt": res_val, "rel": rel(res_val, base), "key": res_name},
              "ffn": {"base": ffn_base, "opt": ffn_val, "rel": rel(ffn_val, ffn_base)},
              "vo": {"base": vo_base, "opt": vo_val, "rel": rel(vo_val, vo_base)},
              "rows_sample": rows_sample}
    return perms, report
