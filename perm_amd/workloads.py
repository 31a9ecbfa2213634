"""Seeded synthetic workloads for the encoder path (weights, activations, Hessians).

Shapes follow the reference's target models; there is no network, so weights
are random-init and activations synthetic, with the statistics each workload
names. The draw order of every generator is fixed: changing it changes the
workload.
"""
import numpy as np

F32 = np.float32

# Qwen3-0.6B linear layers: (name, out_features = rows, in_features = n, Hessian family)
QWEN3_06B_LAYER = [
    ("attn_q", 2048, 1024, "qkv_in"),
    ("attn_k", 1024, 1024, "qkv_in"),
    ("attn_v", 1024, 1024, "qkv_in"),
    ("attn_output", 1024, 2048, "o_in"),
    ("ffn_gate", 3072, 1024, "gateup_in"),
    ("ffn_up", 3072, 1024, "gateup_in"),
    ("ffn_down", 1024, 3072, "down_in"),
]
QWEN3_06B_FAMILIES = {"qkv_in": 1024, "o_in": 2048, "gateup_in": 1024, "down_in": 3072}
QWEN3_06B_LAYERS = 28


def single_linear(seed=0, nrow=1024, n=1024, n_act=8192, outlier_frac=0.01, outlier_gain=20.0):
    """One synthetic Linear on the reference's CPU path.

    W [nrow, n] = N(0, 0.02^2) times a per-row log-normal(sigma 0.5) scale;
    X [n_act, n] = N(0, 1) times per-channel log-normal(sigma 1) scales, with
    floor(outlier_frac * n) channels (rng.choice, without replacement) x outlier_gain;
    H = X^T X / n_act in float64. Returns (W f32, X f32, H f64)."""
    rng = np.random.default_rng(seed)
    W = rng.normal(0.0, 0.02, size=(nrow, n)) * np.exp(rng.normal(0.0, 0.5, size=(nrow, 1)))
    scale = np.exp(rng.normal(0.0, 1.0, size=n))
    out = rng.choice(n, int(outlier_frac * n), replace=False)
    scale[out] *= outlier_gain
    X = (rng.standard_normal((n_act, n)) * scale).astype(F32)
    Xd = X.astype(np.float64)
    H = Xd.T @ Xd / n_act
    return W.astype(F32), X, H


def student_t_activations(n_rows, d, nu=4.0, seed=0, device="cuda", dtype=None):
    """Heavy-tailed activations on the device: Student-t(nu) times per-channel
    log-normal(sigma 1) scales, as bfloat16 by default. Generated with torch's
    device RNG (seeded) so the 65536-row batches never cross PCIe."""
    import torch
    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    z = torch.randn((n_rows, d), generator=g, device=device)
    # chi-square(nu) / nu from nu standard normals squared (nu = 4)
    chi = torch.zeros((n_rows, 1), device=device)
    for _ in range(int(nu)):
        chi += torch.randn((n_rows, 1), generator=g, device=device) ** 2
    t = z / torch.sqrt(chi / nu)
    scale = torch.exp(torch.randn((d,), generator=g, device=device))
    return (t * scale).to(dtype)


def qwen3_layer_weights(layer, seed=0, device="cuda"):
    """Random-init fp32 weights N(0, 0.02^2) for one Qwen3-0.6B decoder layer:
    {name: [rows, n]} on the device."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed * 1000 + layer)
    return {name: torch.randn((rows, n), generator=g, device=device) * 0.02
            for name, rows, n, _fam in QWEN3_06B_LAYER}


QWEN3_06B_DIMS = {"d_model": 1024, "d_ffn": 3072, "n_layers": 28, "n_heads": 16, "n_kv": 8,
                  "head_dim": 128}
QWEN3_06B_VOCAB = 151936


def qwen3_gguf_weights(layers=QWEN3_06B_LAYERS, seed=0, device="cuda"):
    """Random-init float16 weights of the Qwen3-0.6B linear set under their GGUF names
    (token_embd [151936, 1024] plus 7 tensors per layer, [out, in]), for the PERM
    search. Entries are N(0, 0.02^2) times a per-input-channel log-normal(sigma 0.5)
    scale shared by every tensor reading the same space (the residual stream, each
    layer's FFN intermediate and attention value space), so the channel profiles the
    search sorts by are not flat."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def scale(n):
        return torch.exp(0.5 * torch.randn((n,), generator=g, device=device))

    def mat(rows, n, s):
        return (torch.randn((rows, n), generator=g, device=device) * 0.02 * s).to(torch.float16)

    res = scale(1024)
    w = {"token_embd.weight": mat(QWEN3_06B_VOCAB, 1024, res)}
    for l in range(layers):
        ffn, vo = scale(3072), scale(2048)
        for name, rows, n, fam in QWEN3_06B_LAYER:
            s = {"qkv_in": res, "gateup_in": res, "down_in": ffn, "o_in": vo}[fam]
            w[f"blk.{l}.{name}.weight"] = mat(rows, n, s)
    return w


def qwen3_mixed_typemap(names):
    """The mixed container of the tied-output workload: Q6_K for the token
    embedding / output matrix, Q3_K for attention, Q2_K elsewhere."""
    out = {}
    for n in names:
        if n in ("token_embd.weight", "output.weight"):
            out[n] = "Q6_K"
        elif ".attn_" in n:
            out[n] = "Q3_K"
        else:
            out[n] = "Q2_K"
    return out


def imatrix_means(weights, seed=0):
    """imatrix-style importance vectors (positive per-input-channel means) for every
    tensor except the token embedding / output, which llama.cpp quantizes unweighted."""
    rng = np.random.default_rng(seed)
    return {n: (np.abs(rng.standard_normal(w.shape[1])) + 0.1).astype(F32)
            for n, w in weights.items() if n not in ("token_embd.weight", "output.weight")}


# ---------------------------------------------------------------- benchmark configs
# The reference's benchmark configurations beyond the headline one, as tensor lists over
# Hessian families. A family is one input space of a decoder layer: its Hessian comes
# from ``rows`` synthetic activation rows of width d; every tensor reading that input
# shares it. ``qw``: "diag" (imatrix-style channel means diag(H)/N) or None.

LLAMA3_8B_LAYER = [
    ("attn_q", 4096, 4096, "qkv_in"),
    ("attn_k", 1024, 4096, "qkv_in"),
    ("attn_v", 1024, 4096, "qkv_in"),
    ("attn_output", 4096, 4096, "o_in"),
    ("ffn_gate", 14336, 4096, "gateup_in"),
    ("ffn_up", 14336, 4096, "gateup_in"),
    ("ffn_down", 4096, 14336, "down_in"),
]
LLAMA3_8B_FAMILIES = {"qkv_in": 4096, "o_in": 4096, "gateup_in": 4096, "down_in": 14336}


def config_spec(name):
    """{"families": {key: (d, rows, activation kind)}, "tensors": [(key, rows, n, family,
    container, qw)], "layers", "normalize"} of a named workload:

    single-linear   one 1024 x 1024 Linear, Q2_K, H = X^T X / 8192 from float32 rows
                    (single_linear: 1 % outlier channels x20), qw = diag(H)
    tied-output     the Qwen3-0.6B 28-layer set with Q3_K attention and Q2_K MLP, plus the
                    tied 151936 x 1024 output matrix in Q6_K with no qw, its H from 65536
                    final-hidden-state rows N(0, 1) with log-normal channel scales
    llama3-8b-layer one Llama-3-8B decoder layer in Q4_K: H 4096^2 for q/k/v, o and
                    gate/up, 14336^2 for down, from 131072 rows with 0.5 % outlier
                    channels x50
    """
    if name == "single-linear":
        return {"families": {"linear_in": (1024, 8192, "single-linear")},
                "tensors": [("linear", 1024, 1024, "linear_in", "Q2_K", "diag")],
                "layers": 1, "normalize": True}
    if name == "tied-output":
        fams, tens = {}, []
        for l in range(QWEN3_06B_LAYERS):
            for fam, d in QWEN3_06B_FAMILIES.items():
                fams[f"blk.{l}.{fam}"] = (d, 65536, "student-t")
            for nm, rows, n, fam in QWEN3_06B_LAYER:
                tens.append((f"blk.{l}.{nm}", rows, n, f"blk.{l}.{fam}",
                             "Q3_K" if nm.startswith("attn") else "Q2_K", "diag"))
        fams["output_in"] = (1024, 65536, "lognormal")
        tens.append(("output", QWEN3_06B_VOCAB, 1024, "output_in", "Q6_K", None))
        return {"families": fams, "tensors": tens, "layers": QWEN3_06B_LAYERS,
                "normalize": False}
    if name == "llama3-8b-layer":
        fams = {f"blk.0.{fam}": (d, 131072, "outliers") for fam, d in LLAMA3_8B_FAMILIES.items()}
        tens = [(f"blk.0.{nm}", rows, n, f"blk.0.{fam}", "Q4_K", "diag")
                for nm, rows, n, fam in LLAMA3_8B_LAYER]
        return {"families": fams, "tensors": tens, "layers": 1, "normalize": False}
    raise KeyError(name)


def family_activations(kind, rows, d, seed, device="cuda"):
    """Synthetic activation rows of one Hessian family on the device:
    student-t   Student-t (nu = 4) times log-normal(sigma 1) channel scales, bfloat16
    lognormal   N(0, 1) times log-normal(sigma 1) channel scales, bfloat16
    outliers    as lognormal, with 0.5 % of the channels (at least one) scaled x50
    single-linear   single_linear's float32 rows (host draw, seed 0; 1 % outliers x20)
    """
    import torch
    if kind == "student-t":
        return student_t_activations(rows, d, nu=4.0, seed=seed, device=device)
    if kind == "single-linear":
        _w, X, _h = single_linear(seed=0, n=d, n_act=rows)
        return torch.from_numpy(X).to(device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    scale = torch.exp(torch.randn((d,), generator=g, device=device))
    if kind == "outliers":
        k = max(1, int(0.005 * d))
        scale[torch.randperm(d, generator=g, device=device)[:k]] *= 50.0
    elif kind != "lognormal":
        raise KeyError(kind)
    return (torch.randn((rows, d), generator=g, device=device) * scale).to(torch.bfloat16)


def spec_weights(spec, seed=0, device="cuda"):
    """Random-init float32 weights N(0, 0.02^2) of every tensor of a spec, on the device
    (single-linear: single_linear's W, with its per-row log-normal scales)."""
    import torch
    if any(kind == "single-linear" for _d, _r, kind in spec["families"].values()):
        (name, rows, n, *_), = spec["tensors"]
        W, _x, _h = single_linear(seed=0, nrow=rows, n=n)
        return {name: torch.from_numpy(W).to(device)}
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return {name: torch.randn((rows, n), generator=g, device=device) * 0.02
            for name, rows, n, _fam, _tt, _qw in spec["tensors"]}
