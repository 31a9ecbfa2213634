"""PERM index-move oracle (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates the Qwen3 space map's index constructions and moves
(coldpress/perm/spacemaps/qwen3.py:94-123 o_input_index / input_perm, :141-188
apply_perms) as numpy fancy indexing on [out, in] weight matrices, plus the
Hessian move H[np.ix_(p, p)] of ef.py:289-290. Pinned by exact invertibility
and by the reference tests' expectations (test_spacemap.py:53-64 shapes and
permutation validity; test_perm_optimize.py:63-100 movement of res / ffn /
attn_output input statistics).
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
