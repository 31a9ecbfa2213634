"""PERM index oracle and the host-side index logic of perm_amd.perm (no GPU):
shapes / validity as the reference's test_spacemap.py:53-64 checks them, exact
invertibility, and the input-statistics moves of test_perm_optimize.py:63-100."""
import numpy as np

from oracle import perm_oracle as Po
from perm_amd import perm as gp

DIMS = {"d_model": 256, "d_ffn": 512, "n_layers": 2, "n_heads": 4, "n_kv": 2, "head_dim": 64}


def random_perms(dims, seed=0):
    rng = np.random.default_rng(seed)
    return {"res": rng.permutation(dims["d_model"]),
            "ffn": [rng.permutation(dims["d_ffn"]) for _ in range(dims["n_layers"])],
            "vo": [[rng.permutation(dims["head_dim"]) for _ in range(dims["n_kv"])]
                   for _ in range(dims["n_layers"])]}


def test_input_perm_shapes_and_validity():
    perms = random_perms(DIMS, seed=7)
    assert gp.input_perm("token_embd.weight", perms, DIMS).shape == (DIMS["d_model"],)
    assert gp.input_perm("blk.0.attn_q.weight", perms, DIMS).shape == (DIMS["d_model"],)
    assert gp.input_perm("blk.1.ffn_down.weight", perms, DIMS).shape == (DIMS["d_ffn"],)
    aout = gp.input_perm("blk.0.attn_output.weight", perms, DIMS)
    assert aout.shape == (DIMS["n_heads"] * DIMS["head_dim"],)
    assert np.array_equal(np.sort(aout), np.arange(DIMS["n_heads"] * DIMS["head_dim"]))
    assert gp.input_perm("output_norm.weight", perms, DIMS) is None


def test_index_constructions_match_oracle():
    perms = random_perms(DIMS, seed=3)
    for l in range(2):
        assert np.array_equal(gp.o_input_index(perms, l, DIMS), Po.o_input_index(perms, l, DIMS))
        assert np.array_equal(gp.v_output_index(perms, l, DIMS), Po.v_output_index(perms, l, DIMS))
    # q heads of one GQA group share their kv head's permutation
    o = gp.o_input_index(perms, 0, DIMS)
    hd = DIMS["head_dim"]
    assert np.array_equal(o[0:hd], perms["vo"][0][0]) and np.array_equal(o[hd:2 * hd] - hd, perms["vo"][0][0])
    assert np.array_equal(o[2 * hd:3 * hd] - 2 * hd, perms["vo"][0][1])


def test_moves_invert_exactly():
    perms = random_perms(DIMS, seed=5)
    rng = np.random.default_rng(0)
    d, f, q, kv = DIMS["d_model"], DIMS["d_ffn"], DIMS["n_heads"] * DIMS["head_dim"], DIMS["n_kv"] * DIMS["head_dim"]
    W = {"attn_q": rng.standard_normal((q, d)), "attn_k": rng.standard_normal((kv, d)),
         "attn_v": rng.standard_normal((kv, d)), "attn_output": rng.standard_normal((d, q)),
         "ffn_gate": rng.standard_normal((f, d)), "ffn_up": rng.standard_normal((f, d)),
         "ffn_down": rng.standard_normal((d, f))}
    Wp = Po.permute_layer(W, perms, 1, DIMS)
    P, Pf = np.asarray(perms["res"]), np.asarray(perms["ffn"][1])
    o_idx, v_idx = Po.o_input_index(perms, 1, DIMS), Po.v_output_index(perms, 1, DIMS)
    inv = gp.inverse
    back = {"attn_q": Wp["attn_q"][:, inv(P)], "attn_k": Wp["attn_k"][:, inv(P)],
            "attn_v": Wp["attn_v"][inv(v_idx)][:, inv(P)],
            "attn_output": Wp["attn_output"][inv(P)][:, inv(o_idx)],
            "ffn_gate": Wp["ffn_gate"][inv(Pf)][:, inv(P)], "ffn_up": Wp["ffn_up"][inv(Pf)][:, inv(P)],
            "ffn_down": Wp["ffn_down"][inv(P)][:, inv(Pf)]}
    for k in W:
        assert np.array_equal(back[k], W[k]), k


def test_input_statistics_move_with_input_perm():
    """An input-space statistic (imatrix means, diag H) moves by input_perm
    (test_perm_optimize.py:96-100): x' = x[:, p] has column statistics s[p]."""
    perms = random_perms(DIMS, seed=1)
    rng = np.random.default_rng(2)
    X = rng.standard_normal((300, DIMS["n_heads"] * DIMS["head_dim"]))
    s = (X ** 2).mean(0)
    p = gp.input_perm("blk.0.attn_output.weight", perms, DIMS)
    assert np.allclose((X[:, p] ** 2).mean(0), s[p], rtol=1e-13, atol=0)
    H = X.T @ X
    assert np.allclose(Po.permute_hessian(H, p), X[:, p].T @ X[:, p], rtol=1e-12, atol=1e-12)
