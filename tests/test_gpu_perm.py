"""GPU PERM moves (row/column gathers) and the permuted-layer EF encode of the
Qwen3-0.6B shape: moves bit-exact against numpy and exactly invertible; EF on
row-permuted tensors gives the row-permuted bytes; EF on column-permuted
tensors (with the Hessian and importance moved along) gives the oracle's bytes
for the same permuted inputs."""
import numpy as np
import pytest
import torch

from oracle import ef_oracle as E
from oracle import perm_oracle as Po

pytestmark = pytest.mark.gpu
F32 = np.float32
DIMS = {"d_model": 1024, "d_ffn": 3072, "n_layers": 1, "n_heads": 16, "n_kv": 8, "head_dim": 128}


@pytest.fixture(scope="module")
def gp():
    from perm_amd import perm
    return perm


def _perms(seed, res=False):
    rng = np.random.default_rng(seed)
    return {"res": rng.permutation(DIMS["d_model"]) if res else np.arange(DIMS["d_model"]),
            "ffn": [rng.permutation(DIMS["d_ffn"])],
            "vo": [[rng.permutation(DIMS["head_dim"]) for _ in range(DIMS["n_kv"])]]}


@pytest.mark.parametrize("dtype", [torch.uint8, torch.bfloat16, torch.float32, torch.float64])
def test_gather_matches_numpy(gp, dtype):
    rng = np.random.default_rng(0)
    for R, C in [(7, 13), (300, 1024), (1, 5000)]:
        a = torch.from_numpy(rng.standard_normal((R, C)).astype(np.float32) * 50).to(dtype).cuda()
        rp, cp = rng.permutation(R), rng.permutation(C)
        want = a.cpu()[torch.from_numpy(rp)][:, torch.from_numpy(cp)]
        assert torch.equal(gp.gather(a, rp, cp).cpu(), want)
        assert torch.equal(gp.gather(a, None, cp).cpu(), a.cpu()[:, torch.from_numpy(cp)])
        assert torch.equal(gp.gather(a, rp, None).cpu(), a.cpu()[torch.from_numpy(rp)])


@pytest.mark.parametrize("shape", [(0, 16), (16, 0), (0, 0)])
def test_gather_empty(gp, shape):
    """Empty tensors permute to empty tensors, as numpy / torch indexing does."""
    R, C = shape
    a = torch.zeros(shape, dtype=torch.float32, device="cuda")
    out = gp.gather(a, np.arange(R)[::-1].copy(), np.arange(C)[::-1].copy())
    assert out.is_cuda and tuple(out.shape) == shape


def test_layer_permute_roundtrip(gp):
    from perm_amd.workloads import qwen3_layer_weights
    W = qwen3_layer_weights(0, seed=3)
    perms = _perms(11, res=True)
    Wp = gp.permute_layer(W, perms, 0, DIMS)
    Wn = {k: v.cpu().numpy() for k, v in W.items()}
    want = Po.permute_layer(Wn, perms, 0, DIMS)
    for k in W:
        assert np.array_equal(Wp[k].cpu().numpy(), want[k]), k
    back = gp.unpermute_layer(Wp, perms, 0, DIMS)
    for k in W:
        assert torch.equal(back[k], W[k]), k


def test_permuted_layer_ef(gp):
    """Config-5 style: ffn and vo spaces permuted (res identity), Q2_K EF."""
    from perm_amd import ef as gef
    from perm_amd.workloads import qwen3_layer_weights, student_t_activations
    from perm_amd.hessians import xtx_accumulate
    W = qwen3_layer_weights(0, seed=5)
    perms = _perms(21)
    N = 65536
    H = {fam: xtx_accumulate(student_t_activations(N, d, seed=i))
         for i, (fam, d) in enumerate([("qkv_in", 1024), ("o_in", 2048), ("gateup_in", 1024), ("down_in", 3072)])}
    fam_of = {"attn_q": "qkv_in", "attn_k": "qkv_in", "attn_v": "qkv_in", "attn_output": "o_in",
              "ffn_gate": "gateup_in", "ffn_up": "gateup_in", "ffn_down": "down_in"}
    Wp = gp.permute_layer(W, perms, 0, DIMS)

    def encode(x, Hm):
        qw = (torch.diagonal(Hm) / N).contiguous()
        raw, _ = gef.ef_encode(x, "Q2_K", qw, Hm)
        return raw

    # row moves: bytes move with the rows, and a row slice of the permuted tensor is the
    # oracle's encode of those rows with the GPU's own factor and order
    for k, idx in (("ffn_gate", perms["ffn"][0]), ("ffn_up", perms["ffn"][0]),
                   ("attn_v", gp.v_output_index(perms, 0, DIMS))):
        Hm = H[fam_of[k]]
        base = encode(W[k], Hm)
        perm_raw = encode(Wp[k], Hm)
        assert torch.equal(perm_raw, base[torch.from_numpy(idx).cuda()]), k
        order = gef.act_order_dev(Hm)
        U, _ = gef.factor_dev(Hm, order, 0.01, checked=True)
        qw = (torch.diagonal(Hm) / N).contiguous().cpu().numpy()
        rows = np.r_[0:4, Wp[k].shape[0] - 4:Wp[k].shape[0]]
        want, _ = E.ef_encode(Wp[k].cpu().numpy()[rows], "Q2_K", qw, None, U=U.cpu().numpy(),
                              order=order.cpu().numpy().astype(np.int64))
        assert np.array_equal(perm_raw.cpu().numpy()[rows], want), k
    # column moves: H and qw move with the input channels; bytes equal the oracle's
    for k, p in (("ffn_down", perms["ffn"][0]), ("attn_output", gp.o_input_index(perms, 0, DIMS))):
        Hp = gp.permute_hessian(H[fam_of[k]], p)
        x = Wp[k][:64].contiguous()
        got = encode(x, Hp).cpu().numpy()
        Hn = Hp.double().cpu().numpy()
        want, _ = E.ef_encode(x.cpu().numpy(), "Q2_K", (np.diag(Hn) / N).astype(F32), Hn,
                              stable_order=True)
        assert np.array_equal(got, want), k


def _hf_perms(dims, seed):
    rng = np.random.default_rng(seed)
    return {"res": rng.permutation(dims["d_model"]),
            "ffn": [rng.permutation(dims["d_ffn"]) for _ in range(dims["n_layers"])],
            "vo": [[rng.permutation(dims["head_dim"]) for _ in range(dims["n_kv"])]
                   for _ in range(dims["n_layers"])]}


def _moves_numpy(sd, perms, dims):
    """The moves of qwen3.apply_perms (qwen3.py:141-188) with numpy fancy indexing."""
    P = perms["res"]
    hd, nkv, nh = dims["head_dim"], dims["n_kv"], dims["n_heads"]
    group = nh // nkv
    w = {k: v.float().numpy() if v.dtype != torch.bfloat16 else v.view(torch.int16).numpy()
         for k, v in sd.items()}
    out = dict(w)
    out["model.embed_tokens.weight"] = w["model.embed_tokens.weight"][:, P]
    out["lm_head.weight"] = w["lm_head.weight"][:, P]
    out["model.norm.weight"] = w["model.norm.weight"][P]
    for l in range(dims["n_layers"]):
        pre, Pf = f"model.layers.{l}.", perms["ffn"][l]
        v_idx = np.concatenate([h * hd + perms["vo"][l][h] for h in range(nkv)])
        o_idx = np.concatenate([q * hd + perms["vo"][l][q // group] for q in range(nh)])
        for n in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            out[pre + n] = w[pre + n][P]
        for n in ("self_attn.q_proj.weight", "self_attn.k_proj.weight"):
            out[pre + n] = w[pre + n][:, P]
        out[pre + "self_attn.v_proj.weight"] = w[pre + "self_attn.v_proj.weight"][np.ix_(v_idx, P)]
        out[pre + "self_attn.o_proj.weight"] = w[pre + "self_attn.o_proj.weight"][np.ix_(P, o_idx)]
        for n in ("mlp.gate_proj.weight", "mlp.up_proj.weight"):
            out[pre + n] = w[pre + n][np.ix_(Pf, P)]
        out[pre + "mlp.down_proj.weight"] = w[pre + "mlp.down_proj.weight"][np.ix_(P, Pf)]
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_apply_perms_state_dict_moves(dtype):
    """apply_perms on an HF state dict (CPU tensors, moved on the GPU) equals numpy's
    moves entry for entry, keeps devices and dtypes, and with consume=True empties the
    moved entries out of the input."""
    from conftest import TINY_DIMS, tiny_hf_decoder
    from perm_amd import perm as gp
    sd = {k: v.to(dtype) for k, v in tiny_hf_decoder("qwen3").state_dict().items()}
    perms = _hf_perms(TINY_DIMS, 5)
    got = gp.apply_perms(dict(sd), perms, TINY_DIMS)
    want = _moves_numpy(sd, perms, TINY_DIMS)
    assert set(got) == set(sd)
    for k, v in got.items():
        assert v.device.type == "cpu" and v.dtype == dtype, k
        a = v.float().numpy() if dtype != torch.bfloat16 else v.view(torch.int16).numpy()
        assert np.array_equal(a, want[k]), k
    src = dict(sd)
    gp.apply_perms(src, perms, TINY_DIMS, consume=True)
    assert sorted(src) == sorted(k for k in sd if "q_norm" in k or "k_norm" in k)


@pytest.mark.parametrize("tie", [False, True])
def test_apply_perms_inplace_preserves_logits(tie):
    """The reference's G3 gate (gates.py:21-32, qwen3.g3_check): the permuted fp32 model
    gives the original logits (rel < 1e-4), for an untied and a tied lm_head."""
    from conftest import TINY_DIMS, tiny_hf_decoder
    from perm_amd import perm as gp
    model = tiny_hf_decoder("qwen3", tie=tie, seed=2)
    ids = torch.from_numpy(np.random.default_rng(1).integers(0, 128, (1, 24)))
    with torch.no_grad():
        ref = model(ids).logits
    before = model.model.layers[0].mlp.down_proj.weight.detach().clone()
    gp.apply_perms_inplace(model, _hf_perms(TINY_DIMS, 9), TINY_DIMS)
    assert not torch.equal(before, model.model.layers[0].mlp.down_proj.weight)
    assert (model.lm_head.weight is model.model.embed_tokens.weight) == tie
    with torch.no_grad():
        got = model(ids).logits
    rel = float((got - ref).abs().max() / ref.abs().max())
    assert rel < 1e-4, rel
