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
    N = 8192
    H = {fam: xtx_accumulate(student_t_activations(N, d, seed=i))
         for i, (fam, d) in enumerate([("qkv_in", 1024), ("o_in", 2048), ("gateup_in", 1024), ("down_in", 3072)])}
    fam_of = {"attn_q": "qkv_in", "attn_k": "qkv_in", "attn_v": "qkv_in", "attn_output": "o_in",
              "ffn_gate": "gateup_in", "ffn_up": "gateup_in", "ffn_down": "down_in"}
    Wp = gp.permute_layer(W, perms, 0, DIMS)

    def encode(x, Hm):
        qw = (torch.diagonal(Hm) / N).contiguous()
        raw, _ = gef.ef_encode(x, "Q2_K", qw, Hm)
        return raw

    # row moves: bytes move with the rows
    for k, idx in (("ffn_gate", perms["ffn"][0]), ("ffn_up", perms["ffn"][0]),
                   ("attn_v", gp.v_output_index(perms, 0, DIMS))):
        base = encode(W[k], H[fam_of[k]])
        perm_raw = encode(Wp[k], H[fam_of[k]])
        assert torch.equal(perm_raw, base[torch.from_numpy(idx).cuda()]), k
    # column moves: H and qw move with the input channels; bytes equal the oracle's
    for k, p in (("ffn_down", perms["ffn"][0]), ("attn_output", gp.o_input_index(perms, 0, DIMS))):
        Hp = gp.permute_hessian(H[fam_of[k]], p)
        x = Wp[k][:64].contiguous()
        got = encode(x, Hp).cpu().numpy()
        Hn = Hp.double().cpu().numpy()
        want, _ = E.ef_encode(x.cpu().numpy(), "Q2_K", (np.diag(Hn) / N).astype(F32), Hn,
                              stable_order=True)
        assert np.array_equal(got, want), k
