"""Full-shape parity cases beyond the headline workload.

* Tied Qwen3-0.6B output matrix (151936 x 1024) under Q6_K EF with no importance
  vector, H from 65536 final-hidden-state rows N(0,1) with log-normal channel
  scales; a Q3_K attention tensor of the same model.
* Llama-3-8B-shaped ffn_down (4096 x 14336) under Q4_K EF with H (14336^2) from
  131072 activation rows with 0.5 % outlier channels x50: the fp64 factor at
  n = 14336 and the sweep.

The oracle cannot redo these in test time at full size, so the size-independent
property used is row independence: EF of a row slice with the same factor and
order equals the same rows of the full GPU encode, and the slice is compared
bit-exactly with the oracle's sweep fed the GPU's float32 factor and order."""
import numpy as np
import pytest
import torch

from oracle import ef_oracle as E

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def mods():
    from perm_amd import ef, hessians, workloads
    return ef, hessians, workloads


def _say(m):
    print(m, flush=True)


def _activations(N, d, seed, outlier_frac=0.0, gain=1.0, heavy=False):
    from perm_amd.workloads import student_t_activations
    if heavy:
        return student_t_activations(N, d, seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    scale = torch.exp(torch.randn((d,), generator=g, device="cuda"))
    if outlier_frac:
        k = int(outlier_frac * d)
        idx = torch.randperm(d, generator=g, device="cuda")[:k]
        scale[idx] *= gain
    return (torch.randn((N, d), generator=g, device="cuda") * scale).to(torch.bfloat16)


def _check_slice(ef, x, tt, qw, H, U, order, raw, rows):
    xs = x[rows].cpu().numpy()
    qn = qw.cpu().numpy() if qw is not None else None
    want, _ = E.ef_encode(xs, tt, qn, None, U=U.cpu().numpy(), order=order.cpu().numpy().astype(np.int64))
    got = raw[rows].cpu().numpy()
    assert np.array_equal(got, want), f"{tt}: rows {rows} differ from the oracle"


def test_tied_output_q6k(mods):
    ef, hs, wl = mods
    _say("config: tied output 151936 x 1024, Q6_K, qw None")
    H = hs.xtx_accumulate(_activations(65536, 1024, seed=7))
    g = torch.Generator(device="cuda").manual_seed(1)
    W = torch.randn((151936, 1024), generator=g, device="cuda") * 0.02
    order = ef.act_order_dev(H)
    U, _ = ef.factor_dev(H, order)
    (raw, rec), = ef.ef_encode_dev([{"ttype": "Q6_K", "x": W, "qw": None, "U": U, "order": order}])
    assert raw.shape == (151936, 4 * 210) and torch.isfinite(rec).all()
    for rows in (slice(0, 8), slice(151920, 151936)):
        _check_slice(ef, W, "Q6_K", None, H, U, order, raw, rows)


def test_attention_q3k(mods):
    ef, hs, wl = mods
    _say("config: q_proj 2048 x 1024, Q3_K, qw = diag(H)/N")
    H = hs.xtx_accumulate(_activations(65536, 1024, seed=3, heavy=True))
    W = wl.qwen3_layer_weights(0, seed=9)["attn_q"]
    qw = (torch.diagonal(H) / 65536).contiguous()
    order = ef.act_order_dev(H)
    U, _ = ef.factor_dev(H, order)
    (raw, _), = ef.ef_encode_dev([{"ttype": "Q3_K", "x": W, "qw": qw, "U": U, "order": order}])
    _check_slice(ef, W, "Q3_K", qw, H, U, order, raw, slice(1000, 1064))


def test_llama3_8b_down_q4k(mods):
    ef, hs, wl = mods
    n, nrow, N = 14336, 4096, 131072
    _say("config: Llama-3-8B ffn_down 4096 x 14336, Q4_K, H 14336^2 from 131072 rows")
    H = hs.xtx_accumulate(_activations(N, n, seed=5, outlier_frac=0.005, gain=50.0))
    order = ef.act_order_dev(H)
    U64, used = ef.factor_dev(H, order, out_dtype=torch.float64)
    assert used == [0.01]
    # U^T U (Hp + lambda I) = I, probed with random vectors in float64 on the device
    o = order.long()
    Hp = H.double()[o][:, o]
    lam = 0.01 * float(torch.diagonal(Hp).mean()) + 1e-8
    v = torch.randn((n, 4), device="cuda", dtype=torch.float64)
    r = U64.T @ (U64 @ (Hp @ v + lam * v))
    assert float((r - v).abs().max() / v.abs().max()) < 1e-6
    del Hp
    U = U64.float()
    del U64
    g = torch.Generator(device="cuda").manual_seed(2)
    W = torch.randn((nrow, n), generator=g, device="cuda") * 0.02
    qw = (torch.diagonal(H) / N).contiguous()
    (raw, rec), = ef.ef_encode_dev([{"ttype": "Q4_K", "x": W, "qw": qw, "U": U, "order": order}])
    assert raw.shape == (nrow, 56 * 144) and torch.isfinite(rec).all()
    _check_slice(ef, W, "Q4_K", qw, H, U, order, raw, slice(4090, 4096))


def test_llama3_8b_layer_other_tensors_q4k(mods):
    """The rest of the Llama-3-8B layer (config 4): q 4096 x 4096, k / v 1024 x 4096,
    o 4096 x 4096, gate / up 14336 x 4096 under Q4_K EF in one batched call, each input
    space's H (4096^2) from 131072 rows with 0.5 % outlier channels x50; row slices at the
    start, middle and end of every tensor equal the oracle's encode of those rows with the
    GPU's factor and order."""
    ef, hs, wl = mods
    N, n = 131072, 4096
    _say("config: Llama-3-8B q/k/v/o/gate/up, Q4_K, H 4096^2 from 131072 rows")
    fams = {}
    for i, fam in enumerate(("qkv_in", "o_in", "gateup_in")):
        fams[fam] = hs.xtx_accumulate(_activations(N, n, seed=20 + i, outlier_frac=0.005,
                                                   gain=50.0))
    Hb = torch.stack([fams[f] for f in ("qkv_in", "o_in", "gateup_in")])
    order = ef.act_order_dev(Hb)
    U, used = ef.factor_dev(Hb, order)
    assert used == [0.01] * 3
    slot = {"qkv_in": 0, "o_in": 1, "gateup_in": 2}
    g = torch.Generator(device="cuda").manual_seed(4)
    items, shapes = [], []
    for name, rows, nn_, fam in wl.LLAMA3_8B_LAYER:
        if fam == "down_in":
            continue
        W = torch.randn((rows, nn_), generator=g, device="cuda") * 0.02
        i = slot[fam]
        qw = (torch.diagonal(Hb[i]) / N).contiguous()
        items.append({"ttype": "Q4_K", "x": W, "qw": qw, "U": U[i], "order": order[i]})
        shapes.append((name, rows))
    outs = ef.ef_encode_dev(items)
    for (name, rows), it, (raw, rec) in zip(shapes, items, outs):
        assert raw.shape == (rows, 16 * 144) and torch.isfinite(rec).all()
        sel = np.r_[0:2, rows // 2:rows // 2 + 2, rows - 2:rows]
        _say(f"  {name}: rows {sel.tolist()}")
        _check_slice(ef, it["x"], "Q4_K", it["qw"], None, it["U"], it["order"], raw, sel)
