"""GPU X^T X accumulation against the float64 closed form (1e-5 relative
Frobenius), for bf16 and float32 activations, ragged shapes and beta = 1."""
import numpy as np
import pytest
import torch

from oracle import hess_oracle as Ho

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hs():
    from perm_amd import hessians
    return hessians


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,d", [(4096, 1024), (1000, 200), (33, 136), (70000, 256), (12345, 1032)])
def test_xtx_matches_closed_form(hs, dtype, N, d):
    print(f"xtx {dtype} N={N} d={d}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(N + d)
    X = (torch.randn((N, d), generator=g, device="cuda") *
         torch.exp(torch.randn((d,), generator=g, device="cuda"))).to(dtype)
    H = hs.xtx_accumulate(X)
    ref = Ho.xtx(X.float().cpu().numpy())
    assert Ho.rel_fro(H.cpu().numpy(), ref) < 1e-5
    assert torch.allclose(H, H.T, rtol=1e-4, atol=1e-5 * float(H.abs().max()))


def test_accumulates_in_place(hs):
    g = torch.Generator(device="cuda").manual_seed(0)
    X1 = torch.randn((3000, 512), generator=g, device="cuda").to(torch.bfloat16)
    X2 = torch.randn((5000, 512), generator=g, device="cuda").to(torch.bfloat16)
    acc = hs.HessianAccumulator(512)
    acc.add(X1).add(X2.reshape(10, 500, 512))
    ref, cnt = Ho.accumulate([X1.float().cpu().numpy(), X2.float().cpu().numpy()])
    assert acc.n == cnt == 8000
    assert Ho.rel_fro(acc.H.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_zero_row_batch_adds_nothing(hs, dtype):
    """A batch with no rows leaves H as it was, as the reference's x.T @ x of an empty
    batch adds zeros (hessians.py:137-154); alone and inside a batched call."""
    g = torch.Generator(device="cuda").manual_seed(1)
    H = torch.randn((256, 256), generator=g, device="cuda")
    before = H.clone()
    hs.xtx_accumulate(torch.zeros((0, 256), device="cuda", dtype=dtype), H)
    assert torch.equal(H, before)
    hs.xtx_accumulate_many([torch.zeros((0, 256), device="cuda", dtype=dtype)] * 2, [H, H.clone()])
    assert torch.equal(H, before)
    assert torch.equal(hs.xtx_accumulate(torch.zeros((2, 0, 128), device="cuda", dtype=dtype)),
                       torch.zeros((128, 128), device="cuda"))


def test_collect_hessians_hooks(hs):
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.GELU(),
                                torch.nn.Linear(512, 256)).cuda().to(torch.bfloat16)
    batches = [torch.randn((4, 64, 256), device="cuda", dtype=torch.bfloat16) for _ in range(3)]
    res, unmapped = hs.collect_hessians(model, batches, {"0": "blk.0.ffn_up.weight",
                                                         "2": "blk.0.ffn_down.weight"})
    assert unmapped == [] and set(res) == {"blk.0.ffn_up.weight", "blk.0.ffn_down.weight"}
    assert res["blk.0.ffn_up.weight"]["n"] == 3 * 4 * 64
    X0 = torch.cat([b.reshape(-1, 256) for b in batches]).float().cpu().numpy()
    assert Ho.rel_fro(res["blk.0.ffn_up.weight"]["H"].cpu().numpy(), Ho.xtx(X0)) < 1e-5
    with pytest.raises(ValueError, match="different"):
        hs.collect_hessians(model, batches, {"0": "x.weight"}, gguf_ne0={"x.weight": 128})


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_batched_accumulation(hs, dtype):
    """Many (X, H) jobs in one call, mixed shapes (grouped per shape), with H accumulated
    in place: every H within 1e-5 of its own closed form, and more jobs of one shape than
    one launch carries (224)."""
    g = torch.Generator(device="cuda").manual_seed(7)
    shapes = [(2048, 1024)] * 3 + [(999, 256)] * 2 + [(4096, 520)] + [(64, 136)] * 230
    Xs, Hs, base = [], [], []
    for k, (N, d) in enumerate(shapes):
        Xs.append((torch.randn((N, d), generator=g, device="cuda") *
                   torch.exp(torch.randn((d,), generator=g, device="cuda"))).to(dtype))
        H0 = torch.randn((d, d), generator=g, device="cuda")
        H0 = H0 @ H0.T
        base.append(H0.cpu().numpy().astype(np.float64))
        Hs.append(H0.contiguous())
    print(f"batched {dtype}: {len(shapes)} jobs", flush=True)
    hs.xtx_accumulate_many(Xs, Hs)
    for k in list(range(7)) + [100, 235]:
        ref = base[k] + Ho.xtx(Xs[k].float().cpu().numpy())
        assert Ho.rel_fro(Hs[k].cpu().numpy(), ref) < 1e-5, k
