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
    ne0 = {"blk.0.ffn_up.weight": 256, "blk.0.ffn_down.weight": 512}
    res, unmapped = hs.collect_hessians(model, batches, ne0, "qwen3", 1,
                                        name_map={"0": "blk.0.ffn_up", "2": "blk.0.ffn_down"},
                                        log=lambda *_: None)
    assert unmapped == [] and set(res) == {"blk.0.ffn_up.weight", "blk.0.ffn_down.weight"}
    assert res["blk.0.ffn_up.weight"]["n"] == 3 * 4 * 64
    assert isinstance(res["blk.0.ffn_up.weight"]["H"], np.ndarray)
    X0 = torch.cat([b.reshape(-1, 256) for b in batches]).float().cpu().numpy()
    assert Ho.rel_fro(res["blk.0.ffn_up.weight"]["H"], Ho.xtx(X0)) < 1e-5
    with pytest.raises(ValueError, match=r"ne\[0\]|mis-key|MISMATCH"):
        hs.collect_hessians(model, batches, {"x.weight": 128}, "qwen3", 1, name_map={"0": "x"},
                            log=lambda *_: None)


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


def test_collect_hessians_on_a_hf_decoder(hs):
    """The drop-in collector on a tiny Qwen3 decoder (coldpress/hessians.py:85-179 with the
    reference test's expectations, test_hessians.py:22-33): every linear keyed by its GGUF
    name through the built-in map, H equal to X^T X of the inputs the module saw (float64
    closed form of the same inputs, captured by plain hooks), q/k/v and gate/up holding
    equal but separate host arrays (one accumulator on the device), and the layer shards
    [0, 1) (with output) and [1, 2) splitting the set."""
    from conftest import tiny_hf_decoder
    model = tiny_hf_decoder("qwen3").cuda()
    names = hs.build_name_map(model, "qwen3", 2)
    linears = {n: m for n, m in model.named_modules() if isinstance(m, torch.nn.Linear)}
    ne0 = {names[n] + ".weight": m.in_features for n, m in linears.items()}
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    batches = [torch.randint(0, 128, (32,), device="cuda", generator=g) for _ in range(3)]
    seen = {n: [] for n in linears}
    hooks = [m.register_forward_hook(
        lambda mod, inp, out, n=n: seen[n].append(inp[0].reshape(-1, inp[0].shape[-1]).double().cpu()))
        for n, m in linears.items()]
    with torch.no_grad():
        for ids in batches:
            model(ids.unsqueeze(0))
    for h in hooks:
        h.remove()
    full, unmapped = hs.collect_hessians(model, batches, ne0, "qwen3", 2, log=lambda *_: None)
    # the embedding maps to token_embd, which this ne0 leaves out: unmapped, as the
    # reference's planner (which also walks nn.Embedding) reports it
    assert unmapped == ["model.embed_tokens (-> token_embd.weight, not in the GGUF)"]
    assert set(full) == set(ne0)
    for n in linears:
        gname = names[n] + ".weight"
        X = torch.cat(seen[n]).numpy()
        assert full[gname]["n"] == X.shape[0] == 96
        assert Ho.rel_fro(full[gname]["H"], X.T @ X) < 1e-5, gname
    for l in (0, 1):
        for a, b in ((f"blk.{l}.attn_q.weight", f"blk.{l}.attn_v.weight"),
                     (f"blk.{l}.ffn_gate.weight", f"blk.{l}.ffn_up.weight")):
            assert np.array_equal(full[a]["H"], full[b]["H"])
            assert not np.shares_memory(full[a]["H"], full[b]["H"])
    dev, _ = hs.collect_hessians(model, batches, ne0, "qwen3", 2, log=lambda *_: None,
                                 keep_on_device=True)
    assert dev["blk.0.attn_q.weight"]["H"] is dev["blk.0.attn_k.weight"]["H"]
    assert torch.equal(dev["blk.1.ffn_down.weight"]["H"].cpu(),
                       torch.from_numpy(full["blk.1.ffn_down.weight"]["H"]))
    lo, _ = hs.collect_hessians(model, batches, ne0, "qwen3", 2, layer_lo=0, layer_hi=1,
                                log=lambda *_: None)
    hi, _ = hs.collect_hessians(model, batches, ne0, "qwen3", 2, layer_lo=1, layer_hi=2,
                                log=lambda *_: None)
    assert set(lo) == {k for k in ne0 if not k.startswith("blk.1.")}
    assert set(hi) == {k for k in ne0 if k.startswith("blk.1.")}
    for k in ne0:
        part = lo if k in lo else hi
        assert Ho.rel_fro(part[k]["H"], full[k]["H"]) < 1e-6


def _rows_fp64(X, J, chunk=16384):
    """Rows J of X^T X in float64 on the device, summed over row chunks: [len(J), d]."""
    out = torch.zeros((len(J), X.shape[1]), dtype=torch.float64, device=X.device)
    for r0 in range(0, X.shape[0], chunk):
        Xc = X[r0:r0 + chunk].double()
        out += torch.mm(Xc[:, J].T.contiguous(), Xc)
    return out


@pytest.mark.parametrize("kind,N,d,jobs", [("student-t", 65536, 2048, 1), ("student-t", 65536, 3072, 2),
                                           ("outliers", 131072, 4096, 1),
                                           ("outliers", 131072, 14336, 1)])
def test_gate_at_config_sizes(hs, kind, N, d, jobs):
    """The 1e-5 relative Frobenius gate (hessians.py:147 forms x.T @ x in float32) at the
    benchmark configurations' Hessian sizes: Student-t bf16 rows for the Qwen3-0.6B o_in /
    down_in spaces, log-normal rows with 0.5 % of channels x50 for the Llama-3-8B spaces.
    Sampled rows of H (the 16 largest diagonal entries, which take in the x50 channels, and
    48 random ones) against float64 sums of the same bf16 rows; H symmetric bit for bit; a
    second accumulation of the same X equal bit for bit."""
    from perm_amd import workloads as wl
    print(f"gate {kind} N={N} d={d} jobs={jobs}", flush=True)
    Xs = [wl.family_activations(kind, N, d, seed=11 + k) for k in range(jobs)]
    Hs = [torch.zeros((d, d), device="cuda") for _ in range(jobs)]
    hs.xtx_accumulate_many(Xs, Hs)
    again = [torch.zeros((d, d), device="cuda") for _ in range(jobs)]
    hs.xtx_accumulate_many(Xs, again)
    g = torch.Generator(device="cpu").manual_seed(d)
    for X, H, H2 in zip(Xs, Hs, again):
        assert torch.equal(H, H2)
        assert torch.equal(H, H.T)
        top = torch.topk(torch.diagonal(H), 16).indices.cpu()
        rest = torch.randperm(d, generator=g)[:64]
        J = torch.unique(torch.cat([top, rest[~torch.isin(rest, top)][:48]])).cuda()
        ref = _rows_fp64(X, J)
        err = float(torch.linalg.norm(H[J].double() - ref) / torch.linalg.norm(ref))
        print(f"  rel err {err:.2e} over {len(J)} rows", flush=True)
        assert err < 1e-5


@pytest.mark.parametrize("dtype,N,d,jobs", [(torch.bfloat16, 65536, 1024, 56),
                                            (torch.bfloat16, 12345, 1032, 3),
                                            (torch.float32, 8192, 1024, 1),
                                            (torch.float32, 70000, 256, 2)])
def test_same_x_same_h(hs, dtype, N, d, jobs):
    """Two accumulations of the same X into the same starting H give the same H bit for bit,
    both through the batched call (the benchmark's 56-job d = 1024 class, five row splits)
    and through single calls, for plans with one and with several row splits; and each
    job's H is within 1e-5 of the float64 closed form."""
    print(f"repro {dtype} N={N} d={d} jobs={jobs}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(N + d + jobs)
    Xs = [(torch.randn((N, d), generator=gen, device="cuda") *
           torch.exp(torch.randn((d,), generator=gen, device="cuda"))).to(dtype) for _ in range(jobs)]
    H0 = torch.randn((d, d), generator=gen, device="cuda")
    H0 = H0 + H0.T
    runs = []
    for _ in range(2):
        Hs = [H0.clone() for _ in range(jobs)]
        hs.xtx_accumulate_many(Xs, Hs)
        runs.append(Hs)
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    one = [hs.xtx_accumulate(Xs[0], H0.clone()) for _ in range(2)]
    assert torch.equal(one[0], one[1])
    for k in sorted({0, jobs - 1}):
        ref = H0.double() + _rows_fp64(Xs[k].float(), torch.arange(d, device="cuda"))
        err = float(torch.linalg.norm(runs[0][k].double() - ref) / torch.linalg.norm(ref))
        assert err < 1e-5, (k, err)
