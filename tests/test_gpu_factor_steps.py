"""The fused chain step of the factorization (one launch per 64 columns, for calls of at
most four matrices on a GPU the factorization has to itself).

Its tiles run the same block code, with the same arguments, as the separate inner-update,
diagonal-block and panel launches that larger batches (and factorizations queued beside EF
work) take, so U must be the same bit for bit on either path. Its panel tiles wait
(bounded) for their diagonal block; the bound is forced to 0 from the host
(cp_chol_wait_limit), so the waits give up at once while every kernel still ends, and the
call must then fail loudly (FactorTimeout, flag bit 2 of the asynchronous form)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _hessians(n, batch, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    X = torch.randn(batch, n + 256, n, device="cuda", generator=g)
    X[:, :, : max(1, n // 100)] *= 20.0
    return (X.transpose(1, 2) @ X).contiguous()


@pytest.mark.parametrize("n", [64, 100, 1000, 3072])
def test_fused_steps_give_the_separate_launches_factor(n):
    from perm_amd import _lib
    from perm_amd import ef
    print(f"fused steps n={n}", flush=True)
    lib = _lib.load()
    H = _hessians(n, 5, seed=n)
    U5, _ = ef.factor_dev(H, None, 0.01, out_dtype=torch.float64)        # separate launches
    U4, _ = ef.factor_dev(H[:4].contiguous(), None, 0.01, out_dtype=torch.float64)  # fused
    U1, _ = ef.factor_dev(H[:1].contiguous(), None, 0.01, out_dtype=torch.float64)
    assert torch.equal(U4, U5[:4]) and torch.equal(U1[0], U5[0])
    lib.cp_chol_compact_tiles(1)  # beside EF work: the separate launches at batch 1 too
    try:
        U1c, _ = ef.factor_dev(H[:1].contiguous(), None, 0.01, out_dtype=torch.float64)
    finally:
        lib.cp_chol_compact_tiles(0)
    assert torch.equal(U1c, U1)
    Hd = H[0].double()
    Hd = Hd + (0.01 * Hd.diagonal().mean() + 1e-8) * torch.eye(n, device="cuda", dtype=torch.float64)
    U = U1[0]
    assert (U.T @ U @ Hd - torch.eye(n, device="cuda", dtype=torch.float64)).abs().max().item() < 1e-8


def test_fused_step_give_up_is_reported():
    from perm_amd import _lib
    from perm_amd import ef
    lib = _lib.load()
    H = _hessians(1024, 2, seed=7)
    print("fused steps: wait bound 0", flush=True)
    lib.cp_chol_wait_limit(0)
    try:
        with pytest.raises(_lib.FactorTimeout, match="gave up"):
            ef.factor_dev(H, None, 0.01)
        _, flags = ef.factor_dev_async(H, None, 0.01)
        assert np.any(flags.cpu().numpy() & 4)
    finally:
        lib.cp_chol_wait_limit(-1)
    print("fused steps: default bound", flush=True)
    U, used = ef.factor_dev(H, None, 0.01, out_dtype=torch.float64)
    _, flags = ef.factor_dev_async(H, None, 0.01)
    assert used == [0.01, 0.01] and not np.any(flags.cpu().numpy())
    U5, _ = ef.factor_dev(torch.cat([H, H, H[:1]]).contiguous(), None, 0.01,
                          out_dtype=torch.float64)
    assert torch.equal(U, U5[:2])
