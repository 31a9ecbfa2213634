"""Index arguments are checked on the host before anything reaches the GPU.

The reference's moves are numpy fancy indexing (H[np.ix_(p, p)] at ef.py:289-290,
x[:, perm]), which raise IndexError for an entry out of range; its act order is
always a permutation (np.argsort). Every host wrapper that hands an index array to
a kernel checks it first, so these tests run on the CPU: a CPU tensor or a numpy
array is rejected before the library is even loaded."""
import numpy as np
import pytest
import torch

from perm_amd import _lib


def test_check_index_ranges_and_negative_entries():
    a = _lib.check_index(np.array([0, -1, 3, -4]), 4)
    assert a.dtype == np.int32 and a.tolist() == [0, 3, 3, 0]
    with pytest.raises(IndexError, match="out of bounds"):
        _lib.check_index(np.array([0, 4]), 4)
    with pytest.raises(IndexError, match="out of bounds"):
        _lib.check_index([0, -5], 4)
    with pytest.raises(IndexError):
        _lib.check_index(np.array([0.5, 1.0]), 4)
    # the same rules for torch tensors (CPU here; CUDA tensors take device reductions)
    t = _lib.check_index(torch.tensor([2, -1, 0]), 3)
    assert t.dtype == torch.int32 and t.tolist() == [2, 2, 0]
    with pytest.raises(IndexError):
        _lib.check_index(torch.tensor([3]), 3)
    # non-integer index tensors are refused, as the numpy branch refuses them, not truncated
    for bad in (torch.tensor([0.7, 1.0]), torch.tensor([0, 1], dtype=torch.float16),
                torch.tensor([1 + 0j]), torch.tensor([True, False])):
        with pytest.raises(IndexError, match="integers"):
            _lib.check_index(bad, 4)
    with pytest.raises(IndexError, match="integers"):
        _lib.check_index(np.array([True, False]), 4)


def test_check_index_permutations():
    assert _lib.check_index(np.array([2, 0, 1]), 3, permutation=True).tolist() == [2, 0, 1]
    assert _lib.check_index(np.array([-1, 0, 1]), 3, permutation=True).tolist() == [2, 0, 1]
    with pytest.raises(IndexError, match="not a permutation"):
        _lib.check_index(np.array([0, 0, 1]), 3, permutation=True)
    with pytest.raises(IndexError, match="not a permutation"):
        _lib.check_index(np.array([0, 1]), 3, permutation=True)
    # batched orders: every row a permutation
    good = np.stack([np.arange(5), np.arange(5)[::-1]])
    assert _lib.check_index(good, 5, permutation=True).shape == (2, 5)
    bad = good.copy()
    bad[1, 0] = 0
    with pytest.raises(IndexError):
        _lib.check_index(bad, 5, permutation=True)
    with pytest.raises(IndexError):
        _lib.check_index(torch.from_numpy(bad), 5, permutation=True)


def test_gather_and_hessian_moves_reject_bad_indices():
    from perm_amd import perm
    H = torch.zeros(6, 6, dtype=torch.float64)  # never reaches a device
    with pytest.raises(IndexError):
        perm.permute_hessian(H, np.array([0, 1, 2, 3, 4, 6]))
    with pytest.raises(IndexError):
        perm.gather(H, None, np.array([0, 1, 2, 3, 4, -7]))
    with pytest.raises(ValueError):
        perm.gather(H, np.arange(5), None)


def test_input_perm_rejects_malformed_permutations():
    from perm_amd import perm
    dims = {"d_model": 8, "d_ffn": 16, "n_layers": 1, "n_heads": 2, "n_kv": 1, "head_dim": 4}
    perms = perm.identity_perms(dims)
    assert perm.input_perm("blk.0.attn_q.weight", perms, dims).tolist() == list(range(8))
    bad = dict(perms, res=np.array([0, 1, 2, 3, 4, 5, 6, 8]))
    with pytest.raises(IndexError):
        perm.input_perm("blk.0.attn_q.weight", bad, dims)
    with pytest.raises(IndexError):
        perm.input_perm("token_embd.weight", bad, dims)
    dup = dict(perms, ffn=[np.r_[np.arange(15), 0]])
    with pytest.raises(IndexError):
        perm.input_perm("blk.0.ffn_down.weight", dup, dims)
    vo = dict(perms, vo=[[np.array([0, 1, 2, 2])]])
    with pytest.raises(IndexError):
        perm.input_perm("blk.0.attn_output.weight", vo, dims)
    with pytest.raises(ValueError):
        perm.input_perm("blk.0.attn_q.weight", dict(perms, res=np.arange(7)), dims)


def test_factor_and_ef_reject_orders_that_are_not_permutations():
    from perm_amd import ef
    H = torch.eye(4, dtype=torch.float64)
    with pytest.raises(IndexError):
        ef.factor_dev(H, np.array([0, 1, 2, 4]))
    with pytest.raises(IndexError):
        ef.factor_dev_async(H, np.array([0, 1, 1, 2]))
    with pytest.raises(IndexError):
        ef.factor_dev(torch.stack([H, H]), np.array([[0, 1, 2, 3], [3, 2, 1, 1]]))
    with pytest.raises(ValueError):
        ef.factor_dev(H, np.arange(3))
    item = {"ttype": "Q2_K", "x": torch.zeros(2, 256), "qw": None,
            "U": torch.zeros(256, 256), "order": np.r_[np.arange(255), 256]}
    with pytest.raises(IndexError):
        ef.ef_encode_dev([item])
