"""cp_ef_encode_noalloc (the EF encode without a caller workspace or any device
allocation, for callers that cannot allocate) against cp_ef_encode with a caller
workspace: byte-identical container bytes and reconstructions, on two calls in a row,
the second with a smaller tensor of another type (the static workspace keeps the
first call's contents), and a clear error for a tensor beyond its size."""
import numpy as np
import pytest
import torch

from conftest import correlated_hessian, heavy_tailed

pytestmark = pytest.mark.gpu
F32 = np.float32


def _say(msg):
    print(msg, flush=True)


def _case(nrow, n, tt, seed):
    from perm_amd import ef as gef
    W = torch.from_numpy(heavy_tailed(nrow, n, seed=seed)).cuda()
    H = torch.from_numpy(correlated_hessian(n, 2 * n, seed=seed + 1)).cuda()
    qw = (torch.diagonal(H) / (2 * n)).float().contiguous()
    order = gef.act_order_dev(H)
    U, _ = gef.factor_dev(H, order, 0.01, checked=True)
    return W, qw, U, order


def _encode(lib, _lib, tt, W, qw, U, order, noalloc):
    from perm_amd.kquant import BYTES_PER_SB
    nrow, n = W.shape
    raw = torch.full((nrow, n // 256 * BYTES_PER_SB[tt]), 0xA5, dtype=torch.uint8, device="cuda")
    rec = torch.full((nrow, n), float("nan"), device="cuda")
    args = (_lib.TTYPE[tt], _lib.ptr(W), nrow, n, _lib.ptr(qw), _lib.ptr(U), _lib.ptr(order), 2,
            _lib.ptr(raw), _lib.ptr(rec))
    if noalloc:
        st = lib.cp_ef_encode_noalloc(*args, _lib.stream_ptr())
    else:
        t = _lib.EfTensor(_lib.TTYPE[tt], nrow, n, W.data_ptr(), qw.data_ptr(), U.data_ptr(),
                          order.data_ptr(), raw.data_ptr(), rec.data_ptr())
        ws = _lib.workspace(lib.cp_ef_ws_bytes(ctypes_array(_lib, t), 1))
        st = lib.cp_ef_encode(*args, _lib.ptr(ws), ws.numel(), _lib.stream_ptr())
    _lib.check(st)
    torch.cuda.synchronize()
    return raw, rec


def ctypes_array(_lib, t):
    return (_lib.EfTensor * 1)(t)


def test_noalloc_matches_workspace_entry_twice():
    from perm_amd import _lib
    lib = _lib.load()
    assert lib.cp_ef_noalloc_max_ws_bytes() == 64 << 20
    for nrow, n, tt, seed in [(1024, 3072, "Q2_K", 3), (96, 512, "Q4_K", 7)]:
        _say(f"noalloc: {tt} [{nrow}, {n}]")
        W, qw, U, order = _case(nrow, n, tt, seed)
        want = _encode(lib, _lib, tt, W, qw, U, order, noalloc=False)
        got = _encode(lib, _lib, tt, W, qw, U, order, noalloc=True)
        # the static workspace's status word: no sweep wave gave up
        assert lib.cp_ef_read_status(None, _lib.stream_ptr()) == _lib.CP_OK
        assert torch.equal(got[0], want[0]), (tt, nrow, n)
        assert torch.equal(got[1], want[1]), (tt, nrow, n)


def test_noalloc_rejects_a_tensor_beyond_its_workspace():
    from perm_amd import _lib
    lib = _lib.load()
    nrow, n = 4096, 1024  # about 73 MB of EF workspace
    t = _lib.EfTensor(_lib.TTYPE["Q2_K"], nrow, n, None, None, None, None, None, None)
    assert lib.cp_ef_ws_bytes((_lib.EfTensor * 1)(t), 1) > lib.cp_ef_noalloc_max_ws_bytes()
    W = torch.zeros(nrow, n, device="cuda")
    U = torch.zeros(n, n, device="cuda")
    order = torch.arange(n, dtype=torch.int32, device="cuda")
    raw = torch.zeros(nrow, n // 256 * 84, dtype=torch.uint8, device="cuda")
    st = lib.cp_ef_encode_noalloc(_lib.TTYPE["Q2_K"], _lib.ptr(W), nrow, n, None, _lib.ptr(U),
                                  _lib.ptr(order), 2, _lib.ptr(raw), None, _lib.stream_ptr())
    assert st == _lib.CP_ERR_WORKSPACE
    assert b"allocation-free" in lib.cp_last_error()
