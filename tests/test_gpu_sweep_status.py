"""The multi-wave EF sweep's bounded wait reports a give-up instead of failing silently.

A wave of a multi-wave stripe waits (bounded) for the earlier blocks of its stripe. The
spin bound is forced to 0 from the host (cp_ef_wait_limit), so waves give up at once; every
kernel still ends normally. The call's status word must then say so, through the C ABI
(cp_ef_read_status) and the host drivers (SweepTimeout), and a normal bound must give a
clean status and the oracle's bytes again."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import correlated_hessian, heavy_tailed
from oracle import ef_oracle as E

pytestmark = pytest.mark.gpu
F32 = np.float32


def _item(nrow=96, n=1024, seed=3):
    W = heavy_tailed(nrow, n, seed=seed)
    H = correlated_hessian(n, 2048, seed=seed + 1)
    qw = (np.diag(H) / 2048).astype(F32)
    order = E.act_order(H, stable=True)
    U = E.inv_upper_factor(H[np.ix_(order, order)], 0.01).astype(F32)
    item = {"ttype": "Q2_K", "x": torch.from_numpy(W).cuda(), "qw": torch.from_numpy(qw).cuda(),
            "U": torch.from_numpy(U).cuda(), "order": torch.from_numpy(order.astype(np.int32)).cuda()}
    return item, (W, qw, H, order, U)


def test_give_up_is_reported(monkeypatch):
    from perm_amd import _lib
    from perm_amd import ef
    lib = _lib.load()
    monkeypatch.setenv("CP_EF_SWEEP_WAVES", "8")  # 96 x 1024: 8 waves per 16-row stripe
    item, (W, qw, H, order, U) = _item()
    print("status: wait bound 0, 8 waves per stripe", flush=True)
    lib.cp_ef_wait_limit(0)
    try:
        words = []
        ef.ef_encode_dev([item], 2, status=words)
        torch.cuda.synchronize()
        rs, wv = (ctypes.c_int * 1)(), (ctypes.c_int * 1)()
        lib.cp_ef_last_sweep(ctypes.cast(rs, ctypes.c_void_p), ctypes.cast(wv, ctypes.c_void_p))
        assert wv[0] == 8
        assert int(words[0].item()) & 1
        assert ef.status_failed(words)
        with pytest.raises(_lib.SweepTimeout):
            ef.check_status(words)
        # the default path reads the word through the C ABI (cp_ef_read_status)
        with pytest.raises(_lib.SweepTimeout, match="gave up"):
            ef.ef_encode_dev([item], 2)
        # the batched driver reads it with the factorization flags
        Hd = torch.from_numpy(H).cuda()
        with pytest.raises(_lib.SweepTimeout):
            ef.ef_encode_many([{"name": "t", "ttype": "Q2_K", "x": item["x"], "qw": item["qw"],
                                "H": Hd}])
    finally:
        lib.cp_ef_wait_limit(-1)
    print("status: default bound", flush=True)
    words = []
    (raw, rec), = ef.ef_encode_dev([item], 2, status=words)
    assert not ef.status_failed(words)
    want_raw, want_rec = E.ef_encode(W, "Q2_K", qw, H, n_iter=2, U=U, order=order)
    assert np.array_equal(raw.cpu().numpy(), want_raw)
    assert np.array_equal(rec.cpu().numpy(), want_rec)


def test_read_status_through_the_c_abi():
    """cp_ef_read_status on a clean call's workspace returns CP_OK; on a workspace whose
    word has the give-up bit, CP_ERR_TIMEOUT with a message."""
    from perm_amd import _lib
    lib = _lib.load()
    ws = torch.zeros(256, dtype=torch.uint8, device="cuda")
    assert lib.cp_ef_read_status(_lib.ptr(ws), _lib.stream_ptr()) == _lib.CP_OK
    ws[:4].view(torch.int32).fill_(1)
    assert lib.cp_ef_read_status(_lib.ptr(ws), _lib.stream_ptr()) == _lib.CP_ERR_TIMEOUT
    assert b"gave up" in lib.cp_last_error()
