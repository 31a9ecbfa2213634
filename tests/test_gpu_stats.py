"""The encode driver's err-vs-stock statistic on the GPU (cp_sq_err_sum): the float32
value of (((recon - x) ** 2) * w).sum() (coldpress/ef.py:299-300) bit for bit against
numpy's own sum of the same arrays, through totals under one 8192-term chunk, partial last
chunks, rows narrower than a 128-term leaf, the tied-output matrix's size and no rows."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(1, 4), (3, 40), (5, 332), (3, 1000), (2, 4096), (7, 3072),
                                   (100, 256), (9, 8192), (2, 10000), (3, 24580), (1024, 3072),
                                   (151936, 1024), (0, 256)])
def test_sq_err_sum_equals_numpy(shape):
    from perm_amd import ef
    print(f"sq err {shape}", flush=True)
    rng = np.random.default_rng(shape[0] + 31 * shape[1])
    x = (rng.standard_normal(shape, dtype=np.float32) ** 3).astype(np.float32)
    r = (x + rng.standard_normal(shape, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    w = np.abs(rng.standard_normal(shape[1], dtype=np.float32)) + np.float32(0.1)
    xd, rd, wd = (torch.from_numpy(a).cuda() for a in (x, r, w))
    for ww, wwd in ((w, wd), (np.ones(shape[1], np.float32), None)):
        want = (((r - x) ** 2) * ww).sum()
        got = ef.sq_err_sum_dev(rd, xd, wwd).cpu().numpy()
        assert got.tobytes() == want.tobytes(), (shape, got, want)
