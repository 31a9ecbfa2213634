"""Parity of the EF call the headline bench times: the Qwen3-0.6B-shaped 28-layer set
(196 Q2_K tensors, three Hessian size classes on concurrent streams, built by
bench.build_workload / hessian_phase / ef_phase exactly as the timed step is).

The d = 1024 class holds 140 tensors, so its sweep task table (44 tasks per store)
and its tensor descriptor table (24 per store) reach the device in several chunks;
the d = 2048 and d = 3072 classes hold 28 each. For tensors at both ends of every
chunk, row slices from the start, the middle and the end of the tensor are compared
byte for byte with the oracle (coldpress/ef.py:179-218 restated) run on those rows
with the GPU's own factor, order and importance vector: EF rows are independent, so
the slice's bytes must equal the GPU's rows of the full call."""
import numpy as np
import pytest
import torch

from oracle import ef_oracle as E

pytestmark = pytest.mark.gpu
F32 = np.float32


def _say(msg):
    print(msg, flush=True)


def _chunk_ends(count, *sizes):
    idx = {0, count - 1}
    for size in sizes:
        for c0 in range(0, count, size):
            idx |= {c0, min(c0 + size, count) - 1}
    return sorted(idx)


@pytest.fixture(scope="module")
def bench_run():
    import bench
    from perm_amd import workloads as wl
    layers = wl.QWEN3_06B_LAYERS
    _say(f"bench parity: building the {layers}-layer workload")
    X, W, H, slot = bench.build_workload(layers, "cuda")
    bench.hessian_phase(X, H, slot)
    del X
    torch.cuda.synchronize()
    keep = {}
    _say("bench parity: EF of the 196 tensors (three concurrent size classes)")
    outs = bench.ef_phase(W, H, slot, layers, "exact", keep=keep)
    torch.cuda.synchronize()
    # the items of each class in the order ef_phase builds them
    classes = {}
    for d in sorted(H, reverse=True):
        members = []
        for l in range(layers):
            for name, _rows, _n, fam in wl.QWEN3_06B_LAYER:
                dd, i = slot[(l, fam)]
                if dd == d:
                    members.append((l, name, i))
        classes[d] = members
    res = {d: (classes[d], out) for d, out in zip(sorted(H, reverse=True), outs)}
    return W, keep, res


@pytest.mark.parametrize("d", [1024, 2048, 3072])
def test_bench_call_rows_match_oracle(bench_run, d):
    W, keep, res = bench_run
    members, out = res[d]
    assert len(out) == len(members) == {1024: 140, 2048: 28, 3072: 28}[d]
    U, order, qw = keep[d]
    for k in _chunk_ends(len(members), 44, 24):
        l, name, i = members[k]
        w = W[l][name]
        nrow, n = w.shape
        rows = np.r_[0:4, nrow // 2 - 2:nrow // 2 + 2, nrow - 4:nrow]
        _say(f"bench parity: class {d}, item {k} (layer {l} {name} [{nrow}, {n}]), rows {rows.tolist()}")
        Ui = U[i].cpu().numpy()
        oi = order[i].cpu().numpy().astype(np.int64)
        qi = qw[i].cpu().numpy()
        x = w.cpu().numpy()[rows]
        want_raw, want_rec = E.ef_encode(x, "Q2_K", qi, None, n_iter=2, U=Ui, order=oi)
        raw, rec = out[k]
        assert np.array_equal(raw.cpu().numpy()[rows], want_raw), (d, k)
        assert np.array_equal(rec.cpu().numpy()[rows], want_rec), (d, k)
