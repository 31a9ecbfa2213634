#!/usr/bin/env python3
"""EF k-quant encode (Q2_K) + Hessian X^T X throughput on one MI355X.

Workload (one step): the Qwen3-0.6B-shaped layer set, random-init, 28 decoder
layers x 7 linear tensors -- q 2048x1024, k/v 1024x1024, o 1024x2048,
gate/up 3072x1024, down 1024x3072: 440,401,920 weights.
  1. Hessians: per layer the 4 distinct input Hessians (qkv_in d=1024,
     o_in 2048, gateup_in 1024, down_in 3072), each H = X^T X over 65536
     synthetic bf16 activation rows (Student-t nu=4, per-channel log-normal
     scales), float32 accumulation on MFMA.
  2. EF encode: act order + damped fp64 inverse-Hessian factor per distinct H,
     then GPTQ error feedback (2 iterations) of all 196 tensors into Q2_K with
     qw = diag(H)/N (imatrix-style channel means), and the final decode.
Activations and weights are generated on the device before the timed region.

value = EF Mweights/s = 440.4e6 / (EF time per step); the Hessian TFLOP/s
(N*d*(d+1) per Hessian: the kernel computes the lower triangle) is reported beside it. cpu_baseline: the numpy oracle
(a port of the reference's ef.py / kquant.py) on a row subsample of one layer,
extrapolated to the full workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "EF k-quant encode Mweights/s (Q2_K) + Hessian X^T·X TFLOP/s, 1 GPU"
ROWS = 65536
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
# HBM bytes per ef_sweep_rows_kernel launch of the 28-layer exact-mode workload (mean of
# the sequential pass's six launches), from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs,
# each scaled by what the counter reads for a plain 1 GiB copy (`--workload copy`):
# FETCH_SIZE x 2.0, WRITE_SIZE x 1.0. Source: profiles/ef_sweep_rows_qwen3-0.6b_q2k_pmc.md.
SWEEP_TRAFFIC_BYTES = 10.594e9


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_workload(layers, device):
    import torch
    from perm_amd import workloads as wl
    X, W = [], []
    for l in range(layers):
        X.append({fam: wl.student_t_activations(ROWS, d, nu=4.0, seed=1000 * l + i, device=device)
                  for i, (fam, d) in enumerate(wl.QWEN3_06B_FAMILIES.items())})
        W.append(wl.qwen3_layer_weights(l, seed=0, device=device))
        if (l + 1) % 7 == 0 or l + 1 == layers:
            log(f"generated layer {l + 1}/{layers}")
    # Hessian accumulators, batched by matrix size (qkv_in and gateup_in share d=1024)
    H = {1024: torch.zeros((2 * layers, 1024, 1024), device=device),
         2048: torch.zeros((layers, 2048, 2048), device=device),
         3072: torch.zeros((layers, 3072, 3072), device=device)}
    slot = {}
    for l in range(layers):
        slot[(l, "qkv_in")] = (1024, l)
        slot[(l, "gateup_in")] = (1024, layers + l)
        slot[(l, "o_in")] = (2048, l)
        slot[(l, "down_in")] = (3072, l)
    torch.cuda.synchronize()
    return X, W, H, slot


def hessian_phase(X, H, slot):
    """Every layer's Hessians, one batched accumulation per matrix size."""
    from perm_amd.hessians import xtx_accumulate_many
    for Hb in H.values():
        Hb.zero_()
    xs, hs = [], []
    for l, fams in enumerate(X):
        for fam, Xf in fams.items():
            d, i = slot[(l, fam)]
            xs.append(Xf)
            hs.append(H[d][i])
    xtx_accumulate_many(xs, hs)


def ef_phase(W, H, slot, layers, mode, concurrent=True):
    """Act order + factor per Hessian size class, then EF of that class's tensors.
    With ``concurrent`` each size class runs on its own stream, so one class's
    factorization overlaps another's sweep (perm_amd.ef.encode_size_classes)."""
    from perm_amd import ef as gef
    from perm_amd import workloads as wl

    def builder(d):
        def build(U, order):
            # qw = diag(H) / N for every Hessian of the class in one kernel
            qw = (H[d].diagonal(dim1=1, dim2=2) / float(ROWS)).contiguous()
            items = []
            for l in range(layers):
                for name, _rows, _n, fam in wl.QWEN3_06B_LAYER:
                    dd, i = slot[(l, fam)]
                    if dd != d:
                        continue
                    items.append({"ttype": "Q2_K", "x": W[l][name], "qw": qw[i],
                                  "U": U[i], "order": order[i], "recon": True})
            return items
        return build

    classes = [(H[d], builder(d)) for d in sorted(H, reverse=True)]
    if concurrent:
        return gef.encode_size_classes(classes, n_iter=2, mode=mode, damp=0.01)
    outs = []
    for Hb, build in classes:
        order = gef.act_order_dev(Hb)
        U, _ = gef.factor_dev(Hb, order, 0.01)
        outs.append(gef.ef_encode_dev(build(U, order), n_iter=2, mode=mode))
    return outs


def cpu_baseline(W, H, slot, layers, total_weights):
    """Time the numpy oracle (port of coldpress/ef.py:46-218 + kquant.py) on
    128- and 512-row subsamples of layer 0's 7 tensors, with one factorization
    per tensor as the reference does (ef.py:189), and extrapolate:
    T(tensor) = T_factor + a + b * nrow, times 28 identical layers."""
    import numpy as np
    from oracle import ef_oracle as E
    from perm_amd import workloads as wl
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # threadpoolctl missing or unreadable
        blas_threads = 1
    t_total = 0.0
    t_spent = 0.0
    per = []
    for name, rows, n, fam in wl.QWEN3_06B_LAYER:
        d, i = slot[(0, fam)]
        Hn = H[d][i].double().cpu().numpy()
        qw = (np.diag(Hn) / ROWS).astype(np.float32)
        Wn = W[0][name].cpu().numpy()
        t0 = time.perf_counter()
        order = E.act_order(Hn)
        U = E.inv_upper_factor(Hn[np.ix_(order, order)], 0.01).astype(np.float32)
        t_fact = time.perf_counter() - t0
        ts = {}
        for r in (128, 512):
            t0 = time.perf_counter()
            E.ef_encode(Wn[:r], "Q2_K", qw, Hn, U=U)
            ts[r] = time.perf_counter() - t0
        b = (ts[512] - ts[128]) / 384.0
        a = ts[128] - 128 * b
        t_tensor = t_fact + a + b * rows
        per.append((name, t_fact, ts[128], ts[512], t_tensor))
        t_total += t_tensor
        t_spent += t_fact + ts[128] + ts[512]
        log(f"cpu {name}: factor {t_fact:.2f}s ef128 {ts[128]:.2f}s ef512 {ts[512]:.2f}s "
            f"-> full tensor {t_tensor:.1f}s")
    t_total *= layers
    return {
        "value": total_weights / t_total / 1e6,
        "unit": "Mweights/s",
        "cores": int(blas_threads),
        "kind": "port",
        "sample": (f"numpy oracle (port of ef.py/kquant.py) on layer 0's 7 tensors at 128 and 512 "
                   f"rows + one factorization per tensor ({t_spent:.1f} s of CPU work); "
                   f"extrapolated linearly in rows to all {layers} layers "
                   f"(est. {t_total:.0f} s for the full encode); sweep and codec are "
                   f"single-threaded numpy, the factorization uses {blas_threads} BLAS threads"),
        "host_cpus": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
    }


PERM_METRIC = "PERM container-objective search Mweights/s (Qwen3-0.6B space map), 1 GPU"


def perm_search_weights(dims, rows_sample, n_keys):
    """Weights the search round-trips through the codec: (1 + n_keys) residual
    evaluations over every residual-space tensor (the embedding at its row sample),
    then two ffn_down and two attn_output evaluations per layer."""
    from perm_amd import workloads as wl
    L, d = dims["n_layers"], dims["d_model"]
    res = min(rows_sample, wl.QWEN3_06B_VOCAB) * d + L * d * sum(
        r for name, r, _n, fam in wl.QWEN3_06B_LAYER if fam in ("qkv_in", "gateup_in"))
    return (1 + n_keys) * res + L * 2 * d * dims["d_ffn"] + \
        L * 2 * d * dims["n_heads"] * dims["head_dim"]


def perm_cpu_baseline(weights, ttypes, qws, rows_sample, n_keys, dims):
    """The numpy oracle's tensor_err (a port of objective.py + kquant.py) called as the
    search calls it on the embedding (its 16384-row sample) and on every tensor of
    layer 0 (residual-space tensors with a column permutation, ffn_down and
    attn_output whole), timed per class and extrapolated by round-tripped weights."""
    import numpy as np
    from oracle import perm_oracle as Po
    from perm_amd import workloads as wl
    L = dims["n_layers"]
    rng = np.random.default_rng(1)
    spent, total_t = 0.0, 0.0
    classes = [("token_embd.weight", 1 + n_keys, 1)]
    for name, _r, _n, fam in wl.QWEN3_06B_LAYER:
        classes.append((f"blk.0.{name}.weight",
                        (1 + n_keys) if fam in ("qkv_in", "gateup_in") else 2, L))
    for name, reps, layers in classes:
        x = weights[name].cpu().numpy()
        perm = rng.permutation(x.shape[1])
        t0 = time.perf_counter()
        Po.tensor_err(x, ttypes[name], qws.get(name), perm=perm,
                      rows_sample=rows_sample if name == "token_embd.weight" else None)
        dt = time.perf_counter() - t0
        spent += dt
        total_t += dt * reps * layers
        log(f"cpu {name} {ttypes[name]}: {dt:.2f}s")
    work = perm_search_weights(dims, rows_sample, n_keys)
    return {"value": work / total_t / 1e6, "unit": "Mweights/s", "cores": 1, "kind": "port",
            "sample": (f"numpy oracle tensor_err (port of objective.py / kquant.py) called as the "
                       f"search calls it on the 16384-row embedding sample and on each of layer "
                       f"0's 7 tensors ({spent:.1f} s of CPU work), scaled by evaluations and "
                       f"layers to the search's {work} round-tripped weights (est. {total_t:.0f} s; "
                       f"the column profiles and the sort are not counted); single-threaded numpy"),
            "host_cpus": os.cpu_count()}


def perm_main(args):
    """The Qwen3-0.6B PERM search (coldpress/perm/spacemaps/qwen3.py:284-355) with every
    objective evaluation on the GPU: one step = one full search."""
    import ctypes
    import torch
    from perm_amd import _lib, objective, perm as gp
    from perm_amd import workloads as wl
    lib = _lib.load()
    dims = dict(wl.QWEN3_06B_DIMS, n_layers=args.layers)
    rows_sample = 16384
    log(f"building PERM workload: {args.layers} layers + embedding, f16")
    w = wl.qwen3_gguf_weights(layers=args.layers)
    ttypes = wl.qwen3_mixed_typemap(w)
    qws = wl.imatrix_means(w)
    n_keys = 3
    work = perm_search_weights(dims, rows_sample, n_keys)
    quiet = lambda *_: None  # noqa: E731
    for i in range(args.warmup):
        gp.optimize(w, ttypes, qws, dims, rows_sample=rows_sample, log=quiet)
        torch.cuda.synchronize()
        log(f"warmup {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        perms, report = gp.optimize(w, ttypes, qws, dims, rows_sample=rows_sample, log=quiet)
        log(f"step {i + 1}/{args.steps} done")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    # one profiled residual evaluation (the search's largest pass): phases by HIP events
    names = gp.res_space_tensors(w, dims)
    items = [dict(x=w[n], ttype=ttypes[n], qw=qws.get(n), perm=perms["res"],
                  rows_sample=rows_sample) for n in names]
    lib.cp_err_profile(1)
    objective.tensor_err_many(items)
    buf = (ctypes.c_float * 5)()
    lib.cp_err_phase_ms(ctypes.cast(buf, ctypes.c_void_p), 5)
    lib.cp_err_profile(0)
    ph = list(buf)
    res_w = sum(min(rows_sample, w[n].shape[0]) * w[n].shape[1] for n in names)
    # the encode kernels are VALU-bound; the column sums read 8 B and the gather
    # moves 6 B (f16 in, f32 out) per weight -- the HBM-bound phases
    colsum_bw = res_w * 8 / (ph[3] * 1e-3) / 1e9
    roof = {"kernel": "err_colsum_kernel", "bound": "hbm", "achieved": colsum_bw,
            "peak": 8000.0, "unit": "GB/s", "frac": colsum_bw / 8000.0, "traffic": None,
            "avg_launch_ms": ph[3], "launches_per_step": None,
            "note": "the search's dominant phase is the VALU-bound encode (phases_ms)"}
    result = {
        "metric": PERM_METRIC, "value": work / (wall / args.steps) / 1e6, "unit": "Mweights/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init f16 weights with per-channel log-normal scales)",
        "config": {"workload": f"qwen3-0.6b-shaped PERM search, {args.layers} layers + "
                               f"151936x1024 embedding, Q6_K/Q3_K/Q2_K, rows_sample 16384",
                   "layers": args.layers, "roundtrip_weights": work, "rows_sample": rows_sample,
                   "candidates": {"res": n_keys, "ffn": 1, "vo": 1}},
        "report": {k: v for k, v in report.items() if k != "seconds"},
        "res_pass": {"weights": res_w, "phases_ms": {
            "gather": ph[0], "encode": ph[1], "decode": ph[2], "colsum": ph[3], "total": ph[4]}},
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle tensor_err on 256-row slices)")
        result["cpu_baseline"] = perm_cpu_baseline(w, ttypes, qws, rows_sample, n_keys, dims)
        result["gpu_over_cpu"] = result["value"] / result["cpu_baseline"]["value"]
    print(json.dumps(result))


def copy_main(args):
    """A plain elementwise device copy of 1 GiB (read 1 GiB, write 1 GiB) per step: the
    known-size kernel against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are
    scaled into HBM bytes."""
    import torch
    nbytes = 1 << 30
    x = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(args.warmup):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "device copy GB/s (HBM byte-counter calibration)", "value": gbs, "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic", "config": {"workload": "copy", "kernel": "torch.mul(x, 1.0, out=y)",
                                        "bytes_read": nbytes, "bytes_written": nbytes}}))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--layers", type=int, default=28,
                    help="decoder layers (28 = the full workload; fewer only for quick checks)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ef-mode", choices=["mfma", "exact"], default="exact",
                    help="cross-block error propagation: MFMA GEMM or the reference's exact order")
    ap.add_argument("--workload", choices=["ef", "perm-search", "copy"], default="ef",
                    help="ef: the EF encode + Hessians line (default); perm-search: the PERM "
                         "space-map search on the GPU objective; copy: a plain 1 GiB device "
                         "copy, the calibration run for the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        msg = (f"bench.py runs on one GPU only (got --gpus {args.gpus}); the encoder path "
               f"shards by tensor / row stripe with no exchange between GPUs")
        print(msg, file=sys.stderr)
        print(json.dumps({"metric": METRIC, "error": msg}))
        sys.exit(2)

    import torch
    from perm_amd import _lib
    from perm_amd import workloads as wl
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    if args.workload == "perm-search":
        perm_main(args)
        return
    if args.workload == "copy":
        copy_main(args)
        return
    lib = _lib.load()
    dev = "cuda"
    layers = args.layers
    total_weights = layers * sum(r * n for _, r, n, _ in wl.QWEN3_06B_LAYER)
    # the Hessian kernel computes the lower triangle only: N*d*(d+1) algorithmic flops per H
    hess_flops = layers * sum(float(ROWS) * d * (d + 1) for d in wl.QWEN3_06B_FAMILIES.values())
    ef_flops = 2 * layers * sum(r * n * (n - 1) for _, r, n, _ in wl.QWEN3_06B_LAYER)
    log(f"building workload: {layers} layers, {total_weights} weights")
    X, W, H, slot = build_workload(layers, dev)
    mode = _lib.CP_EF_MFMA if args.ef_mode == "mfma" else _lib.CP_EF_EXACT
    other = _lib.CP_EF_EXACT if mode == _lib.CP_EF_MFMA else _lib.CP_EF_MFMA

    def step():
        hs, he, ee = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        hs.record()
        hessian_phase(X, H, slot)
        he.record()
        ef_phase(W, H, slot, layers, mode)
        ee.record()
        return hs, he, ee

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup {i + 1}/{args.warmup} done")

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks = []
    for i in range(args.steps):
        marks.append(step())
        log(f"step {i + 1}/{args.steps} done")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # after the timed region: one sequential EF pass with per-phase timing
    import ctypes
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    lib.cp_ef_profile(1)
    p0.record()
    phases = []
    for d in sorted(H, reverse=True):
        ef_phase(W, {d: H[d]}, slot, layers, mode, concurrent=False)
        buf = (ctypes.c_float * 5)()
        lib.cp_ef_phase_ms(ctypes.cast(buf, ctypes.c_void_p), 5)
        phases.append(list(buf))
    p1.record()
    lib.cp_ef_profile(0)
    torch.cuda.synchronize()
    seq_ms = p0.elapsed_time(p1)

    # one untimed-by-contract step of the other EF mode, reported for comparison
    o0, o1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    o0.record()
    ef_phase(W, H, slot, layers, other)
    o1.record()
    torch.cuda.synchronize()
    other_ms = o0.elapsed_time(o1)

    hess_ms = sum(hs.elapsed_time(he) for hs, he, _ in marks) / args.steps
    ef_ms = sum(he.elapsed_time(ee) for _, he, ee in marks) / args.steps
    ph = [sum(p[k] for p in phases) for k in range(5)]
    ms_per_step = wall * 1e3 / args.steps
    ef_mw = total_weights / (ef_ms * 1e-3) / 1e6
    hess_tflops = hess_flops / (hess_ms * 1e-3) / 1e12

    # dominant kernel: the Hessian MFMA kernel (one launch per Hessian) or the EF sweep
    hess_launches = len(H)  # one batched launch per Hessian size
    sweep_launches = 2 * len(H)  # sequential pass: two iterations per size class
    if hess_ms >= ph[2]:
        avg_ms = hess_ms / hess_launches
        flops_per_launch = hess_flops / hess_launches
        ach = flops_per_launch / (avg_ms * 1e-3) / 1e12
        roof = {"kernel": "hess_bf16_tri_kernel", "bound": "mfma", "achieved": ach,
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": ach / PEAK_BF16_TFLOPS,
                "traffic": None, "avg_launch_ms": avg_ms, "launches_per_step": hess_launches}
    else:
        avg_ms = ph[2] / sweep_launches
        flops_per_launch = ef_flops / sweep_launches
        ach = flops_per_launch / (avg_ms * 1e-3) / 1e12
        exact_full = mode == _lib.CP_EF_EXACT and layers == 28
        roof = {"kernel": ("ef_sweep_mfma_kernel" if mode == _lib.CP_EF_MFMA
                           else "ef_sweep_rows_kernel"), "bound": "mfma", "achieved": ach,
                "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": ach / PEAK_FP32_TFLOPS,
                "traffic": SWEEP_TRAFFIC_BYTES if exact_full else None,
                "avg_launch_ms": avg_ms, "launches_per_step": sweep_launches}

    result = {
        "metric": METRIC,
        "value": ef_mw,
        "unit": "Mweights/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init weights, Student-t bf16 activations; generated on device)",
        "config": {"workload": f"qwen3-0.6b-shaped {layers}-layer Q2_K EF + Hessians",
                   "layers": layers, "tensors": 7 * layers, "weights": total_weights,
                   "hessians": 4 * layers, "hessian_rows": ROWS, "activations": "bf16",
                   "container": "Q2_K", "qw": "diag(H)/N", "n_iter": 2, "damp": 0.01,
                   "act_order": True, "ef_mode": args.ef_mode},
        "ef": {"ms": ef_ms, "mweights_per_s": ef_mw, "flops_update": ef_flops,
               "sequential_pass": {"ms": seq_ms, "phase_ms": {
                   "factor_and_setup": seq_ms - sum(ph), "setup": ph[0], "commit": ph[1],
                   "sweep": ph[2], "repack": ph[3], "decode": ph[4]}},
               "other_mode": {"mode": "exact" if mode == _lib.CP_EF_MFMA else "mfma",
                              "ms": other_ms,
                              "mweights_per_s": total_weights / (other_ms * 1e-3) / 1e6}},
        "hessian": {"ms": hess_ms, "tflops": hess_tflops, "flops": hess_flops,
                    "frac_of_bf16_peak": hess_tflops / PEAK_BF16_TFLOPS},
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle on a layer-0 row subsample)")
        result["cpu_baseline"] = cpu_baseline(W, H, slot, layers, total_weights)
        result["gpu_over_cpu"] = ef_mw / result["cpu_baseline"]["value"]
    print(json.dumps(result))


if __name__ == "__main__":
    main()
