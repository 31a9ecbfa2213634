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


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _pmc_child(counter, regex, argv, outdir, timeout=180):
    """One rocprofv3 --pmc run of ``bench.py <argv>`` as a child process: [(kernel, value)]
    of ``counter`` per dispatch of the kernels matching ``regex``, in dispatch order. The
    child runs in its own session; past ``timeout`` seconds the whole group (the profiler
    and the profiled program) is killed and the run counts as failed."""
    import csv
    import shutil
    import signal
    import subprocess
    prof = shutil.which("rocprofv3")
    if prof is None:
        raise RuntimeError("rocprofv3 not on PATH")
    cmd = [prof, "--pmc", counter, "--kernel-include-regex", regex, "--output-format", "csv",
           "-d", outdir, "-o", "p", "--", sys.executable, "-u", os.path.abspath(__file__), *argv]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    proc = subprocess.Popen(cmd, cwd=ROOT, env=env, stdout=subprocess.DEVNULL,
                            stderr=subprocess.PIPE, text=True, start_new_session=True)
    try:
        _out, err = proc.communicate(timeout=timeout)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.communicate()
        raise RuntimeError(f"{counter} run of {argv[1]} exceeded {timeout} s")
    path = os.path.join(outdir, "p_counter_collection.csv")
    if not os.path.exists(path):
        raise RuntimeError(f"{counter} run exited {proc.returncode} without counters: "
                           f"{err.strip().splitlines()[-1:]}")
    rows = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                key = int(r["Dispatch_Id"])
                name, val = rows.get(key, (r["Kernel_Name"], 0.0))
                rows[key] = (name, val + float(r["Counter_Value"]))
    # rocprofv3 may end with a signal after the program finished and the file is complete;
    # the caller checks the dispatch count it expects
    return [rows[k] for k in sorted(rows)]


def last_sweep_kernel(lib):
    """The kernel of the calling thread's last EF sweep launch, as the library reports it."""
    import ctypes
    rs, wv = (ctypes.c_int * 1)(), (ctypes.c_int * 1)()
    lib.cp_ef_last_sweep(ctypes.cast(rs, ctypes.c_void_p), ctypes.cast(wv, ctypes.c_void_p))
    if wv[0] > 1:
        return f"ef_sweep_pipe_kernel<{rs[0]}, {wv[0]}>"
    return f"ef_sweep_rows_kernel<{rs[0]}>"


def measure_sweep_traffic(layers):
    """HBM bytes per launch of the exact EF sweep (ef_sweep_rows_kernel / ef_sweep_pipe_kernel,
    one launch per size class and iteration): the mean over the
    sequential pass's launches (two per size class) of FETCH_SIZE and WRITE_SIZE, each read
    in its own rocprofv3 --pmc child run of ``--workload sweep-pass`` and scaled by what the
    same counter reads for the 1 GiB copy of ``--workload copy`` (reads and writes exactly
    2^30 bytes). Runs before this process touches the GPU. Returns (bytes, detail)."""
    import tempfile
    tmp = tempfile.mkdtemp(prefix="bench_pmc_", dir=os.environ.get("TMPDIR", "/tmp"))
    t0 = time.perf_counter()
    kib = float(1 << 30) / 1024.0
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        copy = _pmc_child(counter, "MulFunctor", ["--workload", "copy", "--steps", "1",
                                                  "--warmup", "0"],
                          os.path.join(tmp, f"copy_{counter}"))
        if len(copy) != 1 or copy[0][1] <= 0:
            raise RuntimeError(f"copy calibration: {len(copy)} dispatches of the copy kernel")
        sweep = _pmc_child(counter, "ef_sweep_(rows|pipe)", ["--workload", "sweep-pass",
                                                             "--layers", str(layers)],
                           os.path.join(tmp, f"sweep_{counter}"))
        if len(sweep) != 6:
            raise RuntimeError(f"sweep pass: {len(sweep)} sweep dispatches, expected 6")
        scale = kib / copy[0][1]
        got[counter] = {"copy_kib": copy[0][1], "scale": scale,
                        "per_launch_bytes": [v * 1024.0 * scale for _n, v in sweep]}
        log(f"traffic: {counter} measured ({time.perf_counter() - t0:.0f} s so far)")
    fetch = got["FETCH_SIZE"]["per_launch_bytes"]
    write = got["WRITE_SIZE"]["per_launch_bytes"]
    total = (sum(fetch) + sum(write)) / len(fetch)
    detail = {"source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, one child run each of "
                        "`bench.py --workload sweep-pass` (the sequential pass's six sweep "
                        "launches) and of `--workload copy` (1 GiB read + 1 GiB written) for "
                        "the counter scale, run by this bench before its own timed steps",
              "fetch_bytes_per_launch": fetch, "write_bytes_per_launch": write,
              "fetch_scale": got["FETCH_SIZE"]["scale"], "write_scale": got["WRITE_SIZE"]["scale"],
              "seconds": time.perf_counter() - t0}
    return total, detail


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


def ef_phase(W, H, slot, layers, mode, concurrent=True, keep=None):
    """Act order + factor per Hessian size class, then EF of that class's tensors.
    With ``concurrent`` each size class runs on its own stream, so one class's
    factorization overlaps another's sweep (perm_amd.ef.encode_size_classes).
    ``keep`` (a dict, for parity checks) receives each class's (U, order, qw) by size."""
    from perm_amd import ef as gef
    from perm_amd import workloads as wl

    def builder(d):
        def build(U, order):
            # qw = diag(H) / N for every Hessian of the class in one kernel
            qw = (H[d].diagonal(dim1=1, dim2=2) / float(ROWS)).contiguous()
            if keep is not None:
                keep[d] = (U, order, qw)
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
    # one class at a time, queued as encode_size_classes queues each class: a single
    # factorization attempt whose flags are read after the class's EF, so the host does
    # not wait between the factorization and the EF; a failed matrix sends the class
    # through the escalating factorization and the EF again
    outs = []
    for Hb, build in classes:
        order = gef.act_order_dev(Hb)
        U, flags = gef.factor_dev_async(Hb, order, 0.01, checked=True)
        words = []
        out = gef.ef_encode_dev(build(U, order), n_iter=2, mode=mode, checked=True, status=words)
        if int(flags.sum()):
            U, _ = gef.factor_dev(Hb, order, 0.01, checked=True)
            out = gef.ef_encode_dev(build(U, order), n_iter=2, mode=mode, checked=True)
        else:
            gef.check_status(words)
        outs.append(out)
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


FORMAT_TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]


def formats_cpu_baseline(W0, qws0, Hs):
    """The numpy oracle (a port of kquant.py / scale_tune.py / hessians.py) on samples:
    layer 0's ffn_up (3072 x 1024) per container (encode + decode), one 3072 x 3072
    Hessian (pack + expand); extrapolated per weight / per entry."""
    import numpy as np
    from oracle import hess_oracle as Ho
    from oracle import kquant_oracle as Ko
    x = W0["ffn_up"].cpu().numpy()
    qw = qws0[x.shape[1]].cpu().numpy()
    per_w = {}
    spent = 0.0
    for tt in FORMAT_TYPES:
        t0 = time.perf_counter()
        raw = Ko.QUANTIZE[tt](x, None if tt == "Q8_0" else qw)
        Ko.DEQUANTIZE[tt](raw, x.shape[1])
        dt = time.perf_counter() - t0
        spent += dt
        per_w[tt] = dt / x.size
    H = Hs[3072][0].cpu().numpy()
    t0 = time.perf_counter()
    H16, dg, hs = Ho.h2_pack(H)
    Ho.h2_expand(H16, hs, dg)
    h2_dt = time.perf_counter() - t0
    spent += h2_dt
    return per_w, h2_dt / H.size, spent


def formats_main(args):
    """Data-format rows on the Qwen3-0.6B-shaped layer set (28 layers, 196 tensors,
    440,401,920 weights, imatrix-style qw): encode and decode of all six containers, the
    linear form of the five k-quants (extract A / B / d / dmin, then reconstruct), and the
    Hessian storage format (pack to float16 + diag32 + hscale, expand to float64) of the
    112 Hessians' shapes. One step = every format over the whole set."""
    import numpy as np
    import torch
    from perm_amd import _lib, hessians, kquant, scale_tune
    from perm_amd import workloads as wl
    layers = args.layers
    lib = _lib.load()
    W = [wl.qwen3_layer_weights(l, seed=0, device="cuda") for l in range(layers)]
    g = torch.Generator(device="cuda").manual_seed(7)
    qws = {n: torch.rand(n, device="cuda", generator=g) + 0.05 for n in (1024, 2048, 3072)}
    xs = [(w[name], qws[n]) for w in W for name, _r, n, _f in wl.QWEN3_06B_LAYER]
    total_w = sum(x.numel() for x, _ in xs)
    # Hessian-shaped float32 matrices with entries past float16's range (the scaled path)
    Hs = {1024: torch.randn((2 * layers, 1024, 1024), device="cuda", generator=g) * 4e4,
          2048: torch.randn((layers, 2048, 2048), device="cuda", generator=g) * 4e4,
          3072: torch.randn((layers, 3072, 3072), device="cuda", generator=g) * 4e4}
    h_entries = sum(Hb.numel() for Hb in Hs.values())
    dec_out = [torch.empty_like(x) for x, _ in xs]
    h16 = {d: torch.empty(Hb.shape, dtype=torch.float16, device="cuda") for d, Hb in Hs.items()}
    hdg = {d: torch.empty(Hb.shape[:2], dtype=torch.float32, device="cuda") for d, Hb in Hs.items()}
    hsc = {d: torch.empty(Hb.shape[0], dtype=torch.float32, device="cuda") for d, Hb in Hs.items()}
    hexp = torch.empty(3072 * 3072, dtype=torch.float64, device="cuda")
    hs_host = {}  # the per-matrix scales as a reader holds them (from the file: host values)
    ws = _lib.workspace(256, torch.device("cuda"))
    torch.cuda.synchronize()

    def run_type(tt, check=False):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        ev[0].record()
        raws = [kquant.quantize_dev(tt, x, None if tt == "Q8_0" else q) for x, q in xs]
        ev[1].record()
        for (x, _), raw, out in zip(xs, raws, dec_out):
            kquant.dequantize_dev(tt, raw, x.shape[1], out=out)
        ev[2].record()
        lins = []
        if tt != "Q8_0":
            lins = [scale_tune.extract_linear_dev(raw, tt, x.shape[1]) for (x, _), raw in zip(xs, raws)]
        ev[3].record()
        recs = [scale_tune._reconstruct_dev(L["d"], L["dmin"], L["A"], L["B"], L["shape"]) for L in lins]
        ev[4].record()
        torch.cuda.synchronize()
        if check:  # the linear form reconstructs exactly what the decoder gives
            for i in (0, len(xs) - 1):
                if recs and not torch.equal(torch.nan_to_num(recs[i]), torch.nan_to_num(dec_out[i])):
                    raise RuntimeError(f"{tt}: linear-form reconstruction differs from the decoder")
        raw_bytes = sum(r.numel() for r in raws)
        return [ev[k].elapsed_time(ev[k + 1]) for k in range(4)], raw_bytes

    def run_h2():
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record()
        for d, Hb in Hs.items():
            for i in range(Hb.shape[0]):
                _lib.check(lib.cp_h2_pack(_lib.ptr(Hb[i]), d, _lib.ptr(h16[d][i]), _lib.ptr(hdg[d][i]),
                                          _lib.ptr(hsc[d][i:i + 1]), _lib.ptr(ws), ws.numel(),
                                          _lib.stream_ptr()))
        ev[1].record()
        for d, Hb in Hs.items():
            out = hexp[:d * d].view(d, d)
            for i in range(Hb.shape[0]):
                _lib.check(lib.cp_h2_expand(_lib.ptr(h16[d][i]), 1, d, hs_host[d][i],
                                            _lib.ptr(hdg[d][i]), _lib.ptr(out), _lib.stream_ptr()))
        ev[2].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])

    # one launch over a large tensor shows the decode kernel's own HBM rate (the
    # per-tensor calls above carry ~7 us of launch each): every n = 1024 tensor stacked
    big = torch.cat([x for x, _ in xs if x.shape[1] == 1024])
    big_out = torch.empty_like(big)
    big_raw = {tt: kquant.quantize_dev(tt, big, None if tt == "Q8_0" else qws[1024])
               for tt in FORMAT_TYPES}

    def run_big(tt, reps=5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            kquant.dequantize_dev(tt, big_raw[tt], big.shape[1], out=big_out)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for tt in FORMAT_TYPES:
        run_type(tt, check=True)
        run_big(tt, 1)
    for d, Hb in Hs.items():
        hs_host[d] = [1.0] * Hb.shape[0]
    run_h2()
    hs_host.update({d: hsc[d].cpu().tolist() for d in Hs})
    log(f"formats: {len(xs)} tensors, {total_w} weights, {h_entries} Hessian entries")
    acc = {tt: np.zeros(4) for tt in FORMAT_TYPES}
    raw_b = {}
    h2 = np.zeros(2)
    for _ in range(args.warmup):
        for tt in FORMAT_TYPES:
            run_type(tt)
        run_h2()
    t0 = time.perf_counter()
    for k in range(args.steps):
        for tt in FORMAT_TYPES:
            ms, raw_b[tt] = run_type(tt)
            acc[tt] += ms
        h2 += np.array(run_h2())
        log(f"step {k + 1}/{args.steps} done")
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    per = {}
    enc_dec_ms = 0.0
    dec_bytes, dec_ms = 0.0, 0.0
    for tt in FORMAT_TYPES:
        e, dcd, ex, rc = acc[tt] / args.steps
        enc_dec_ms += e + dcd
        dec_bytes += raw_b[tt] + 4.0 * total_w
        dec_ms += dcd
        per[tt] = {"encode_ms": e, "decode_ms": dcd, "encode_mweights_per_s": total_w / e / 1e3,
                   "decode_gb_per_s": (raw_b[tt] + 4.0 * total_w) / (dcd * 1e-3) / 1e9,
                   "container_bytes": raw_b[tt]}
        if tt != "Q8_0":
            nsb = total_w // 256
            lin_bytes = raw_b[tt] + 4.0 * total_w + 8.0 * nsb  # in: bytes; out: A, B int16, d, dmin
            per[tt]["linear_extract_ms"] = ex
            per[tt]["linear_extract_gb_per_s"] = lin_bytes / (ex * 1e-3) / 1e9
            per[tt]["linear_reconstruct_ms"] = rc
            per[tt]["linear_reconstruct_gb_per_s"] = (4.0 * total_w + 8.0 * nsb + 4.0 * total_w) / (rc * 1e-3) / 1e9
    for tt in FORMAT_TYPES:
        ms = run_big(tt)
        per[tt]["decode_large_ms"] = ms
        per[tt]["decode_large_gb_per_s"] = (big_raw[tt].numel() + 4.0 * big.numel()) / (ms * 1e-3) / 1e9
    pack_ms, expand_ms = h2 / args.steps
    h2_res = {"matrices": sum(Hb.shape[0] for Hb in Hs.values()), "entries": h_entries,
              "pack_ms": pack_ms, "pack_gb_per_s": 6.0 * h_entries / (pack_ms * 1e-3) / 1e9,
              "expand_ms": expand_ms, "expand_gb_per_s": 10.0 * h_entries / (expand_ms * 1e-3) / 1e9}
    value = len(FORMAT_TYPES) * total_w / (enc_dec_ms * 1e-3) / 1e6
    big_bytes = sum(big_raw[tt].numel() + 4.0 * big.numel() for tt in FORMAT_TYPES)
    big_ms = sum(per[tt]["decode_large_ms"] for tt in FORMAT_TYPES)
    dec_bw = big_bytes / (big_ms * 1e-3) / 1e9
    roof = {"kernel": "kq_decode_kernel / q8_decode_kernel (six containers)", "bound": "hbm",
            "achieved": dec_bw, "peak": 8000.0, "unit": "GB/s", "frac": dec_bw / 8000.0,
            "traffic": None, "avg_launch_ms": big_ms / len(FORMAT_TYPES), "launches_per_step": None,
            "note": (f"one launch per container over the {big.shape[0]} x {big.shape[1]} stack of every "
                     f"n = 1024 tensor; algorithmic bytes: the container bytes read + 4 B per weight "
                     f"written. The per-tensor decodes of the step run at "
                     f"{dec_bytes / (dec_ms * 1e-3) / 1e9:.0f} GB/s (launch-bound). The encodes are "
                     f"VALU-bound (the make_q*_quants candidate searches).")}
    result = {
        "metric": "container codec encode+decode Mweights/s (Q2_K..Q6_K, Q8_0), 1 GPU",
        "value": value, "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall_ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init weights, random positive qw; Hessian-shaped random "
                "float32 matrices past float16's range; generated on device)",
        "config": {"workload": "qwen3-0.6b-shaped 28-layer tensor set, every container",
                   "layers": layers, "tensors": len(xs), "weights": total_w,
                   "containers": FORMAT_TYPES, "qw": "random positive (none for Q8_0)",
                   "hessians": h2_res["matrices"]},
        "formats": per, "hessian_storage": h2_res, "roofline": roof,
    }
    if not args.no_cpu_baseline:
        per_w, h2_per_entry, spent = formats_cpu_baseline(W[0], qws, Hs)
        cpu_s = sum(per_w.values()) * total_w
        result["cpu_baseline"] = {
            "value": len(FORMAT_TYPES) * total_w / cpu_s / 1e6, "unit": "Mweights/s", "cores": 1,
            "kind": "port",
            "sample": (f"numpy oracle QUANTIZE + DEQUANTIZE (port of kquant.py) on layer 0's ffn_up "
                       f"(3072x1024) per container and the h2 pack + expand of one 3072x3072 matrix "
                       f"({spent:.1f} s of CPU work), extrapolated per weight to the six containers "
                       f"over {total_w} weights (est. {cpu_s:.0f} s); single-threaded numpy"),
            "host_cpus": os.cpu_count()}
        result["cpu_baseline"]["hessian_storage_entries_per_s"] = 1.0 / h2_per_entry
        result["gpu_over_cpu"] = value / result["cpu_baseline"]["value"]
    print(json.dumps(result))


def gguf_cpu_baseline(Wl0, Hl0, emb, rows, layers, n_emb_rows, typemap, total_w):
    """The numpy oracle (port of ef.py / kquant.py) doing the driver's per-tensor work:
    for each of layer 0's 7 tensors one factorization (per tensor, as ef.py:189) and the
    EF at 128 and 512 rows, extrapolated linearly in rows and to every layer; the
    embedding's weighted Q6_K RTN timed on 256 rows and scaled to its rows. File I/O is
    not counted."""
    import numpy as np
    from oracle import ef_oracle as E
    from oracle import kquant_oracle as Ko
    from perm_amd import workloads as wl
    t_total, spent = 0.0, 0.0
    for name, nrow, n, fam in wl.QWEN3_06B_LAYER:
        tt = typemap[f"blk.0.{name}.weight"]
        Hn = Hl0[fam]
        t0 = time.perf_counter()
        order = E.act_order(Hn)
        U = E.inv_upper_factor(Hn[np.ix_(order, order)], 0.01).astype(np.float32)
        t_fact = time.perf_counter() - t0
        ts = {}
        for r in (128, 512):
            t0 = time.perf_counter()
            E.ef_encode(Wl0[name][:r], tt, None, Hn, U=U)
            ts[r] = time.perf_counter() - t0
        b = (ts[512] - ts[128]) / 384.0
        t_total += (t_fact + ts[128] - 128 * b + b * nrow) * layers
        spent += t_fact + ts[128] + ts[512]
    w_emb = (np.diag(Hl0["qkv_in"]) / rows).astype(np.float32)
    t0 = time.perf_counter()
    Ko.QUANTIZE["Q6_K"](emb, w_emb)
    dt = time.perf_counter() - t0
    spent += dt
    t_total += dt * n_emb_rows / emb.shape[0]
    return {"value": total_w / t_total / 1e6, "unit": "Mweights/s", "cores": 1, "kind": "port",
            "sample": (f"numpy oracle (port of ef.py / kquant.py): layer 0's 7 tensors at 128 and "
                       f"512 rows with one factorization each, and the embedding's weighted Q6_K "
                       f"RTN on 256 rows ({spent:.1f} s of CPU work), extrapolated to the artifact's "
                       f"{total_w} weights (est. {t_total:.0f} s; file I/O not counted); the sweep "
                       f"and codec are single-threaded numpy"),
            "host_cpus": os.cpu_count()}


def gguf_main(args):
    """The encode_gguf driver (coldpress/ef.py:223-317) end to end on a synthetic
    Qwen3-0.6B artifact written to a temporary directory: the f16 GGUF (token_embd
    151936 x 1024 plus 28 layers x 7 tensors), the stock quant (Q6_K embedding, Q3_K
    attention, Q2_K elsewhere, encoded on the GPU) and the per-family Hessian files
    (H = X^T X over 16384 Student-t bf16 rows per family, stored in the float16 format).
    One step = one encode_gguf call: read the f16 weights and the Hessians, EF every
    tensor with a Hessian (act order, fp64 factor, two iterations), weighted RTN of the
    embedding, write the output GGUF."""
    import shutil
    import tempfile
    import numpy as np
    import torch
    from perm_amd import ef as gef
    from perm_amd import gates, hessians, kquant
    from perm_amd import workloads as wl
    from perm_amd.gguffile import GGUFWriter, ValueType
    layers = args.layers
    tmp = tempfile.mkdtemp(prefix="cp_gguf_bench_")
    try:
        f16, stock, hdir, out = (os.path.join(tmp, k) for k in ("f16.gguf", "stock.gguf", "hess", "ef.gguf"))
        w = wl.qwen3_gguf_weights(layers=layers, device="cuda")
        typemap = wl.qwen3_mixed_typemap(w.keys())
        total_w = sum(t.numel() for t in w.values())
        wr = GGUFWriter(f16, "qwen3")
        wr.add_kv("qwen3.block_count", layers, ValueType.UINT32)
        for name, t in w.items():
            wr.add_tensor(name, t.cpu().numpy())
        wr.write()
        wr = GGUFWriter(stock, "qwen3")
        wr.add_kv("qwen3.block_count", layers, ValueType.UINT32)
        for name, t in w.items():
            wr.add_tensor(name, kquant.quantize_dev(typemap[name], t.float().contiguous()).cpu().numpy(),
                          typemap[name])
        wr.write()
        rows = 16384
        fams = {}
        for l in range(layers):
            for i, (fam, d) in enumerate(wl.QWEN3_06B_FAMILIES.items()):
                X = wl.student_t_activations(rows, d, nu=4.0, seed=1000 * l + i, device="cuda")
                fams[f"blk.{l}.{fam}"] = {"H": hessians.xtx_accumulate(X), "n": rows}
        hessians.save_hessians(fams, hdir)
        base_in = None
        if not args.no_cpu_baseline:
            base_in = ({nm: w[f"blk.0.{nm}.weight"].float().cpu().numpy()
                        for nm, *_ in wl.QWEN3_06B_LAYER},
                       {fam: fams[f"blk.0.{fam}"]["H"].double().cpu().numpy()
                        for fam in wl.QWEN3_06B_FAMILIES},
                       w["token_embd.weight"][:256].float().cpu().numpy(),
                       w["token_embd.weight"].shape[0])
        del fams, w
        torch.cuda.synchronize()
        log(f"artifact: {total_w} weights, {4 * layers} Hessian files in {tmp}")
        quiet = (lambda *_: None)
        for _ in range(args.warmup):
            gef.encode_gguf(f16, stock, hdir, out, log=quiet)
        t0 = time.perf_counter()
        for k in range(args.steps):
            stats = gef.encode_gguf(f16, stock, hdir, out, log=quiet)
            log(f"step {k + 1}/{args.steps} done")
        torch.cuda.synchronize()
        sec = (time.perf_counter() - t0) / args.steps
        rep = gates.byte_parity(out, stock)
        modes = {}
        for st in stats.values():
            modes[st["mode"]] = modes.get(st["mode"], 0) + 1
        med = float(np.median([st["rel_err_vs_stock"] for st in stats.values()]))
        value = total_w / sec / 1e6
        result = {
            "metric": "encode_gguf end-to-end Mweights/s (Qwen3-0.6B-shaped artifact), 1 GPU",
            "value": value, "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": sec * 1e3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (random-init f16 weights, Student-t bf16 activations for the "
                    "Hessians; written to a temporary directory)",
            "config": {"workload": "encode_gguf, qwen3-0.6b-shaped artifact", "layers": layers,
                       "tensors": len(stats), "weights": total_w,
                       "containers": "Q6_K token_embd, Q3_K attention, Q2_K elsewhere",
                       "hessian_files": 4 * layers, "hessian_rows": rows, "n_iter": 2},
            "modes": modes, "median_rel_err_vs_stock": med,
            "byte_parity": {"passed": rep["passed"], "total_final": rep["total_final"],
                            "total_stock": rep["total_stock"]},
            "roofline": None,
            "roofline_note": "end to end: host file I/O (GGUF and Hessian reads, GGUF write) plus "
                             "the GPU codec / factor / EF; the kernels' rooflines are in the "
                             "default (ef) and formats lines",
        }
        if base_in is not None:
            Wl0, Hl0, emb, n_emb = base_in
            result["cpu_baseline"] = gguf_cpu_baseline(Wl0, Hl0, emb, rows, layers, n_emb, typemap,
                                                       total_w)
            result["gpu_over_cpu"] = value / result["cpu_baseline"]["value"]
        print(json.dumps(result))
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def sweep_pass_main(args):
    """The ef workload's sequential exact-mode EF pass alone (one size class at a time, two
    sweep launches each), after its Hessians: the run whose sweep launches the HBM byte
    counters are read on. Prints nothing on stdout."""
    import torch
    from perm_amd import _lib
    X, W, H, slot = build_workload(args.layers, "cuda")
    hessian_phase(X, H, slot)
    del X
    torch.cuda.synchronize()
    for d in sorted(H, reverse=True):
        ef_phase(W, {d: H[d]}, slot, args.layers, _lib.CP_EF_EXACT, concurrent=False)
        torch.cuda.synchronize()
        log(f"sweep pass: class {d} done")


def hessian_power_main(args):
    """The ef workload's Hessian phase (112 accumulations, 65536 bf16 rows) on two inputs of
    the same shapes, run by the same kernels: the Student-t activations, then every
    activation set to 1.0. The instruction stream is identical; only the operand bits the
    matrix cores switch differ, so a rate that rises on the constant input is set by the
    chip's power limit (its clock), not by the schedule. Read the clock with rocprofv3
    counters (GRBM_GUI_ACTIVE) on this workload."""
    import numpy as np
    import torch
    from perm_amd import workloads as wl
    layers = args.layers
    X, H, slot = [], {}, {}
    for l in range(layers):
        X.append({fam: wl.student_t_activations(ROWS, d, nu=4.0, seed=1000 * l + i, device="cuda")
                  for i, (fam, d) in enumerate(wl.QWEN3_06B_FAMILIES.items())})
    H = {1024: torch.zeros((2 * layers, 1024, 1024), device="cuda"),
         2048: torch.zeros((layers, 2048, 2048), device="cuda"),
         3072: torch.zeros((layers, 3072, 3072), device="cuda")}
    for l in range(layers):
        slot[(l, "qkv_in")] = (1024, l)
        slot[(l, "gateup_in")] = (1024, layers + l)
        slot[(l, "o_in")] = (2048, l)
        slot[(l, "down_in")] = (3072, l)
    flops = layers * sum(float(ROWS) * d * (d + 1) for d in wl.QWEN3_06B_FAMILIES.values())

    def timed():
        for _ in range(args.warmup):
            hessian_phase(X, H, slot)
        torch.cuda.synchronize()
        ms = []
        for _ in range(args.steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            hessian_phase(X, H, slot)
            b.record()
            torch.cuda.synchronize()
            ms.append(a.elapsed_time(b))
        return float(np.median(ms))

    real = timed()
    log(f"hessian-power: Student-t activations {real:.2f} ms")
    for fams in X:
        for Xf in fams.values():
            Xf.fill_(1.0)
    const = timed()
    log(f"hessian-power: constant activations {const:.2f} ms")
    peak = 2516.6e12

    def rate(ms):
        return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                "frac_of_bf16_peak": flops / (ms * 1e-3) / peak}

    print(json.dumps({
        "metric": "Hessian X^T·X TFLOP/s on real and constant activations, 1 GPU",
        "value": flops / (real * 1e-3) / 1e12, "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": real,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (Student-t bf16 activations; then the same tensors filled with 1.0)",
        "config": {"workload": "hessian-power: the ef workload's Hessian phase", "layers": layers,
                   "hessians": 4 * layers, "hessian_rows": ROWS},
        "student_t": rate(real), "constant": rate(const), "speedup_constant": real / const}))


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


CONFIG_METRIC = "EF k-quant encode Mweights/s + Hessian X^T·X TFLOP/s, 1 GPU"
CONFIG_WORKLOADS = ("single-linear", "tied-output", "llama3-8b-layer")


def config_cpu_baseline(spec, W, H, slot, rows_of, counts_fn):
    """The numpy oracle (port of ef.py:46-218 + kquant.py) on one tensor of every distinct
    (shape, container, importance) class of the spec: the factorization of its Hessian
    (ef.py:189 runs one per tensor) plus EF at two row counts, fit as a + b * rows and
    extrapolated to the class's tensors. A tensor of at most 1024 rows is timed whole."""
    import numpy as np
    from oracle import ef_oracle as E
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # threadpoolctl missing or unreadable
        blas_threads = 1
    classes = {}
    for name, rows, n, fam, tt, qwk in spec["tensors"]:
        classes.setdefault((rows, n, tt, qwk, fam.split(".")[-1]), []).append((name, fam))
    t_total, spent, fact_cache, notes = 0.0, 0.0, {}, []
    for (rows, n, tt, qwk, fkind), members in classes.items():
        name, fam = members[0]
        d, i = slot[fam]
        Hn = H[d][i].double().cpu().numpy()
        qw = (np.diag(Hn) / (1.0 if spec["normalize"] else rows_of[fam])).astype(np.float32) \
            if qwk == "diag" else None
        key = (d, i)
        if key not in fact_cache:
            t0 = time.perf_counter()
            order = E.act_order(Hn)
            U = E.inv_upper_factor(Hn[np.ix_(order, order)], 0.01).astype(np.float32)
            fact_cache[key] = (order, U, time.perf_counter() - t0)
            spent += fact_cache[key][2]
        order, U, t_fact = fact_cache[key]
        Wn = W[name]
        if rows <= 1024:
            t0 = time.perf_counter()
            E.ef_encode(Wn.cpu().numpy(), tt, qw, Hn, U=U, order=order)
            t_rows = time.perf_counter() - t0
            spent += t_rows
            t_tensor = t_fact + t_rows
            notes.append(f"{name} whole")
        else:
            r1, r2 = (8, 32) if n > 4096 else ((32, 128) if n > 1024 else (128, 512))
            ts = {}
            for r in (r1, r2):
                x = Wn[:r].cpu().numpy()
                t0 = time.perf_counter()
                E.ef_encode(x, tt, qw, Hn, U=U, order=order)
                ts[r] = time.perf_counter() - t0
                spent += ts[r]
            b = (ts[r2] - ts[r1]) / (r2 - r1)
            t_tensor = t_fact + ts[r1] + b * (rows - r1)
            notes.append(f"{name} at {r1}/{r2} rows")
        t_total += t_tensor * counts_fn(members)
        log(f"cpu {name} [{rows}x{n}] {tt}: factor {t_fact:.2f}s -> tensor {t_tensor:.1f}s "
            f"(x{counts_fn(members)})")
    total_weights = sum(r * n for _, r, n, *_ in spec["tensors"])
    return {
        "value": total_weights / t_total / 1e6, "unit": "Mweights/s", "cores": int(blas_threads),
        "kind": "port",
        "sample": (f"numpy oracle (port of ef.py/kquant.py), one tensor per shape/container "
                   f"class ({'; '.join(notes)}), one factorization per tensor as the reference "
                   f"does; {spent:.1f} s of CPU work, extrapolated linearly in rows to the "
                   f"{len(spec['tensors'])} tensors (est. {t_total:.0f} s for the full encode); "
                   f"sweep and codec single-threaded numpy, factorization on {blas_threads} "
                   f"BLAS threads"),
        "host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
    }


def config_main(args):
    """One of the reference's other benchmark configurations (perm_amd.workloads.config_spec):
    per step, every Hessian of the spec (batched by size), then act order, factorization and
    two-iteration EF of every tensor (size classes on concurrent streams) with the final
    decode. value = EF Mweights/s; a sequential pass after the timed steps gives the
    factorization and sweep times the rooflines use."""
    import ctypes
    import torch
    from perm_amd import _lib, hessians
    from perm_amd import ef as gef
    from perm_amd import workloads as wl
    lib = _lib.load()
    spec = wl.config_spec(args.workload)
    fams = spec["families"]
    log(f"{args.workload}: {len(fams)} Hessians, {len(spec['tensors'])} tensors")
    X = {}
    for i, (k, (d, rows, kind)) in enumerate(fams.items()):
        X[k] = wl.family_activations(kind, rows, d, seed=1000 + i)
    W = wl.spec_weights(spec)
    sizes = sorted({d for d, _r, _k in fams.values()}, reverse=True)
    keys = {d: [k for k, (dd, _r, _k) in fams.items() if dd == d] for d in sizes}
    H = {d: torch.zeros((len(keys[d]), d, d), device="cuda") for d in sizes}
    slot = {k: (d, i) for d in sizes for i, k in enumerate(keys[d])}
    rows_of = {k: r for k, (_d, r, _k) in fams.items()}
    torch.cuda.synchronize()
    total_weights = sum(r * n for _, r, n, *_ in spec["tensors"])
    hess_flops = sum(float(r) * d * (d + 1) for d, r, _k in fams.values())
    ef_flops = 2 * sum(r * n * (n - 1) for _, r, n, *_ in spec["tensors"])
    fact_flops = sum(2.0 / 3.0 * d ** 3 for d, _r, _k in fams.values())

    def hessian_phase():
        for Hb in H.values():
            Hb.zero_()
        hessians.xtx_accumulate_many([X[k] for k in fams], [H[slot[k][0]][slot[k][1]] for k in fams])
        if spec["normalize"]:
            for k in fams:
                H[slot[k][0]][slot[k][1]].div_(float(rows_of[k]))

    def builder(d):
        def build(U, order):
            items = []
            for name, rows, n, fam, tt, qwk in spec["tensors"]:
                dd, i = slot[fam]
                if dd != d:
                    continue
                qw = None
                if qwk == "diag":
                    scale = 1.0 if spec["normalize"] else float(rows_of[fam])
                    qw = (torch.diagonal(H[d][i]) / scale).contiguous()
                items.append({"ttype": tt, "x": W[name], "qw": qw, "U": U[i], "order": order[i],
                              "recon": True})
            return items
        return build

    def ef_phase():
        return gef.encode_size_classes([(H[d], builder(d)) for d in sizes], n_iter=2,
                                       mode="exact", damp=0.01)

    def step():
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record()
        hessian_phase()
        ev[1].record()
        outs = ef_phase()
        ev[2].record()
        del outs  # released after the end mark: freeing the outputs is the caller's work
        return ev

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
    hess_ms = sum(a.elapsed_time(b) for a, b, _ in marks) / args.steps
    ef_ms = sum(b.elapsed_time(c) for _, b, c in marks) / args.steps

    # sequential pass: per size class, the factorization then the EF with phase timing.
    # One untimed factorization per size first: this pass runs on the caller's stream,
    # where a small batch's first factorization also creates its look-ahead stream.
    for d in sizes:
        gef.factor_dev_async(H[d], gef.act_order_dev(H[d]), 0.01, checked=True)
    torch.cuda.synchronize()
    fact_ms, phases, kernels = 0.0, [], {}
    lib.cp_ef_profile(1)
    for d in sizes:
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record()
        order = gef.act_order_dev(H[d])
        U, flags = gef.factor_dev_async(H[d], order, 0.01, checked=True)
        f1.record()
        words = []
        gef.ef_encode_dev(builder(d)(U, order), 2, _lib.CP_EF_EXACT, checked=True, status=words)
        if int(flags.sum()):  # a failed matrix: the escalating factorization, EF again
            U, _ = gef.factor_dev(H[d], order, 0.01, checked=True)
            gef.ef_encode_dev(builder(d)(U, order), 2, _lib.CP_EF_EXACT, checked=True)
        else:
            gef.check_status(words)
        kernels[d] = last_sweep_kernel(lib)
        buf = (ctypes.c_float * 5)()
        lib.cp_ef_phase_ms(ctypes.cast(buf, ctypes.c_void_p), 5)
        torch.cuda.synchronize()
        fact_ms += f0.elapsed_time(f1)
        phases.append(list(buf))
        del U, order
    lib.cp_ef_profile(0)
    ph = [sum(p[k] for p in phases) for k in range(5)]
    sweep_launches = 2 * len(sizes)
    avg_ms = ph[2] / sweep_launches
    ach = ef_flops / sweep_launches / (avg_ms * 1e-3) / 1e12
    ef_mw = total_weights / (ef_ms * 1e-3) / 1e6
    containers = sorted({tt for *_, tt, _q in spec["tensors"]})
    result = {
        "metric": CONFIG_METRIC, "value": ef_mw, "unit": "Mweights/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init weights, synthetic activations; generated on device)",
        "config": {"workload": args.workload, "tensors": len(spec["tensors"]),
                   "weights": total_weights, "hessians": len(fams),
                   "hessian_rows": sorted({r for _d, r, _k in fams.values()}),
                   "hessian_sizes": sizes, "containers": containers, "n_iter": 2, "damp": 0.01,
                   "act_order": True, "ef_mode": "exact"},
        "roofline": {"kernel": " / ".join(sorted(set(kernels.values()))), "bound": "mfma",
                     "achieved": ach, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": ach / PEAK_FP32_TFLOPS, "traffic": None, "avg_launch_ms": avg_ms,
                     "launches_per_step": sweep_launches,
                     "sweep_kernel_by_size": {str(d): k for d, k in kernels.items()}},
        "ef": {"ms": ef_ms, "mweights_per_s": ef_mw, "flops_update": ef_flops,
               "sequential_pass": {"factor_ms": fact_ms, "setup": ph[0], "commit": ph[1],
                                   "sweep": ph[2], "repack": ph[3], "decode": ph[4]}},
        "factor": {"ms": fact_ms, "flops": fact_flops,
                   "tflops": fact_flops / (fact_ms * 1e-3) / 1e12,
                   "frac_of_fp64_peak": fact_flops / (fact_ms * 1e-3) / 1e12 / 78.6},
        "hessian": {"ms": hess_ms, "flops": hess_flops,
                    "tflops": hess_flops / (hess_ms * 1e-3) / 1e12,
                    "activations": "f32" if spec["normalize"] else "bf16"},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle on one tensor per class)")
        result["cpu_baseline"] = config_cpu_baseline(spec, W, H, slot, rows_of, len)
        result["gpu_over_cpu"] = ef_mw / result["cpu_baseline"]["value"]
    print(json.dumps(result))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # two warm-up steps: the first step of a process runs its first Hessian and EF
    # launches (slower, whichever size class it hits) and the second still settles
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28,
                    help="decoder layers (28 = the full workload; fewer only for quick checks)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ef-mode", choices=["mfma", "exact"], default="exact",
                    help="cross-block error propagation: MFMA GEMM or the reference's exact order")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 child runs that measure the sweep's HBM bytes "
                         "(roofline.traffic is then null)")
    ap.add_argument("--workload", choices=["ef", *CONFIG_WORKLOADS, "perm-search", "formats",
                                           "gguf", "copy", "sweep-pass", "hessian-power"],
                    default="ef",
                    help="ef: the EF encode + Hessians line (default); single-linear, "
                         "tied-output, llama3-8b-layer: the other benchmark configurations "
                         "(perm_amd.workloads.config_spec); perm-search: the PERM "
                         "space-map search on the GPU objective; formats: every container's "
                         "codec, the linear form and the Hessian storage format; gguf: the "
                         "encode_gguf driver end to end; copy: a plain "
                         "1 GiB device copy, the calibration run for the HBM byte counters; "
                         "sweep-pass: the ef workload's sequential EF pass alone, the run "
                         "the sweep's HBM byte counters are read on; hessian-power: the ef "
                         "workload's Hessian phase on its activations and on constant ones "
                         "(the same kernels: the clock's dependence on the operand data)")
    args = ap.parse_args()
    if args.gpus != 1:
        msg = (f"bench.py runs on one GPU only (got --gpus {args.gpus}); the encoder path "
               f"shards by tensor / row stripe with no exchange between GPUs")
        print(msg, file=sys.stderr)
        print(json.dumps({"metric": METRIC, "error": msg}))
        sys.exit(2)

    # the sweep's HBM bytes, from child rocprofv3 runs started before this process
    # initializes the GPU
    traffic, traffic_detail = None, None
    if (args.workload == "ef" and args.ef_mode == "exact" and not args.no_traffic):
        log("traffic: rocprofv3 FETCH_SIZE / WRITE_SIZE child runs (sweep pass, copy)")
        try:
            traffic, traffic_detail = measure_sweep_traffic(args.layers)
        except Exception as e:  # reported in the line, never fatal for the bench
            traffic_detail = {"error": f"{type(e).__name__}: {e}"}
            log(f"traffic: not measured ({traffic_detail['error']})")

    import torch
    from perm_amd import _lib
    from perm_amd import workloads as wl
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    if args.workload == "sweep-pass":
        sweep_pass_main(args)
        return
    if args.workload in CONFIG_WORKLOADS:
        config_main(args)
        return
    if args.workload == "perm-search":
        perm_main(args)
        return
    if args.workload == "copy":
        copy_main(args)
        return
    if args.workload == "hessian-power":
        hessian_power_main(args)
        return
    if args.workload == "formats":
        formats_main(args)
        return
    if args.workload == "gguf":
        gguf_main(args)
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
        outs = ef_phase(W, H, slot, layers, mode)
        ee.record()
        del outs  # released after the end mark: freeing the outputs is the caller's work
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

    # after the timed region: one sequential EF pass with per-phase timing. One untimed
    # pass first: the sequential pass allocates on the caller's stream, where the timed
    # steps left no cached blocks of its sizes, and a first hipMalloc of several GB takes
    # tens of milliseconds of host time that its residual phase would otherwise absorb
    import ctypes
    for d in sorted(H, reverse=True):
        ef_phase(W, {d: H[d]}, slot, layers, mode, concurrent=False)
    torch.cuda.synchronize()
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    lib.cp_ef_profile(1)
    p0.record()
    phases, kernels = [], {}
    for d in sorted(H, reverse=True):
        ef_phase(W, {d: H[d]}, slot, layers, mode, concurrent=False)
        kernels[d] = last_sweep_kernel(lib)
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
    outs = ef_phase(W, H, slot, layers, other)
    o1.record()
    del outs
    torch.cuda.synchronize()
    other_ms = o0.elapsed_time(o1)

    hess_ms = sum(hs.elapsed_time(he) for hs, he, _ in marks) / args.steps
    ef_ms = sum(he.elapsed_time(ee) for _, he, ee in marks) / args.steps
    ph = [sum(p[k] for p in phases) for k in range(5)]
    ms_per_step = wall * 1e3 / args.steps
    ef_mw = total_weights / (ef_ms * 1e-3) / 1e6
    hess_tflops = hess_flops / (hess_ms * 1e-3) / 1e12

    # dominant kernel of the line's value (EF throughput): the EF sweep. The Hessian
    # kernel, timed outside the EF window, reports its own fraction of the bf16 peak
    # in the "hessian" object.
    sweep_launches = 2 * len(H)  # sequential pass: two iterations per size class
    avg_ms = ph[2] / sweep_launches
    flops_per_launch = ef_flops / sweep_launches
    ach = flops_per_launch / (avg_ms * 1e-3) / 1e12
    roof = {"kernel": ("ef_sweep_mfma_kernel" if mode == _lib.CP_EF_MFMA
                       else " / ".join(sorted(set(kernels.values())))),
            "bound": "mfma", "achieved": ach,
            "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": ach / PEAK_FP32_TFLOPS,
            "traffic": traffic, "avg_launch_ms": avg_ms,
            "launches_per_step": sweep_launches}
    if mode == _lib.CP_EF_EXACT:
        roof["sweep_kernel_by_size"] = {str(d): k for d, k in kernels.items()}
    if traffic_detail is not None:
        roof["traffic_detail"] = traffic_detail

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
