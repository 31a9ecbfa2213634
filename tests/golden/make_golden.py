"""Write the k-quant golden byte vectors from the reference encoder.

Run once, in a container that holds the reference checkout (it is read from
/root/reference; nothing else in this repository reads that path):

    python tests/golden/make_golden.py

The reference's coldpress/kquant.py depends on numpy only, so it is loaded
straight from its file with importlib; no other reference module is touched.
Only its outputs are committed (``kquant_golden.npz``): inputs this script
synthesises, the container bytes the reference encoders produce for them, the
reference decoders' reconstructions, and the outputs of the four sub-block
fitting routines on random inputs (kquant.py:42-235), so that a mismatch in the
bytes can be traced to the routine that caused it.

The inputs cover the edge cases a bit-exact encoder has to get right: dead
(all-zero / constant) sub-blocks, a lone outlier, sign-only blocks, |x| ties
between +v and -v (first-index argmax), magnitudes whose fp16 scale is
subnormal, underflows to 0 or overflows to inf, -0.0 entries, and an
importance vector with zeros.
"""
import importlib.util
import os
import sys

import numpy as np

REF = "/root/reference/coldpress/kquant.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kquant_golden.npz")
F32 = np.float32
TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]


def load_reference():
    spec = importlib.util.spec_from_file_location("reference_kquant", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def heavy(nrow, n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((nrow, n)) ** 3).astype(F32)
    x *= rng.uniform(0.2, 3.0, size=(nrow, 1)).astype(F32)
    return x


def linear_like(nrow, n, seed):
    """Rows like a random-init Linear: N(0, 0.02^2) times a log-normal row scale."""
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, 0.02, size=(nrow, n)) * np.exp(rng.normal(0.0, 0.5, size=(nrow, 1)))
    return w.astype(F32)


def edge_row():
    """One row of 16 superblocks, each an edge case."""
    rng = np.random.default_rng(11)
    sbs = []
    sbs.append(np.zeros(256))                                   # all zero
    sbs.append(np.full(256, 0.37))                              # constant positive
    sbs.append(np.full(256, -1.25))                             # constant negative
    z = np.zeros(256); z[77] = 3.0; sbs.append(z)               # lone outlier
    sbs.append(-np.abs(rng.standard_normal(256)))               # negative only
    t = rng.standard_normal(256)                                # +v / -v ties in |x|
    for s in range(16):
        t[16 * s + 3] = 2.5; t[16 * s + 9] = -2.5
    for s in range(8):
        t[32 * s + 20] = -4.0; t[32 * s + 21] = 4.0
    sbs.append(t)
    sbs.append(rng.standard_normal(256) * 1e-6)                 # fp16 subnormal scales
    sbs.append(rng.standard_normal(256) * 1e-9)                 # fp16 scale underflow
    sbs.append(rng.standard_normal(256) * 2e6)                  # fp16 scale overflow
    sbs.append(np.repeat(rng.standard_normal(16), 16))          # constant per sub-block
    m = rng.standard_normal(256); m[::2] = 0.0; sbs.append(m)   # half zeros
    nz = rng.standard_normal(256); nz[rng.random(256) < 0.3] = -0.0; sbs.append(nz)
    sbs.append(np.abs(rng.standard_normal(256)) + 5.0)          # positive, far from 0
    q = np.round(rng.standard_normal(256) * 4) / 4; sbs.append(q)   # on a coarse grid
    s2 = rng.standard_normal(256); s2[:128] = 0.0; sbs.append(s2)   # dead first half
    sbs.append(rng.standard_normal(256) ** 5)                   # very heavy tail
    return np.concatenate(sbs).astype(F32)[None, :]


def importance(n, seed, zeros=False):
    x = np.abs(heavy(1, n, seed))[0] + F32(1e-3)
    if zeros:
        x[::7] = 0.0
    return x.astype(F32)


def main():
    if not os.path.exists(REF):
        sys.exit(f"reference encoder not found at {REF}")
    kq = load_reference()
    inputs = {
        "heavy": heavy(8, 1024, seed=1),
        "linear": linear_like(16, 1024, seed=0),
        "edge": edge_row(),
    }
    out = {}
    for name, x in inputs.items():
        n = x.shape[1]
        out[f"x/{name}"] = x
        qws = {"ref": None, "imat": importance(n, 3), "imatz": importance(n, 4, zeros=True)}
        for qn, qw in qws.items():
            if qw is not None:
                out[f"qw/{name}/{qn}"] = qw
            for tt in TYPES:
                with np.errstate(all="ignore"):
                    raw = kq.QUANTIZE[tt](x, qw)
                    rec = kq.DEQUANTIZE[tt](raw, n)
                out[f"raw/{name}/{qn}/{tt}"] = raw
                if name != "linear":
                    out[f"rec/{name}/{qn}/{tt}"] = rec.astype(F32)

    # sub-block fitting routines on their own (random sub-blocks, random weights)
    rng = np.random.default_rng(5)
    xs16 = (rng.standard_normal((64, 16)) ** 3).astype(F32)
    xs32 = (rng.standard_normal((64, 32)) ** 3).astype(F32)
    w16 = np.abs(rng.standard_normal((64, 16))).astype(F32) + F32(0.01)
    w32 = np.abs(rng.standard_normal((64, 32))).astype(F32) + F32(0.01)
    pos16 = np.abs(xs16)
    out["fit/x16"], out["fit/x32"], out["fit/w16"], out["fit/w32"] = xs16, xs32, w16, w32
    with np.errstate(all="ignore"):
        for tag, args in {
            "qkx_q2ref": (xs16, np.abs(xs16), 3, -0.5, 0.1, 15, True, False),
            "qkx_q2imp": (xs16, w16, 3, -0.9, 0.05, 36, False, True),
            "qkx_q4ref": (xs32, w32, 15, -1.0, 0.1, 20, False, False),
            "qkx_q4imp": (xs32, w32, 15, -0.9, 0.05, 36, False, True),
        }.items():
            s, m, L = kq.make_qkx_quants(*args)
            out[f"fit/{tag}/scale"], out[f"fit/{tag}/min"], out[f"fit/{tag}/L"] = s, m, L
        for tag, (xx, ww, nm) in {"qx4w": (xs16, w16, 4), "qx32": (xs16, None, 32),
                                  "qx32w": (xs16, w16, 32)}.items():
            s, L = kq.make_qx_quants(xx, ww, nm)
            out[f"fit/{tag}/scale"], out[f"fit/{tag}/L"] = s, L
        s, L = kq.make_q3_quants(xs16, 4)
        out["fit/q3/scale"], out["fit/q3/L"] = s, L
        for tag, nm in {"qp15": 15, "qp63": 63}.items():
            d, L = kq.make_qp_quants(pos16, w16, nm)
            out[f"fit/{tag}/d"], out[f"fit/{tag}/L"] = d, L
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
