"""k-quant codec oracle (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates the encoders and decoders of coldpress/kquant.py (the reference's own
numpy re-implementation of the llama.cpp k-quant containers). The restatement
is bit-exact with the reference, which requires reproducing its float32
arithmetic step for step:

* every reduction is a numpy ``sum(axis, dtype=float32)`` over an axis of the
  same length as in the reference, so numpy's pairwise summation order (8
  interleaved accumulators for 8 <= n <= 128, halving split above) is the same;
* products associate left to right exactly as the reference writes them;
* no fused multiply-add; division and sqrt are correctly rounded (numpy).

Pinned by the golden byte vectors in tests/golden/kquant_golden.npz, written by
tests/golden/make_golden.py from the reference encoder itself. The linear form of
scale_tune.py (linear_parts / linear_reconstruct) is pinned by its exact identity with
those golden-pinned decoders (tests/test_oracle_kquant.py).
"""
import numpy as np

F32 = np.float32
QK_K = 256
EPS_GROUP = F32(1e-15)                       # kquant.py:18
MAGIC = F32(12582912.0)                      # 1.5 * 2**23

# kquant.py:21-22
BYTES_PER_SB = {"Q2_K": 84, "Q3_K": 110, "Q4_K": 144, "Q5_K": 176, "Q6_K": 210}
SUB_W = {"Q2_K": 16, "Q3_K": 16, "Q4_K": 32, "Q5_K": 32, "Q6_K": 16}


# ------------------------------------------------------------------ scalars

def rint_magic(v):
    """Round half to even through the float32 magic-number add (kquant.py:25-28).

    The low 23 mantissa bits of (v + 1.5*2**23) minus 2**22. Exact for |v| < 2**22;
    outside that range the result is the same deterministic bit pattern garbage
    as the reference (callers clip)."""
    s = np.ascontiguousarray(v, dtype=F32) + MAGIC
    return (s.view(np.int32) & 0x7FFFFF) - 0x400000


def half_bits(v):
    """float32 -> float16, round to nearest even (kquant.py:36-37)."""
    return np.asarray(v, dtype=F32).astype(np.float16)


def half_round(v):
    """float32 -> float16 -> float32 (kquant.py:31-33)."""
    return half_bits(v).astype(F32)


def _fsum(a, axis=-1):
    return a.sum(axis, dtype=F32)


def _first_absmax(x):
    """(index, |x| at it, signed x at it) of the first largest |x| along axis 1."""
    ax = np.abs(x)
    i = ax.argmax(1)
    rows = np.arange(x.shape[0])
    return i, ax[rows, i], x[rows, i]


# ------------------------------------------------------------------ sub-block fits

def fit_affine(x, w, nmax, rmin, rdelta, nstep, mad, strict_dead):
    """Weighted affine grid fit x ~ scale*L + min, L in [0, nmax] (kquant.py:42-94).

    The ``make_qkx2`` / ``make_qkx3`` search: an initial fit from the block
    range, then nstep+1 candidate inverse scales (rmin + rdelta*s + nmax)/range,
    each followed by a closed-form weighted least-squares (scale, min); a
    candidate is kept when its weighted error (|.| if ``mad`` else squared) is
    strictly lower. The range is recomputed from the running min each candidate.
    ``strict_dead`` (qkx3) calls a block dead when max <= min instead of ==.
    Returns (scale [NB], -min [NB], L [NB, n] uint8)."""
    x = x.astype(F32)
    w = w.astype(F32)
    hi = x.max(1)
    lo = np.minimum(x.min(1), F32(0))
    sw = _fsum(w)
    swx = _fsum(w * x)
    dead = (hi <= lo) if strict_dead else (hi == lo)

    def err(scale, off, Lf):
        r = scale[:, None] * Lf + off[:, None] - x
        r = np.abs(r) if mad else r * r
        return _fsum(w * r)

    inv = F32(nmax) / np.where(dead, F32(1), hi - lo)
    scale = F32(1) / inv
    L = np.clip(rint_magic(inv[:, None] * (x - lo[:, None])), 0, nmax)
    best = err(scale, lo, L.astype(F32))
    for step in range(nstep + 1):
        rng_ = hi - lo
        rng_ = np.where(rng_ > 0, rng_, F32(1))
        inv_c = (F32(rmin) + F32(rdelta) * F32(step) + F32(nmax)) / rng_
        Lc = np.clip(rint_magic(inv_c[:, None] * (x - lo[:, None])), 0, nmax)
        Lf = Lc.astype(F32)
        sl = _fsum(w * Lf)
        sl2 = _fsum(w * Lf * Lf)
        sxl = _fsum(w * Lf * x)
        det = sw * sl2 - sl * sl
        with np.errstate(divide="ignore", invalid="ignore"):
            s_c = (sw * sxl - swx * sl) / det
            m_c = (sl2 * swx - sl * sxl) / det
            s_alt = sxl / sl2
        clamp = m_c > 0
        m_c = np.where(clamp, F32(0), m_c)
        s_c = np.where(clamp, s_alt, s_c)
        e_c = err(s_c, m_c, Lf)
        take = (det > 0) & (e_c < best) & ~dead
        L = np.where(take[:, None], Lc, L)
        best = np.where(take, e_c, best)
        scale = np.where(take, s_c, scale)
        lo = np.where(take, m_c, lo)
    scale = np.where(dead, F32(0), scale)
    L = np.where(dead[:, None], 0, L)
    return scale.astype(F32), (-lo).astype(F32), L.astype(np.uint8)


def fit_signed(x, w, nmax):
    """Symmetric signed fit x ~ scale*L, L in [-nmax, nmax-1] (kquant.py:97-133).

    ``make_qx_quants`` with rmse_type 1: the inverse scale starts at -nmax / (the
    signed value of largest magnitude) and 18 nearby candidates
    -(nmax + 0.1*s)/that, s = +-1..9, are tried; a candidate wins when
    sumlx^2 > best*suml2. Weights are ``w`` or x*x when w is None.
    Returns (scale [NB], L + nmax int32)."""
    x = x.astype(F32)
    _, amax, sext = _first_absmax(x)
    dead = amax < EPS_GROUP
    sext = np.where(dead, F32(1), sext)
    w = (x * x if w is None else w).astype(F32)

    def trial(inv):
        L = np.clip(rint_magic(inv[:, None] * x), -nmax, nmax - 1)
        Lf = L.astype(F32)
        return L, _fsum(w * x * Lf), _fsum(w * Lf * Lf)

    L, slx, sl2 = trial(-F32(nmax) / sext)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(sl2 != 0, slx / sl2, F32(0))
    best = scale * slx
    for s in [*range(-9, 0), *range(1, 10)]:
        Lc, slx_c, sl2_c = trial(-(F32(nmax) + F32(0.1) * F32(s)) / sext)
        take = (sl2_c > 0) & (slx_c * slx_c > best * sl2_c) & ~dead
        with np.errstate(divide="ignore", invalid="ignore"):
            s_c = slx_c / sl2_c
        L = np.where(take[:, None], Lc, L)
        scale = np.where(take, s_c, scale)
        best = np.where(take, s_c * slx_c, best)
    scale = np.where(dead, F32(0), scale)
    L = np.where(dead[:, None], 0, L)
    return scale.astype(F32), (L + nmax).astype(np.int32)


def _descend(x, w, L, slx, sl2, lo, hi, active, signed):
    """Coordinate descent on the codes of a fixed-grid fit, in element order.

    Up to 5 sweeps; in each, element i may move to
    rint(x_i * sl2' / slx') (sums without element i) when that raises
    sumlx^2/suml2 (cross-multiplied); a block stops after a sweep with no move.
    ``signed`` selects the make_q3_quants variant (kquant.py:152-174: condition
    slx' > 0, acceptance also needs the new suml2 > 0, codes clipped to
    [lo, hi]) versus make_qp_quants (kquant.py:208-230: condition slx' > 0 and
    sl2' > 0, codes only capped at hi)."""
    n = x.shape[1]
    for _ in range(5):
        moved = np.zeros(x.shape[0], bool)
        for i in range(n):
            wi, xi, Li = w[:, i], x[:, i], L[:, i]
            slx_o = slx - wi * xi * Li
            sl2_o = sl2 - wi * Li * Li
            ok = (slx_o > 0) & active if signed else (slx_o > 0) & (sl2_o > 0) & active
            with np.errstate(divide="ignore", invalid="ignore"):
                q = rint_magic(xi * sl2_o / np.where(slx_o == 0, F32(1), slx_o))
            q = (np.clip(q, lo, hi) if signed else np.minimum(q, hi)).astype(F32)
            slx_n = slx_o + wi * xi * q
            sl2_n = sl2_o + wi * q * q
            better = slx_n * slx_n * sl2 > slx * slx * sl2_n
            take = ok & (q != Li) & better
            if signed:
                take &= sl2_n > 0
            L[:, i] = np.where(take, q, Li)
            slx = np.where(take, slx_n, slx)
            sl2 = np.where(take, sl2_n, sl2)
            moved |= take
        active &= moved
        if not active.any():
            break
    return L, slx, sl2


def fit_signed_descent(x, nmax=4):
    """make_q3_quants (kquant.py:136-179): signed fit with x*x weights, then
    coordinate descent. Returns (scale [NB], L + nmax int32)."""
    x = x.astype(F32)
    _, amax, sext = _first_absmax(x)
    dead = amax < EPS_GROUP
    sext = np.where(dead, F32(1), sext)
    inv = -F32(nmax) / sext
    L = np.clip(rint_magic(inv[:, None] * x), -nmax, nmax - 1).astype(F32)
    w = x * x
    slx = _fsum(w * x * L)
    sl2 = _fsum(w * L * L)
    L, slx, sl2 = _descend(x, w, L, slx, sl2, -nmax, nmax - 1, ~dead, signed=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(sl2 > 0, slx / sl2, F32(0))
    scale = np.where(dead, F32(0), scale)
    L = np.where(dead[:, None], F32(0), L)
    return scale.astype(F32), L.astype(np.int32) + nmax


def fit_nonneg(x, w, nmax):
    """make_qp_quants (kquant.py:182-235): quantize non-negative super-block
    scales to [0, nmax]. The first candidate's error uses the UNclamped codes;
    8 candidates (0.1*s + nmax)/max, s = +-1..4; then coordinate descent.
    Returns (d [NB], L [NB, n] uint8)."""
    x = x.astype(F32)
    w = w.astype(F32)
    top = x.max(1)
    dead = top < EPS_GROUP
    top = np.where(dead, F32(1), top)
    inv = F32(nmax) / top
    L0 = rint_magic(inv[:, None] * x).astype(F32)
    r = x - (F32(1) / inv)[:, None] * L0
    best = _fsum(w * r * r)
    for s in [*range(-4, 0), *range(1, 5)]:
        inv_c = (F32(0.1) * F32(s) + F32(nmax)) / top
        Lc = np.minimum(rint_magic(inv_c[:, None] * x), nmax).astype(F32)
        r = x - (F32(1) / inv_c)[:, None] * Lc
        e_c = _fsum(w * r * r)
        take = (e_c < best) & ~dead
        best = np.where(take, e_c, best)
        inv = np.where(take, inv_c, inv)
    L = np.minimum(rint_magic(inv[:, None] * x), nmax).astype(F32)
    slx = _fsum(w * x * L)
    sl2 = _fsum(w * L * L)
    L, slx, sl2 = _descend(x, w, L, slx, sl2, None, nmax, ~dead, signed=False)
    with np.errstate(divide="ignore", invalid="ignore"):
        d = np.where(sl2 > 0, slx / sl2, F32(0))
    d = np.where(dead, F32(0), d)
    L = np.where(dead[:, None], F32(0), L)
    return d.astype(F32), L.astype(np.uint8)


# ------------------------------------------------------------------ bit layouts
# Element e of a superblock sits in these fields (ggml block_q*_K layouts,
# restated from kquant.py:240-342 and the Q6_K packer at :664-672).

def _spread(L, quarter):
    """[NB, 256] -> [NB, 2, 4, quarter]: half h, lane-group g holds elements
    h*128 + g*32 + l (quarter = 32) -- the shared 2-bit / 6-bit interleave."""
    return L.reshape(L.shape[0], 2, 4, quarter)


def pack_2bit(L):
    """Codes 0..3 -> 64 bytes: byte h*32+l = sum_g L[h*128+g*32+l] << 2g (kquant.py:240-249)."""
    s = _spread(L.astype(np.uint8), 32)
    return (s[:, :, 0] | s[:, :, 1] << 2 | s[:, :, 2] << 4 | s[:, :, 3] << 6).reshape(-1, 64)


def unpack_2bit(qs):
    q = qs.reshape(-1, 2, 1, 32)
    return ((q >> (2 * np.arange(4, dtype=np.uint8))[None, None, :, None]) & 3).reshape(-1, 256)


def pack_nibbles(L):
    """Codes 0..15 -> 128 bytes: chunk c (64 elements) byte c*32+l = L[c*64+l] | L[c*64+32+l] << 4
    (kquant.py:325-332)."""
    s = L.astype(np.uint8).reshape(-1, 4, 2, 32)
    return ((s[:, :, 0] & 0xF) | (s[:, :, 1] & 0xF) << 4).reshape(-1, 128)


def unpack_nibbles(qs):
    b = qs.reshape(-1, 4, 1, 32)
    return np.concatenate([b & 0xF, b >> 4], axis=2).reshape(-1, 256)


def pack_scales_q3(Ls):
    """16 six-bit scales -> 12 bytes (kquant.py:264-276): low nibbles of scales
    0..7 / 8..15 in bytes 0..7 (low / high nibble), the top two bits of scale j
    at bits 2*(j//4) of byte 8 + j%4."""
    l = Ls.astype(np.uint8)
    out = np.zeros((l.shape[0], 12), np.uint8)
    out[:, 0:8] = (l[:, 0:8] & 0xF) | ((l[:, 8:16] & 0xF) << 4)
    for j in range(16):
        out[:, 8 + j % 4] |= (l[:, j] >> 4) << (2 * (j // 4))
    return out


def unpack_scales_q3(sc):
    """12 bytes -> 16 scales 0..63 int32 (subtract 32 for the signed value)."""
    j = np.arange(16)
    lo = np.where(j < 8, sc[:, j % 8] & 0xF, sc[:, j % 8] >> 4).astype(np.int32)
    hi = ((sc[:, 8 + j % 4] >> (2 * (j // 4))) & 3).astype(np.int32)
    return lo | hi << 4


def pack_scales_k4(Ls, Lm):
    """8 six-bit scales and 8 mins -> 12 bytes (kquant.py:293-307,
    ggml get_scale_min_k4 layout)."""
    s = Ls.astype(np.uint8)
    m = Lm.astype(np.uint8)
    out = np.zeros((s.shape[0], 12), np.uint8)
    out[:, 0:4] = s[:, 0:4] | (s[:, 4:8] >> 4) << 6
    out[:, 4:8] = m[:, 0:4] | (m[:, 4:8] >> 4) << 6
    out[:, 8:12] = (s[:, 4:8] & 0xF) | (m[:, 4:8] & 0xF) << 4
    return out


def unpack_scales_k4(sc):
    """12 bytes -> (scales [NB, 8], mins [NB, 8]) int32 0..63."""
    s = np.empty((sc.shape[0], 8), np.int32)
    m = np.empty((sc.shape[0], 8), np.int32)
    s[:, 0:4] = sc[:, 0:4] & 63
    m[:, 0:4] = sc[:, 4:8] & 63
    s[:, 4:8] = (sc[:, 8:12] & 0xF) | (sc[:, 0:4] >> 6) << 4
    m[:, 4:8] = (sc[:, 8:12] >> 4) | (sc[:, 4:8] >> 6) << 4
    return s, m


def pack_q3_codes(L):
    """Codes 0..7 -> (hmask [NB,32], qs [NB,64]): bit j of hmask[l] is the high
    bit of element 32j + l; the low two bits go through pack_2bit (kquant.py:474-483)."""
    L = L.astype(np.int32)
    high = (L > 3).astype(np.uint8).reshape(-1, 8, 32)
    hmask = np.bitwise_or.reduce(high << np.arange(8, dtype=np.uint8)[None, :, None], axis=1)
    return hmask, pack_2bit(np.where(L > 3, L - 4, L))


def unpack_q3_codes(hmask, qs):
    """-> signed codes -4..3: low bits minus 4 where the high bit is clear."""
    lo = unpack_2bit(qs).astype(np.int32)
    hb = ((hmask[:, None, :] >> np.arange(8, dtype=np.uint8)[None, :, None]) & 1).reshape(-1, 256)
    return lo - np.where(hb == 0, 4, 0)


def pack_q6_codes(L):
    """Codes 0..63 -> (ql [NB,128], qh [NB,64]) (kquant.py:664-672)."""
    s = _spread(L.astype(np.uint8), 32)
    ql = np.concatenate([(s[:, :, 0] & 0xF) | (s[:, :, 2] & 0xF) << 4,
                         (s[:, :, 1] & 0xF) | (s[:, :, 3] & 0xF) << 4], axis=2).reshape(-1, 128)
    qh = (s[:, :, 0] >> 4 | (s[:, :, 1] >> 4) << 2 | (s[:, :, 2] >> 4) << 4
          | (s[:, :, 3] >> 4) << 6).reshape(-1, 64)
    return ql, qh


def unpack_q6_codes(ql, qh):
    a = ql.reshape(-1, 2, 2, 32)
    h = qh.reshape(-1, 2, 1, 32)
    low = np.stack([a[:, :, 0] & 0xF, a[:, :, 1] & 0xF, a[:, :, 0] >> 4, a[:, :, 1] >> 4], axis=2)
    high = (h >> (2 * np.arange(4, dtype=np.uint8))[None, None, :, None]) & 3
    return (low.astype(np.int32) | high.astype(np.int32) << 4).reshape(-1, 256)


def pack_q5_codes(L):
    """Codes 0..31 -> (qh [NB,32], qs [NB,128]): bit 2c of qh[l] is the high bit of
    element 64c + l, bit 2c+1 that of element 64c + 32 + l; the low four bits go
    through pack_nibbles (kquant.py:572-583)."""
    L = L.astype(np.int32)
    high = (L > 15).astype(np.uint8).reshape(-1, 4, 2, 32)
    sh = (2 * np.arange(4, dtype=np.uint8))[None, :, None]
    qh = np.bitwise_or.reduce((high[:, :, 0] << sh) | (high[:, :, 1] << (sh + 1)), axis=1)
    return qh, pack_nibbles(np.where(L > 15, L - 16, L))


def unpack_q5_codes(qh, qs):
    """-> codes 0..31 int32."""
    h = qh.reshape(-1, 1, 32)
    sh = (2 * np.arange(4))[None, :, None]
    hb = np.stack([(h >> sh) & 1, (h >> (sh + 1)) & 1], axis=2).reshape(-1, 256)
    return unpack_nibbles(qs).astype(np.int32) + 16 * hb.astype(np.int32)


def stored_codes(tt, raw):
    """Integer codes of every superblock [NB, 256] in the sweep's signed convention
    (Q3_K -4..3, Q6_K -32..31, the affine types 0..top)."""
    b = raw.reshape(-1, BYTES_PER_SB[tt])
    if tt == "Q2_K":
        return unpack_2bit(b[:, 16:80]).astype(np.int32)
    if tt == "Q3_K":
        return unpack_q3_codes(b[:, 0:32], b[:, 32:96])
    if tt == "Q4_K":
        return unpack_nibbles(b[:, 16:144]).astype(np.int32)
    if tt == "Q5_K":
        return unpack_q5_codes(b[:, 16:48], b[:, 48:176])
    if tt == "Q6_K":
        return unpack_q6_codes(b[:, 0:128], b[:, 128:192]) - 32
    raise ValueError(tt)


def _half_field(b, off):
    return b[:, off:off + 2].copy().view(np.float16).astype(F32).reshape(-1)


# ------------------------------------------------------------------ encoders

def _blocks(x):
    nrow, n = x.shape
    if n % QK_K:
        raise AssertionError(f"row length {n} is not a multiple of {QK_K}")
    return x.reshape(-1, QK_K).astype(F32)


def _imatrix_weights(xb, qw, sub, k):
    """Importance weights qw * sqrt(k*sum(x^2)/256 + x^2), per element, as [NB, 256/sub, sub]
    (kquant.py:380-383, :453-455, :537-539; k = 1 for Q2_K, 2 otherwise)."""
    NB = xb.shape[0]
    qwb = np.broadcast_to(np.asarray(qw, F32), (NB * QK_K // qw.shape[-1], qw.shape[-1]))
    qwb = qwb.reshape(NB, QK_K // sub, sub)
    sx2 = _fsum(xb * xb, 1)
    var = (sx2 if k == 1 else F32(k) * sx2) / F32(QK_K)
    xs = xb.reshape(NB, QK_K // sub, sub)
    return qwb * np.sqrt(var[:, None, None] + xs * xs)


def _requant_affine(xb, dl, ml, L, sub, top):
    """Codes on the committed grid where dl != 0, old codes elsewhere (kquant.py:399-405)."""
    dle = np.repeat(dl, sub, axis=1)
    mle = np.repeat(ml, sub, axis=1)
    nz = dle != 0
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.clip(rint_magic((xb + mle) / np.where(nz, dle, F32(1))), 0, top)
    return np.where(nz, q, L)


def _superscale_ref(v, top):
    """ref-path super-scale: codes rint(top/max * v) where max > 0 (kquant.py:364-374)."""
    vmax = v.max(1)
    pos = vmax > 0
    inv = np.where(pos, F32(top) / np.where(pos, vmax, F32(1)), F32(0))
    code = np.where(pos[:, None], rint_magic(inv[:, None] * v), 0)
    return code, np.where(pos, vmax / F32(top), F32(0))


def encode_q2k(x, qw=None):
    """Q2_K: 16 sub-blocks of 16, 2-bit codes, 4-bit scale and min, fp16 d/dmin,
    84 bytes per superblock (kquant.py:347-413)."""
    nrow = x.shape[0]
    xb = _blocks(x)
    NB = xb.shape[0]
    xs = xb.reshape(-1, 16)
    if qw is None:
        scale, mins, L = fit_affine(xs, np.abs(xs), 3, -0.5, 0.1, 15, True, False)
        sc_i, d = _superscale_ref(scale.reshape(NB, 16), 15)
        mn_i, dmin = _superscale_ref(mins.reshape(NB, 16), 15)
    else:
        wt = _imatrix_weights(xb, qw, 16, 1)
        scale, mins, L = fit_affine(xs, wt.reshape(-1, 16), 3, -0.9, 0.05, 36, False, True)
        swt = _fsum(wt, 2)
        d, Ls = fit_nonneg(scale.reshape(NB, 16), swt, 15)
        dmin, Lm = fit_nonneg(mins.reshape(NB, 16), swt, 15)
        sc_i, mn_i = Ls.astype(np.int32), Lm.astype(np.int32)
    d16, dmin16 = half_bits(d), half_bits(dmin)
    dl = d16.astype(F32)[:, None] * sc_i.astype(F32)
    ml = dmin16.astype(F32)[:, None] * mn_i.astype(F32)
    L = _requant_affine(xb, dl, ml, L.reshape(NB, 256), 16, 3)
    out = np.empty((NB, 84), np.uint8)
    out[:, 0:16] = (sc_i.astype(np.uint8) & 0xF) | (mn_i.astype(np.uint8) & 0xF) << 4
    out[:, 16:80] = pack_2bit(L)
    out[:, 80:82] = d16.view(np.uint8).reshape(NB, 2)
    out[:, 82:84] = dmin16.view(np.uint8).reshape(NB, 2)
    return out.reshape(nrow, -1)


def decode_q2k(raw, n):
    b = raw.reshape(-1, 84)
    d, dmin = _half_field(b, 80), _half_field(b, 82)
    dl = d[:, None] * (b[:, 0:16] & 0xF).astype(F32)
    ml = dmin[:, None] * (b[:, 0:16] >> 4).astype(F32)
    L = unpack_2bit(b[:, 16:80]).astype(F32)
    return (np.repeat(dl, 16, 1) * L - np.repeat(ml, 16, 1)).reshape(raw.shape[0], n)


def encode_q3k(x, qw=None):
    """Q3_K: 16 sub-blocks of 16, 3-bit signed codes (hmask + 2 bits), 6-bit
    signed scales, fp16 d, 110 bytes per superblock (kquant.py:432-486)."""
    nrow = x.shape[0]
    xb = _blocks(x)
    NB = xb.shape[0]
    xs = xb.reshape(-1, 16)
    if qw is None:
        scale, L = fit_signed_descent(xs, 4)
        scales = scale.reshape(NB, 16)
        _, _, smax = _first_absmax(scales)
        nz = smax != 0
        inv = np.where(nz, F32(-32) / np.where(nz, smax, F32(1)), F32(0))
        Ls = np.where(nz[:, None], np.clip(rint_magic(inv[:, None] * scales), -32, 31) + 32, 0)
        with np.errstate(divide="ignore"):
            d = np.where(nz, F32(1) / inv, F32(0))
        d = np.where(nz & np.isfinite(d), d, F32(0))
    else:
        wt = _imatrix_weights(xb, qw, 16, 2)
        scale, L = fit_signed(xs, wt.reshape(-1, 16), 4)
        d, Ls = fit_signed(scale.reshape(NB, 16), _fsum(wt, 2), 32)
    packed = pack_scales_q3(Ls.astype(np.int32))
    d16 = half_bits(d)
    dsub = np.repeat(d16.astype(F32)[:, None] * (unpack_scales_q3(packed) - 32).astype(F32), 16, 1)
    nz = dsub != 0
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.clip(rint_magic(xb / np.where(nz, dsub, F32(1))), -4, 3) + 4
    L = np.where(nz, q, L.reshape(NB, 256).astype(np.int32))
    hmask, qs = pack_q3_codes(L)
    out = np.empty((NB, 110), np.uint8)
    out[:, 0:32] = hmask
    out[:, 32:96] = qs
    out[:, 96:108] = packed
    out[:, 108:110] = d16.view(np.uint8).reshape(NB, 2)
    return out.reshape(nrow, -1)


def decode_q3k(raw, n):
    b = raw.reshape(-1, 110)
    d = _half_field(b, 108)
    dl = d[:, None] * (unpack_scales_q3(b[:, 96:108]) - 32).astype(F32)
    q = unpack_q3_codes(b[:, 0:32], b[:, 32:96]).astype(F32)
    return (np.repeat(dl, 16, 1) * q).reshape(raw.shape[0], n)


def _encode_q45(x, qw, q5):
    """Q4_K / Q5_K: 8 sub-blocks of 32, 6-bit scale and min, fp16 d/dmin
    (kquant.py:508-585)."""
    nrow = x.shape[0]
    top = 31 if q5 else 15
    xb = _blocks(x)
    NB = xb.shape[0]
    xs = xb.reshape(NB, 8, 32)
    if qw is None:
        w = np.sqrt(_fsum(xs * xs, 2) / F32(32))[:, :, None] + np.abs(xs)
        rmin, rdelta, nstep = (-0.5, 0.1, 15) if q5 else (-1.0, 0.1, 20)
        scale, mins, L = fit_affine(xs.reshape(-1, 32), w.reshape(-1, 32),
                                    top, rmin, rdelta, nstep, False, False)
        scales, mins = scale.reshape(NB, 8), mins.reshape(NB, 8)
        smax, mmax = scales.max(1), mins.max(1)
        inv_s = np.where(smax > 0, F32(63) / np.where(smax > 0, smax, F32(1)), F32(0))
        inv_m = np.where(mmax > 0, F32(63) / np.where(mmax > 0, mmax, F32(1)), F32(0))
        # the int -> uint8 narrowing wraps before the cap at 63 (kquant.py:530-532)
        Ls = np.minimum(rint_magic(inv_s[:, None] * scales).astype(np.uint8), 63)
        Lm = np.minimum(rint_magic(inv_m[:, None] * mins).astype(np.uint8), 63)
        d, dmin = smax / F32(63), mmax / F32(63)
    else:
        wt = _imatrix_weights(xb, qw, 32, 2)
        scale, mins, L = fit_affine(xs.reshape(-1, 32), wt.reshape(-1, 32),
                                    top, -0.9, 0.05, 36, False, True)
        swt = _fsum(wt, 2)
        d, Ls = fit_nonneg(scale.reshape(NB, 8), swt, 63)
        dmin, Lm = fit_nonneg(mins.reshape(NB, 8), swt, 63)
        if q5:
            Ls, Lm = np.minimum(Ls, 63), np.minimum(Lm, 63)
    d16, dmin16 = half_bits(d), half_bits(dmin)
    packed = pack_scales_k4(Ls, Lm)
    su, mu = unpack_scales_k4(packed)
    dl = d16.astype(F32)[:, None] * su.astype(F32)
    ml = dmin16.astype(F32)[:, None] * mu.astype(F32)
    L = _requant_affine(xb, dl, ml, L.reshape(NB, 256), 32, top).astype(np.uint8)
    head = np.concatenate([d16.view(np.uint8).reshape(NB, 2),
                           dmin16.view(np.uint8).reshape(NB, 2), packed], axis=1)
    if not q5:
        return np.concatenate([head, pack_nibbles(L)], axis=1).reshape(nrow, -1)
    qh, body = pack_q5_codes(L)
    return np.concatenate([head, qh, body], axis=1).reshape(nrow, -1)


def encode_q4k(x, qw=None):
    """Q4_K: 144 bytes per superblock (kquant.py:588-589)."""
    return _encode_q45(x, qw, False)


def encode_q5k(x, qw=None):
    """Q5_K: 176 bytes per superblock (kquant.py:592-593)."""
    return _encode_q45(x, qw, True)


def _decode_q45(raw, n, q5):
    bp = 176 if q5 else 144
    b = raw.reshape(-1, bp)
    d, dmin = _half_field(b, 0), _half_field(b, 2)
    su, mu = unpack_scales_k4(b[:, 4:16])
    if q5:
        L = unpack_q5_codes(b[:, 16:48], b[:, 48:176])
    else:
        L = unpack_nibbles(b[:, 16:144])
    dl = d[:, None] * su.astype(F32)
    ml = dmin[:, None] * mu.astype(F32)
    return (np.repeat(dl, 32, 1) * L.astype(F32) - np.repeat(ml, 32, 1)).reshape(raw.shape[0], n)


def decode_q4k(raw, n):
    return _decode_q45(raw, n, False)


def decode_q5k(raw, n):
    return _decode_q45(raw, n, True)


def encode_q6k(x, qw=None):
    """Q6_K: 16 sub-blocks of 16, 6-bit signed codes, int8 scales, fp16 d,
    210 bytes per superblock (kquant.py:632-678)."""
    nrow, npr = x.shape
    xb = _blocks(x)
    NB = xb.shape[0]
    xs = xb.reshape(-1, 16)
    w = None if qw is None else np.broadcast_to(np.asarray(qw, F32), (nrow, npr)).reshape(-1, 16)
    scale, L = fit_signed(xs, w, 32)
    scales = scale.reshape(NB, 16)
    _, amax, smax = _first_absmax(scales)
    dead = amax < EPS_GROUP
    inv = F32(-128) / np.where(dead, F32(1), smax)
    d = F32(1) / inv
    sc_i = np.minimum(rint_magic(inv[:, None] * scales), 127).astype(np.int8)
    d16 = half_bits(np.where(dead, F32(0), d))
    dsub = np.repeat(d16.astype(F32)[:, None] * sc_i.astype(F32), 16, 1)
    nz = (dsub != 0) & ~dead[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.clip(rint_magic(xb / np.where(nz, dsub, F32(1))), -32, 31) + 32
    L = np.where(nz, q, L.reshape(NB, 256))
    L = np.where(dead[:, None], 0, L).astype(np.uint8)
    sc_i = np.where(dead[:, None], np.int8(0), sc_i)
    ql, qh = pack_q6_codes(L)
    out = np.empty((NB, 210), np.uint8)
    out[:, 0:128] = ql
    out[:, 128:192] = qh
    out[:, 192:208] = sc_i.view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(NB, 2)
    return out.reshape(nrow, -1)


def decode_q6k(raw, n):
    b = raw.reshape(-1, 210)
    d = _half_field(b, 208)
    sc = b[:, 192:208].copy().view(np.int8).astype(np.int32)
    q = (unpack_q6_codes(b[:, 0:128], b[:, 128:192]) - 32).astype(F32)
    dl = d[:, None] * np.repeat(sc, 16, 1).astype(F32)
    return (dl * q).reshape(raw.shape[0], n)


def encode_q80(x, qw=None):
    """Q8_0: blocks of 32, int8 codes rounded half away from zero, fp16 d
    (kquant.py:706-718)."""
    nrow = x.shape[0]
    xb = x.reshape(-1, 32).astype(F32)
    d = np.abs(xb).max(1) / F32(127)
    inv = np.where(d != 0, F32(1) / np.where(d != 0, d, F32(1)), F32(0))
    v = xb * inv[:, None]
    q = np.sign(v) * np.floor(np.abs(v) + F32(0.5))
    out = np.empty((xb.shape[0], 34), np.uint8)
    out[:, 0:2] = half_bits(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:34] = q.astype(np.int8).view(np.uint8)
    return out.reshape(nrow, -1)


def decode_q80(raw, n):
    b = raw.reshape(-1, 34)
    d = _half_field(b, 0)
    return (d[:, None] * b[:, 2:34].copy().view(np.int8).astype(F32)).reshape(raw.shape[0], n)


# ------------------------------------------------------------------ dispatch (kquant.py:732-741)

QUANTIZE = {"Q2_K": encode_q2k, "Q3_K": encode_q3k, "Q4_K": encode_q4k,
            "Q5_K": encode_q5k, "Q6_K": encode_q6k, "Q8_0": encode_q80}
DEQUANTIZE = {"Q2_K": decode_q2k, "Q3_K": decode_q3k, "Q4_K": decode_q4k,
              "Q5_K": decode_q5k, "Q6_K": decode_q6k, "Q8_0": decode_q80}


def roundtrip(x, ttype, qw=None):
    return DEQUANTIZE[ttype](QUANTIZE[ttype](x, qw), x.shape[1])


# ------------------------------------------------------------------ linear form
# coldpress/scale_tune.py:67-173: with the codes fixed, W = d (x) A - dmin (x) B.

_LIN_LAYOUT = {"Q2_K": (80, 82, 16), "Q3_K": (108, None, 16), "Q4_K": (0, 2, 32),
               "Q5_K": (0, 2, 32), "Q6_K": (208, None, 16)}


def linear_parts(raw, tt, n):
    """(d [nrow, n/256], dmin or None, A [nrow, n], B or None) as float32: A the integer
    sub-block scale times the signed code, B the integer sub-block min."""
    d_off, m_off, sub = _LIN_LAYOUT[tt]
    nrow = raw.shape[0]
    b = raw.reshape(-1, BYTES_PER_SB[tt])
    d = _half_field(b, d_off)
    dmin = _half_field(b, m_off) if m_off is not None else None
    q = stored_codes(tt, raw).astype(np.int64)          # signed codes
    if tt == "Q2_K":
        sc, mn = (b[:, 0:16] & 0xF).astype(np.int64), (b[:, 0:16] >> 4).astype(np.int64)
    elif tt == "Q3_K":
        sc, mn = unpack_scales_q3(b[:, 96:108]).astype(np.int64) - 32, None
    elif tt in ("Q4_K", "Q5_K"):
        sc, mn = (v.astype(np.int64) for v in unpack_scales_k4(b[:, 4:16]))
    else:
        sc, mn = b[:, 192:208].copy().view(np.int8).astype(np.int64), None
    A = (np.repeat(sc, sub, 1) * q).astype(F32).reshape(nrow, n)
    B = np.repeat(mn, sub, 1).astype(F32).reshape(nrow, n) if mn is not None else None
    ns = n // QK_K
    return (d.reshape(nrow, ns), dmin.reshape(nrow, ns) if dmin is not None else None, A, B)


def linear_reconstruct(d, dmin, A, B):
    """fl(fl(d*A) - fl(dmin*B)) in float32 (scale_tune.py:162-173)."""
    W = np.repeat(d, QK_K, 1).astype(F32) * A
    if dmin is not None:
        W = W - np.repeat(dmin, QK_K, 1).astype(F32) * B
    return W.astype(F32)
