"""Pins of the oracle's weight quantizers (Q4_K, Q5_K, Q6_K; the ggml_quantize_chunk step of
core/src/quantize.cpp:214, 285) by what the mathematics fixes, without ggml.

The published algorithm (ggml's quantize_row_q4_K_ref / quantize_row_q6_K_ref) fits each sub-block
by searching a fixed grid of candidate scales and keeping the best one. A restatement can get the
grid, the refit or the constraint wrong and still round-trip with a small error, so these tests
check each part by its defining property:
  - make_qkx2_quants (Q4_K, 32 elements, L in [0, 15], x ~ scale*L + min, min <= 0): the result is
    what the search over its 22 candidates gives (the rounding at 15/(max-min), then the 21 grid
    points (-1 + 0.1*is + 15)/(max-min), each refitted by weighted least squares with min <= 0 and
    kept if its weighted squared error is smaller; a kept refit's min offsets the later roundings);
    Q5_K runs the same search with L in [0, 31], 16 grid points (-0.5 + 0.1*is + 31)/(max-min);
  - make_qx_quants (Q6_K, 16 elements, L in [-32, 31], x ~ scale*L): the result is one of the 19
    candidates (-(32 + 0.1*is)/max, is in [-9, 9]) and maximises the x^2-weighted fit quality;
  - the 6-bit scale/min packing inverts exactly under the GGUF decode formula;
  - the final quants are the nearest grid points of the stored scales, and the 6-bit sub-block
    scales the nearest integers of their ratio to the largest.
The searches are recomputed here independently: the candidate roundings with the same fp32
operations, the fits and errors in float64, following both branches wherever fp32 and float64
could decide differently. Planted mistakes in the oracle (a shorter grid, a wider step, no min
clamp, unit weights, a narrower Q6_K grid) must fail these checks.
"""
import numpy as np
import pytest

from densecore_amd import synth

f32 = np.float32


def _subblocks(n, count, seed):
    """Random sub-blocks plus the cases where the constraints bind: all-positive (min clamp), one
    outlier, a constant block, all zero, and tiny values."""
    x = synth.normal(n * count, seed).reshape(count, n).astype(np.float32) * f32(0.02)
    x[0] = np.abs(x[0]) + f32(0.01)            # all positive: min clamps to 0
    x[1] = np.abs(x[1]) * f32(3) + f32(0.05)
    x[2, 5] = f32(0.4)                         # one outlier
    x[3] = f32(0.03)                           # constant
    x[4] = f32(0.0)                            # all zero
    x[5] *= f32(1e-6)                          # tiny
    x[6:40] = np.abs(x[6:40]) + f32(0.002)     # more blocks where the min constraint can bind
    return x


def _clustered(n, count, seed):
    """Tight clusters with one outlier above: the shape where the widest grid point
    (nmax + 1 quanta over the range) wins the Q4_K search."""
    x = synth.normal(n * count, seed).reshape(count, n).astype(np.float32) * f32(0.002)
    top = np.abs(synth.normal(count, seed + 1)).astype(np.float32) * f32(0.01) + f32(0.02)
    x[:, -1] = top
    return x


def _q4k_weights(x):
    av = np.sqrt(np.sum(x.astype(np.float32) * x, dtype=np.float32) / f32(32)).astype(np.float32)
    return (av + np.abs(x)).astype(np.float32)


def _ls_fit_min_le0(x, w, L):
    """argmin over (a, b), b <= 0, of sum w (a L + b - x)^2, in float64; None if degenerate."""
    x, w, L = x.astype(np.float64), w.astype(np.float64), L.astype(np.float64)
    sw, sl, sl2, sx, sxl = w.sum(), (w * L).sum(), (w * L * L).sum(), (w * x).sum(), (w * x * L).sum()
    D = sw * sl2 - sl * sl
    if D <= 0:
        return None
    a = (sw * sxl - sx * sl) / D
    b = (sl2 * sx - sl * sxl) / D
    if b > 0:
        b, a = 0.0, sxl / sl2
    return a, b


def _err(x, w, a, b, L):
    d = a * L.astype(np.float64) + b - x.astype(np.float64)
    return float((w.astype(np.float64) * d * d).sum())


def _roundings(v, lo, hi):
    """The integer vectors clamp(round(v), lo, hi) that fp32 arithmetic could give when each
    element of v is known only to ~1e-6 relative: elements within that of a .5 whose two
    neighbours both survive the clamp may round either way (at most 3 such elements branch)."""
    base = np.clip(np.rint(v), lo, hi).astype(np.int64)
    frac = np.abs(v - np.floor(v) - 0.5)
    near = (frac < 1e-5 * np.maximum(1.0, np.abs(v))) & \
        (np.clip(np.floor(v), lo, hi) != np.clip(np.floor(v) + 1, lo, hi))
    idx = np.flatnonzero(near)[:3]
    out = []
    for bits in range(1 << len(idx)):
        L = base.copy()
        for b, i in enumerate(idx):
            L[i] = int(np.clip(np.floor(v[i]) + ((bits >> b) & 1), lo, hi))
        out.append(L)
    return out


def _qkx2_outcomes(x, w, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20, limit=256):
    """Every result the published grid search can give, restated from its definition: start from
    the rounding at nmax/(max-min) (min = min(x, 0)); for is = 0 .. nstep, round x at
    (rmin + rdelta*is + nmax)/(max - min) relative to the CURRENT min, refit (scale, min <= 0) by
    weighted least squares, and keep the refit (its min then offsets the later roundings) if its
    weighted squared error is smaller. Fits and errors in float64; roundings of fp32 products.
    Where float64 and the C's fp32 could decide differently (a rounding within ~1e-6 of .5 once
    the min is a refit, two different candidates whose errors agree to 1e-5) both branches are
    followed. Returns a list of (scale, min, L), or None if more than `limit` paths arise."""
    mx = f32(x.max())
    mn = min(f32(x.min()), f32(0))
    if mx == mn:
        return [(0.0, float(mn), np.zeros(x.size, dtype=np.int64))]
    iscale = f32(nmax) / f32(mx - mn)
    L0 = np.clip(np.rint((iscale * (x - mn)).astype(np.float32)), 0, nmax).astype(np.int64)
    s0 = float(f32(1) / iscale)
    # a state: (scale, min, L, error, refitted); until a refit is kept the min is fp32 min(x, 0)
    # exactly, as in the C, so its roundings are exact
    states = [(s0, float(mn), L0, _err(x, w, s0, float(mn), L0), False)]
    for is_ in range(nstep + 1):
        nxt = []
        for scale, cur, L, best, refit in states:
            iscale = ((f32(rmin) + f32(rdelta) * f32(is_)) + f32(nmax)) / f32(f32(mx) - f32(cur))
            v = (iscale * (x - f32(cur))).astype(np.float32)
            cands = _roundings(v.astype(np.float64), 0, nmax) if refit else \
                [np.clip(np.rint(v), 0, nmax).astype(np.int64)]
            for La in cands:
                fit = _ls_fit_min_le0(x, w, La)
                if fit is None:
                    nxt.append((scale, cur, L, best, refit))
                    continue
                e = _err(x, w, fit[0], fit[1], La)
                close = not np.array_equal(La, L) and abs(e - best) <= 1e-5 * max(e, best)
                if e < best or close:
                    nxt.append((fit[0], fit[1], La, e, True))
                if e >= best or close:
                    nxt.append((scale, cur, L, best, refit))
        # merge states that agree (same L and fit)
        uniq = {}
        for st in nxt:
            uniq.setdefault((st[2].tobytes(), round(st[0], 12), round(st[1], 12)), st)
        states = list(uniq.values())
        if len(states) > limit:
            return None
    return [(st[0], st[1], st[2]) for st in states]


Q4K_SEARCH = dict(nmax=15, rmin=-1.0, rdelta=0.1, nstep=20)
Q5K_SEARCH = dict(nmax=31, rmin=-0.5, rdelta=0.1, nstep=15)


def _check_qkx2(x, scale, mn, L, search=Q4K_SEARCH):
    """None if (scale, min, L) is a result of the grid search, else the reason it is not."""
    w = _q4k_weights(x)
    nmax = search["nmax"]
    if x.max() == min(x.min(), 0):
        return None if (scale == 0 and np.all(L == 0)) else "constant block"
    if L.min() < 0 or L.max() > nmax:
        return f"L outside [0, {nmax}]"
    if mn > 0:
        return f"min {mn} > 0"
    outs = _qkx2_outcomes(x, w, **search)
    if outs is None:
        return "too many branches"
    match = [o for o in outs if np.array_equal(o[2], L)]
    if not match:
        return "L is not a result of the grid search"
    # the C's fp32 refit against the float64 one: the min suffers cancellation, so its error is
    # judged against the quantization step
    if not any(abs(scale - o[0]) <= 1e-4 * abs(o[0]) + 1e-12 and abs(mn - o[1]) <= 1e-3 * abs(o[0])
               for o in match):
        return f"scale/min ({scale}, {mn}) are not the grid search's fit {[(o[0], o[1]) for o in match]}"
    return None


def _branch_count(x, search=Q4K_SEARCH):
    return [len(_qkx2_outcomes(xb, _q4k_weights(xb), **search) or [0] * 999) for xb in x]


def test_make_qkx2_quants_is_the_grid_optimum(O):
    x = np.concatenate([_subblocks(32, 400, 11), _clustered(32, 600, 13)])
    # the check decides almost every sub-block: one outcome, or a handful from near-ties
    n_out = _branch_count(x)
    assert max(n_out) <= 16 and sum(n > 1 for n in n_out) < 0.1 * len(x), n_out
    for i, xb in enumerate(x):
        scale, mn, L = O.make_qkx2_quants(xb, _q4k_weights(xb))
        assert _check_qkx2(xb, scale, mn, L.astype(np.int64)) is None, (i, _check_qkx2(xb, scale, mn, L.astype(np.int64)))


@pytest.mark.parametrize("plant", ["nstep19", "rdelta0.2", "no_min_clamp"])
def test_make_qkx2_quants_planted_mistakes_fail(O, plant):
    x = np.concatenate([_subblocks(32, 400, 11), _clustered(32, 600, 13)])
    kw = {"nstep19": dict(nstep=19), "rdelta0.2": dict(rdelta=0.2),
          "no_min_clamp": dict(flags=O.PLANT_NO_MIN_CLAMP)}[plant]
    failures = 0
    for xb in x:
        scale, mn, L = O.make_qkx2_quants(xb, _q4k_weights(xb), **kw)
        failures += _check_qkx2(xb, scale, mn, L.astype(np.int64)) is not None
    assert failures > 0, f"planted mistake {plant} passed every check"


def test_make_qkx2_quants_q5_K_is_the_grid_optimum(O):
    """The Q5_K sub-block fit (nmax 31, rmin -0.5, nstep 15) is its grid search's result."""
    x = np.concatenate([_subblocks(32, 300, 15), _clustered(32, 300, 17)])
    n_out = _branch_count(x, Q5K_SEARCH)
    assert max(n_out) <= 16 and sum(n > 1 for n in n_out) < 0.1 * len(x), n_out
    for i, xb in enumerate(x):
        scale, mn, L = O.make_qkx2_quants(xb, _q4k_weights(xb), **Q5K_SEARCH)
        r = _check_qkx2(xb, scale, mn, L.astype(np.int64), Q5K_SEARCH)
        assert r is None, (i, r)


@pytest.mark.parametrize("plant", ["q4k_grid", "nstep14", "rmin-1"])
def test_make_qkx2_quants_q5_K_planted_mistakes_fail(O, plant):
    """Q5_K fits made with a wrong argument (Q4_K's grid, one grid point short, Q4_K's rmin) are
    rejected by the Q5_K check."""
    x = np.concatenate([_subblocks(32, 300, 15), _clustered(32, 300, 17)])
    kw = {"q4k_grid": dict(Q5K_SEARCH, nstep=20, rmin=-1.0), "nstep14": dict(Q5K_SEARCH, nstep=14),
          "rmin-1": dict(Q5K_SEARCH, rmin=-1.0)}[plant]
    failures = 0
    for xb in x:
        scale, mn, L = O.make_qkx2_quants(xb, _q4k_weights(xb), **kw)
        failures += _check_qkx2(xb, scale, mn, L.astype(np.int64), Q5K_SEARCH) is not None
    assert failures > 0, f"planted mistake {plant} passed every check"


def _qx_candidates(x, nmax=32, grid=9):
    """[(l, scale, quality)] of make_qx_quants' candidates, roundings in fp32 as the C."""
    amax_i = int(np.argmax(np.abs(x)))  # first index of the largest |x| (argmax keeps the first)
    mx = f32(x[amax_i])
    w = x.astype(np.float64) ** 2
    out = []
    for is_ in [0] + [i for i in range(-grid, grid + 1) if i != 0]:
        iscale = (f32(-nmax) / mx) if is_ == 0 else (-(f32(nmax) + f32(0.1) * f32(is_)) / mx)
        l = np.clip(np.rint((f32(iscale) * x).astype(np.float32)), -nmax, nmax - 1).astype(np.int64)
        slx, sl2 = float((w * x * l).sum()), float((w * l * l).sum())
        if sl2 > 0:
            out.append((l, slx / sl2, slx * slx / sl2))
    return out


def _check_qx(x, scale, l):
    if np.abs(x).max() < 1e-15:
        return None if (scale == 0 and np.all(l == -32)) else "zero group"  # stored L = 0
    if l.min() < -32 or l.max() > 31:
        return "L outside [-32, 31]"
    cands = _qx_candidates(x)
    best = max(c[2] for c in cands)
    match = [c for c in cands if np.array_equal(c[0], l)]
    if not match:
        return "L is not one of the grid's candidates"
    w = x.astype(np.float64) ** 2
    slx, sl2 = float((w * x * l).sum()), float((w * l * l).sum())
    if slx * slx / sl2 < best * (1 - 1e-5):
        return f"fit quality {slx * slx / sl2:.6g} below the best candidate's {best:.6g}"
    if abs(scale - slx / sl2) > 1e-4 * abs(slx / sl2):
        return "scale is not the least-squares scale of L"
    return None


def test_make_qx_quants_is_the_grid_optimum(O):
    x = _subblocks(16, 600, 12)
    for i, xb in enumerate(x):
        scale, l = O.make_qx_quants(xb)
        assert _check_qx(xb, scale, l) is None, (i, _check_qx(xb, scale, l))


@pytest.mark.parametrize("plant", ["unit_weights", "grid8"])
def test_make_qx_quants_planted_mistakes_fail(O, plant):
    x = _subblocks(16, 600, 12)
    flags = {"unit_weights": O.PLANT_UNIT_WEIGHTS, "grid8": O.PLANT_GRID_8}[plant]
    failures = 0
    for xb in x:
        scale, l = O.make_qx_quants(xb, flags=flags)
        failures += _check_qx(xb, scale, l) is not None
    assert failures > 0, f"planted mistake {plant} passed every check"


def _decode_scale_min(s, j):
    """The GGUF Q4_K sub-block (scale, min) decode, from the format definition."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def test_scale_min_packing_inverts(O):
    rng = np.random.default_rng(7)
    cases = [np.zeros(8, np.uint8), np.full(8, 63, np.uint8), np.arange(8, dtype=np.uint8) * 9]
    cases += [rng.integers(0, 64, 8).astype(np.uint8) for _ in range(2000)]
    for i, ls in enumerate(cases):
        lm = cases[(i * 7 + 3) % len(cases)]
        s = O.pack_scale_min_k4(ls, lm)
        got = [_decode_scale_min(s.astype(np.int64), j) for j in range(8)]
        assert got == [(int(a), int(b)) for a, b in zip(ls, lm)], i


def test_q4_K_quants_are_nearest_and_scales_rounded(O):
    """Final pass of the Q4_K quantizer: every stored quant is the nearest 4-bit grid point of
    d*sc*L - dmin*m to x, and each 6-bit sub-block scale is the nearest integer of
    63 * scale_j / max_j scale_j for the sub-block fits make_qkx2_quants returns."""
    N, K = 8, 1024
    w = synth.normal(N * K, 21, 0.0, 0.02).reshape(N, K)
    w[0, :256] = np.abs(w[0, :256]) + np.float32(0.01)
    q = O.quantize_matrix(12, w).reshape(N, K // 256, 144)
    for n in range(N):
        for b in range(K // 256):
            blk = q[n, b].astype(np.int64)
            d = O.fp16_to_fp32(q[n, b, 0:2].copy().view(np.uint16))[0]
            dmin = O.fp16_to_fp32(q[n, b, 2:4].copy().view(np.uint16))[0]
            xs = w[n, 256 * b:256 * (b + 1)]
            fits = [O.make_qkx2_quants(xs[32 * j:32 * j + 32], _q4k_weights(xs[32 * j:32 * j + 32])) for j in range(8)]
            smax = max(f[0] for f in fits)
            for j in range(8):
                sc, m = _decode_scale_min(blk[4:16], j)
                assert abs(sc - 63 * fits[j][0] / smax) <= 0.5 + 1e-4, (n, b, j)
                if sc == 0:
                    continue
                dj, mj = np.float64(d) * sc, np.float64(dmin) * m
                c, hi = j // 2, j % 2
                nib = (blk[16 + 32 * c:16 + 32 * c + 32] >> (4 * hi)) & 0xF
                xj = xs[32 * j:32 * j + 32].astype(np.float64)
                grid = dj * np.arange(16)[None, :] - mj
                dist = np.abs(xj[:, None] - grid)
                chosen = dist[np.arange(32), nib]
                assert np.all(chosen <= dist.min(axis=1) + 1e-6 * dj), (n, b, j)


def test_q5_K_quants_are_nearest_and_scales_rounded(O):
    """Final pass of the Q5_K quantizer: each 6-bit sub-block scale is the nearest integer of
    63 * scale_j / max_j scale_j for the Q5_K fits, and every stored 5-bit quant (low nibble plus
    the qh bit, read back through dequantize_row) is the nearest of the 32 levels
    d*sc*L - dmin*m to x."""
    N, K = 8, 1024
    w = synth.normal(N * K, 23, 0.0, 0.02).reshape(N, K)
    w[0, :256] = np.abs(w[0, :256]) + np.float32(0.01)
    w[2, 300] = np.float32(0.3)
    q = O.quantize_matrix(13, w).reshape(N, K // 256, 176)
    for n in range(N):
        for b in range(K // 256):
            blk = q[n, b].astype(np.int64)
            d = O.fp16_to_fp32(q[n, b, 0:2].copy().view(np.uint16))[0]
            dmin = O.fp16_to_fp32(q[n, b, 2:4].copy().view(np.uint16))[0]
            xs = w[n, 256 * b:256 * (b + 1)]
            fits = [O.make_qkx2_quants(xs[32 * j:32 * j + 32], _q4k_weights(xs[32 * j:32 * j + 32]), **Q5K_SEARCH)
                    for j in range(8)]
            smax = max(f[0] for f in fits)
            vals = O.dequantize_row(13, q[n, b], 256).astype(np.float64)
            for j in range(8):
                sc, m = _decode_scale_min(blk[4:16], j)
                assert abs(sc - 63 * fits[j][0] / smax) <= 0.5 + 1e-4, (n, b, j)
                if sc == 0:
                    continue
                dj, mj = np.float64(d) * sc, np.float64(dmin) * m
                xj = xs[32 * j:32 * j + 32].astype(np.float64)
                grid = dj * np.arange(32)[None, :] - mj
                dist = np.abs(xj[:, None] - grid)
                chosen = np.abs(xj - vals[32 * j:32 * j + 32])
                assert np.all(chosen <= dist.min(axis=1) + 1e-6 * dj), (n, b, j)


def test_q6_K_quants_are_nearest(O):
    N, K = 8, 1024
    w = synth.normal(N * K, 22, 0.0, 0.02).reshape(N, K)
    w[1, 7] = np.float32(0.5)
    q = O.quantize_matrix(14, w).reshape(N, K // 256, 210)
    for n in range(N):
        for b in range(K // 256):
            d = np.float64(O.fp16_to_fp32(q[n, b, 208:210].copy().view(np.uint16))[0])
            sc = q[n, b, 192:208].view(np.int8).astype(np.int64)
            vals = O.dequantize_row(14, q[n, b], 256).astype(np.float64)
            xs = w[n, 256 * b:256 * (b + 1)].astype(np.float64)
            for g in range(16):
                dj = d * sc[g]
                if dj == 0:
                    continue
                grid = dj * np.arange(-32, 32)[None, :]
                dist = np.abs(xs[16 * g:16 * g + 16, None] - grid)
                chosen = np.abs(xs[16 * g:16 * g + 16] - vals[16 * g:16 * g + 16])
                assert np.all(chosen <= dist.min(axis=1) + 1e-6 * abs(dj)), (n, b, g)
