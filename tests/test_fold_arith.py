"""CPU: the integer decomposition the Q6_K prefill kernel uses to fold each 16-element group's scale
into its weights (densecore_amd/csrc/dcq_prefill_kq.hip, fold4 and the superblock epilogue).

The kernel writes w = (q - 32) * sc as two int8 planes, hi = w >> 6 and lo = w & 63, sums
H = sum_k a_k * hi_k and L = sum_k a_k * lo_k on the int8 MFMA over a superblock, and takes
iS = 64 H + L. These checks pin that decomposition against the direct form of vec_dot_q6_K_q8_K's
per-superblock integer sum, iS = sum_g sc_g * sum_{k in g} (q_k - 32) * a_k, exhaustively over the
(level, scale) pairs and on random superblocks including the extreme ones.
"""
import numpy as np


def planes(q, sc):
    """hi, lo planes of w = (q - 32) * sc as the kernel forms them: 16-bit products (two per packed
    instruction), an arithmetic shift by 6 and a mask of 63."""
    w = (q.astype(np.int32) - 32) * sc.astype(np.int32)
    w16 = w.astype(np.int16)  # the packed 16-bit multiply keeps the low 16 bits
    assert np.array_equal(w16.astype(np.int32), w), "a product does not fit 16 bits"
    hi = (w16 >> 6).astype(np.int32)
    lo = (w16.astype(np.int32) & 63)
    return hi, lo


def test_every_level_and_scale_splits_exactly_into_int8_planes():
    q, sc = np.meshgrid(np.arange(64), np.arange(-128, 128), indexing="ij")
    hi, lo = planes(q.ravel(), sc.ravel())
    w = (q.ravel() - 32) * sc.ravel()
    assert np.array_equal(64 * hi + lo, w)
    assert hi.min() >= -64 and hi.max() <= 64  # int8 operands
    assert lo.min() >= 0 and lo.max() <= 63
    assert np.abs(w).max() == 4096


def superblock_sums(q, sc, a):
    """(direct iS, 64 H + L) for one weight row's superblock: q [256] levels, sc [16] group
    scales, a [256] activation quants."""
    direct = sum(int(sc[g]) * int(np.dot(q[16 * g:16 * g + 16].astype(np.int64) - 32, a[16 * g:16 * g + 16]))
                 for g in range(16))
    hi, lo = planes(q, np.repeat(sc, 16))
    H = int(np.dot(hi.astype(np.int64), a))
    L = int(np.dot(lo.astype(np.int64), a))
    assert abs(H) < 2 ** 22 and abs(L) < 2 ** 31 and abs(64 * H + L) < 2 ** 31  # int32 accumulators
    return direct, 64 * H + L


def test_superblock_sum_equals_the_per_group_form():
    rng = np.random.default_rng(6)
    for _ in range(2000):
        q = rng.integers(0, 64, 256)
        sc = rng.integers(-128, 128, 16)
        a = rng.integers(-127, 128, 256)
        d, f = superblock_sums(q, sc, a)
        assert d == f
    # the extremes: every product at +4096 or -4064 against full-scale activations
    for qv, scv, av in [(0, -128, 127), (0, -128, -127), (0, 127, 127), (63, 127, -127), (63, -128, 127)]:
        d, f = superblock_sums(np.full(256, qv), np.full(16, scv), np.full(256, av))
        assert d == f
