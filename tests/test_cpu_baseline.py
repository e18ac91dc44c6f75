"""The timed CPU baseline (oracle/dcq_cpu_simd.c) against the scalar oracle.

The SIMD restatement must compute the same operator as the scalar oracle: within the output
tolerance on random inputs for every ISA path (scalar, AVX2, AVX-512 VNNI), thread count and
ragged shape, and bit for bit on inputs built so that every fp32 operation of both summation
orders is exact (power-of-two block scales, small integers), where any indexing or sign mistake
in the SIMD code changes the result.
"""
import numpy as np
import pytest

from densecore_amd import synth

Q8_0, Q4_K, Q6_K = 8, 12, 14


def _isas(O):
    best = O.simd_isa()
    return [i for i in (O.ISA_SCALAR, O.ISA_AVX2, O.ISA_AVX512VNNI) if i <= best]


@pytest.mark.parametrize("wt,M,N,K", [(Q8_0, 1, 100, 1024), (Q8_0, 67, 45, 2048), (Q4_K, 1, 99, 2560),
                                      (Q4_K, 9, 33, 512), (Q6_K, 1, 70, 9728), (Q6_K, 3, 17, 256)])
def test_simd_matches_scalar_oracle(O, wt, M, N, K):
    w = synth.normal(N * K, 31 + N, 0.0, 0.02).reshape(N, K)
    x = synth.normal(M * K, 32 + M).reshape(M, K)
    synth.set_outliers(x[0], max(1, K // 100), 20.0, 9)
    wq = O.quantize_matrix(wt, w)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    for isa in _isas(O):
        for nt in (1, 3):
            y = O.simd_mul_mat(wt, wq, x, nthreads=nt, isa=isa)
            O.assert_close(y, y_ref, l1, 1e-4, what=f"SIMD type {wt} isa {isa} threads {nt}")


def _fp16(v):
    return int(np.array(v, dtype=np.float16).view(np.uint16))


def _exact_inputs(wt, M, N, K, rng):
    """Weights with power-of-two fp16 scales and random integer fields; activations whose blocks
    quantize exactly (the block extreme is 127 * 2^-5, so the activation scale is 2^-5, and every
    other value is a small multiple of 2^-5)."""
    x = rng.integers(-3, 4, size=(M, K)).astype(np.float32) * np.float32(2.0 ** -5)
    if wt == Q8_0:
        x[:, ::32] = np.float32(127 * 2.0 ** -5)
        rows = np.zeros((N, K // 32, 34), dtype=np.uint8)
        rows[:, :, 0:2] = np.frombuffer(np.uint16(_fp16(2.0 ** -6)).tobytes(), dtype=np.uint8)
        rows[:, :, 2:] = rng.integers(-15, 16, size=(N, K // 32, 32)).astype(np.int8).view(np.uint8)
    elif wt == Q4_K:
        x[:, ::256] = np.float32(-127 * 2.0 ** -5)
        rows = rng.integers(0, 256, size=(N, K // 256, 144)).astype(np.uint8)
        rows[:, :, 0:2] = np.frombuffer(np.uint16(_fp16(2.0 ** -8)).tobytes(), dtype=np.uint8)
        rows[:, :, 2:4] = np.frombuffer(np.uint16(_fp16(2.0 ** -9)).tobytes(), dtype=np.uint8)
    else:
        x[:, ::256] = np.float32(-127 * 2.0 ** -5)
        rows = rng.integers(0, 256, size=(N, K // 256, 210)).astype(np.uint8)
        rows[:, :, 192:208] = rng.integers(-20, 21, size=(N, K // 256, 16)).astype(np.int8).view(np.uint8)
        rows[:, :, 208:210] = np.frombuffer(np.uint16(_fp16(2.0 ** -8)).tobytes(), dtype=np.uint8)
    return rows.reshape(N, -1), x


@pytest.mark.parametrize("wt,M,N,K", [(Q8_0, 5, 37, 1024), (Q4_K, 4, 21, 1024), (Q6_K, 4, 19, 1024)])
def test_simd_bit_exact_on_exact_arithmetic(O, wt, M, N, K):
    rng = np.random.default_rng(1234 + wt)
    wq, x = _exact_inputs(wt, M, N, K, rng)
    xq = O.quantize_rows(O.vec_dot_type(wt), x)
    # the construction holds: the activation scale is exactly 2^-5 in every block
    if wt == Q8_0:
        d = O.fp16_to_fp32(xq.reshape(M, K // 32, 34)[:, :, :2].copy().view(np.uint16))
    else:
        d = xq.reshape(M, K // 256, 292)[:, :, :4].copy().view(np.float32)
    assert np.all(d == np.float32(2.0 ** -5))
    y_ref = O.mul_mat(wt, wq, x, want_l1=False)
    y64 = np.array([[O.vec_dot_f64(wt, K, wq[n], xq[m]) for n in range(N)] for m in range(M)])
    assert np.array_equal(y_ref.astype(np.float64), y64)  # the scalar oracle is exact here
    for isa in _isas(O):
        y = O.simd_mul_mat(wt, wq, x, nthreads=2, isa=isa)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), f"isa {isa}"


def test_physical_cpus_are_distinct_and_within_the_mask(O):
    cpus, logical = O.physical_cpus()
    assert 1 <= len(cpus) <= logical
    assert len(set(cpus)) == len(cpus)


def test_simd_catches_a_planted_mistake(O):
    """The comparison above is strong enough to see a one-element mistake: flipping one weight
    quantum of an exact-arithmetic input moves the oracle's output, so an SIMD kernel that
    mis-indexed that element would fail the bit-exact check."""
    rng = np.random.default_rng(99)
    wq, x = _exact_inputs(Q8_0, 2, 3, 1024, rng)
    y0 = O.mul_mat(Q8_0, wq, x, want_l1=False)
    bad = wq.copy()
    bad[1, 2 + 7] ^= 1  # one int8 quantum of block 0 of row 1
    y1 = O.mul_mat(Q8_0, bad, x, want_l1=False)
    assert not np.array_equal(y0[:, 1], y1[:, 1]) and np.array_equal(y0[:, [0, 2]], y1[:, [0, 2]])
