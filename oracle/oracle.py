"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg. The product library never
imports it. See dcq_oracle.h for what it restates and how each part is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
Q8_0_X86, Q8_0_REF = 0, 1

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, vp, fp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
        sz = ctypes.c_size_t
        sig = {
            "dcqo_block_size": (i64, [i32]),
            "dcqo_type_size": (i64, [i32]),
            "dcqo_row_size": (i64, [i32, i64]),
            "dcqo_vec_dot_type": (i32, [i32]),
            "dcqo_fp32_to_fp16": (ctypes.c_uint16, [fp]),
            "dcqo_fp16_to_fp32": (fp, [ctypes.c_uint16]),
            "dcqo_fp32_to_fp16_array": (None, [vp, vp, i64]),
            "dcqo_fp16_to_fp32_array": (None, [vp, vp, i64]),
            "dcqo_quantize_row_q8_0": (None, [vp, vp, i64, i32]),
            "dcqo_quantize_row_q8_K": (None, [vp, vp, i64]),
            "dcqo_quantize_rows": (None, [i32, vp, i64, i64, i64, vp, i32]),
            "dcqo_quantize_matrix": (i32, [i32, vp, i64, i64, vp, i32]),
            "dcqo_dequantize_row": (i32, [i32, vp, vp, i64]),
            "dcqo_vec_dot": (fp, [i32, i64, vp, vp]),
            "dcqo_vec_dot_f64": (ctypes.c_double, [i32, i64, vp, vp]),
            "dcqo_vec_dot_l1": (ctypes.c_double, [i32, i64, vp, vp]),
            "dcqo_block_sums_per_row": (i64, [i32, i64]),
            "dcqo_block_sums": (i32, [i32, i64, vp, vp, vp]),
            "dcqo_block_sums_bruteforce": (i32, [i32, i64, vp, vp, vp]),
            "dcqo_dot_rows": (i32, [i32, vp, sz, vp, i64, vp, i64, i64]),
            "dcqo_mul_mat": (i32, [i32, vp, i64, i64, sz, vp, i64, i64, vp, i64, vp, i32, i32]),
            "dcqo_make_qkx2_quants": (fp, [i32, i32, vp, vp, vp, ctypes.POINTER(fp), fp, fp, i32, i32]),
            "dcqo_make_qx_quants": (fp, [i32, i32, vp, vp, i32]),
            "dcqo_pack_scale_min_k4": (None, [vp, vp, vp]),
            "dcqs_isa": (i32, []),
            "dcqs_vec_dot": (fp, [i32, i32, i64, vp, vp]),
            "dcqs_physical_cpus": (i32, [vp, i32, vp]),
            "dcqs_mul_mat": (i32, [i32, i32, vp, i64, i64, sz, vp, i64, i64, vp, i64, i32, vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_size(t, k):
    return int(lib().dcqo_row_size(t, k))


def block_size(t):
    return int(lib().dcqo_block_size(t))


def vec_dot_type(t):
    return int(lib().dcqo_vec_dot_type(t))


def fp32_to_fp16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().dcqo_fp32_to_fp16_array(_p(x), _p(y), x.size)
    return y


def fp16_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().dcqo_fp16_to_fp32_array(_p(h), _p(y), h.size)
    return y


def quantize_rows(vdt, x, variant=Q8_0_X86):
    """Activation quantization of every row of x [m, k] -> uint8 [m, row_size]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    rs = row_size(vdt, k)
    assert rs > 0, (vdt, k)
    y = np.zeros((m, rs), dtype=np.uint8)
    lib().dcqo_quantize_rows(vdt, _p(x), m, k, k, _p(y), variant)
    return y


def quantize_matrix(t, w, nthreads=0):
    """Weight quantization of w [n, k] -> uint8 [n, row_size] (rows packed)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    rs = row_size(t, k)
    y = np.zeros((n, rs), dtype=np.uint8)
    rc = lib().dcqo_quantize_matrix(t, _p(w), n, k, _p(y), nthreads)
    assert rc == 0, rc
    return y


def dequantize_row(t, q, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    y = np.empty(k, dtype=np.float32)
    rc = lib().dcqo_dequantize_row(t, _p(q), _p(y), k)
    assert rc == 0
    return y


def vec_dot(wt, k, w_row, xq_row):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    return float(lib().dcqo_vec_dot(wt, k, _p(w_row), _p(xq_row)))


def vec_dot_f64(wt, k, w_row, xq_row):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    return float(lib().dcqo_vec_dot_f64(wt, k, _p(w_row), _p(xq_row)))


def vec_dot_l1(wt, k, w_row, xq_row):
    """Sum of the magnitudes of the fp32 terms the reference's vec_dot adds: |d_b * I_b| per
    Q8_0 / Q4_0 block; for Q4_K / Q5_K / Q6_K the eight per-superblock lane sums |d * aux32[l]|
    (plus the Q4_K / Q5_K mins term), which can cancel to a much smaller superblock total."""
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    return float(lib().dcqo_vec_dot_l1(wt, k, _p(w_row), _p(xq_row)))


def block_sums_per_row(wt, k):
    return int(lib().dcqo_block_sums_per_row(wt, k))


def block_sums(wt, k, w_row, xq_row):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    out = np.zeros(block_sums_per_row(wt, k), dtype=np.int32)
    assert lib().dcqo_block_sums(wt, k, _p(w_row), _p(xq_row), _p(out)) == 0
    return out


def block_sums_bruteforce(wt, k, w_row, xq_row):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    out = np.zeros(block_sums_per_row(wt, k), dtype=np.int64)
    assert lib().dcqo_block_sums_bruteforce(wt, k, _p(w_row), _p(xq_row), _p(out)) == 0
    return out


def block_sums_matrix(wt, k, wq, xq):
    """int32 [m, n, per_row] block sums of every (activation row, weight row)."""
    m, n = xq.shape[0], wq.shape[0]
    per = block_sums_per_row(wt, k)
    out = np.zeros((m, n, per), dtype=np.int32)
    for mi in range(m):
        for ni in range(n):
            out[mi, ni] = block_sums(wt, k, wq[ni], xq[mi])
    return out


def dot_rows(wt, wq, xq_row, k, n0, n1):
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    y = np.zeros(max(n1 - n0, 0), dtype=np.float32)
    rc = lib().dcqo_dot_rows(wt, _p(wq), wq.shape[1], _p(xq_row), k, _p(y), n0, n1)
    assert rc == 0
    return y


def mul_mat(wt, wq, x, variant=Q8_0_X86, nthreads=0, want_l1=True):
    """GGML_OP_MUL_MAT: Y[m, n] = vec_dot(W row n, quantize(X row m)); also L1 guard."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    n = wq.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    l1 = np.zeros((m, n), dtype=np.float32) if want_l1 else None
    rc = lib().dcqo_mul_mat(wt, _p(wq), n, k, wq.shape[1], _p(x), m, k, _p(y), n,
                            _p(l1) if want_l1 else None, variant, nthreads)
    assert rc == 0, rc
    return (y, l1) if want_l1 else y


def repack_q8_0_rs(wq, k):
    """Row-split layout of Q8_0 rows (the library's own load-time layout, no reference counterpart):
    [N][34*K/32] GGUF Q8_0 rows -> [N][34*K/32] rows holding the K int8 quants first (block b's 32 at
    byte 32b), then the K/32 fp16 scales (block b's at byte K + 2b). A plain byte rearrangement:
    its values are the Q8_0 rows' (the tests check dequantization and every product against the
    Q8_0 rows as well)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    n = wq.shape[0]
    nb = k // 32
    blocks = wq[:, :34 * nb].reshape(n, nb, 34)
    out = np.empty((n, 34 * nb), dtype=np.uint8)
    out[:, :k] = blocks[:, :, 2:].reshape(n, k)
    out[:, k:] = blocks[:, :, :2].reshape(n, 2 * nb)
    return out


def silu(g):
    """ggml_silu, the SwiGLU gate nonlinearity g / (1 + e^-g), in float64 (ggml's definition;
    reference call ggml_silu at core/src/inference.cpp:1796)."""
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


def ffn_gate_up(wt, wg, wu, x, variant=Q8_0_X86, nthreads=0):
    """The reference FFN's gate/up pair and product (core/src/inference.cpp:1794-1796):
    w1 = mul_mat(W1, x), w3 = mul_mat(W3, x), y = silu(w1) * w3, both projections on the same
    quantized x. Returns y (float64) and (g, l1_g, u, l1_u) for the tolerance."""
    g, l1g = mul_mat(wt, wg, x, variant, nthreads)
    u, l1u = mul_mat(wt, wu, x, variant, nthreads)
    return silu(g) * u.astype(np.float64), (g, l1g, u, l1u)


def assert_close_gate_up(y, y_ref, parts, rtol=1e-4, what=""):
    """Tolerance of silu(g) * u when g and u each carry the mul_mat bound
    |dg| <= rtol * max(|g|, L1_g) (same for u): |dy| <= 1.1 |dg| (|u| + |du|) + |silu(g)| |du|
    (|silu'| < 1.1 everywhere)."""
    g, l1g, u, l1u = (np.asarray(a, dtype=np.float64) for a in parts)
    dg = rtol * np.maximum(np.abs(g), l1g)
    du = rtol * np.maximum(np.abs(u), l1u)
    bound = 1.1 * dg * (np.abs(u) + du) + np.abs(silu(g)) * du + 1e-30
    err = np.abs(np.asarray(y, dtype=np.float64) - y_ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} outside the bound; worst at {i}: "
                             f"got {y[i]} want {y_ref[i]} bound {bound[i]}")


def assert_close(y, y_ref, l1, rtol=1e-4, what=""):
    """The output tolerance: |y - y_ref| <= rtol * max(|y_ref|, L1), elementwise.

    L1 = sum of the magnitudes of the fp32 terms of the reference's summation (vec_dot_l1)
    guards outputs whose terms cancel: their fp32 rounding error scales with L1, not with
    |y_ref|.
    """
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    bound = rtol * np.maximum(np.abs(y_ref), np.asarray(l1, dtype=np.float64))
    err = np.abs(y - y_ref)
    bad = err > bound
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outputs outside tolerance; first {idx.tolist()}: "
            f"got {y[tuple(idx[0])]}, want {y_ref[tuple(idx[0])]}, bound {bound[tuple(idx[0])]}")
    rel = err / np.maximum(np.abs(y_ref), 1e-30)
    return float(np.max(err / np.maximum(bound / rtol, 1e-30))), float(np.median(rel))


def relative_error_stats(y, y_ref, rtol=1e-4):
    """The plain elementwise relative error |y - y_ref| / |y_ref| over outputs with y_ref != 0:
    its median, 99th percentile and maximum, and how many outputs exceed rtol (outputs whose fp32
    terms cancel can, while staying inside the L1-guarded bound of assert_close)."""
    y = np.asarray(y, dtype=np.float64).ravel()
    y_ref = np.asarray(y_ref, dtype=np.float64).ravel()
    nz = y_ref != 0
    rel = np.abs(y[nz] - y_ref[nz]) / np.abs(y_ref[nz])
    if rel.size == 0:
        return {"n": 0, "p50": 0.0, "p99": 0.0, "max": 0.0, "n_above": 0, "n_zero_ref": int(y_ref.size)}
    return {"n": int(rel.size), "p50": float(np.percentile(rel, 50)), "p99": float(np.percentile(rel, 99)),
            "max": float(rel.max()), "n_above": int((rel > rtol).sum()), "n_zero_ref": int((~nz).sum())}


# ---------------------------------------------------------------- weight-quantizer test hooks
PLANT_NO_MIN_CLAMP, PLANT_UNIT_WEIGHTS, PLANT_GRID_8 = 1, 2, 4


def make_qkx2_quants(x, weights, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20, flags=0):
    """The Q4_K (defaults) or Q5_K (nmax=31, rmin=-0.5, nstep=15) sub-block fit x ~ scale * L + min
    (min <= 0): returns (scale, min, L uint8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    L = np.zeros(x.size, dtype=np.uint8)
    the_min = ctypes.c_float(0)
    scale = lib().dcqo_make_qkx2_quants(x.size, nmax, _p(x), _p(weights), _p(L), ctypes.byref(the_min),
                                        rmin, rdelta, nstep, flags)
    return float(scale), -float(the_min.value), L


def make_qx_quants(x, nmax=32, flags=0):
    """The Q6_K group fit x ~ scale * (L - nmax): returns (scale, L - nmax as int)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = np.zeros(x.size, dtype=np.int8)
    scale = lib().dcqo_make_qx_quants(x.size, nmax, _p(x), _p(L), flags)
    return float(scale), L.astype(np.int64) - nmax


def pack_scale_min_k4(ls, lm):
    ls = np.ascontiguousarray(ls, dtype=np.uint8)
    lm = np.ascontiguousarray(lm, dtype=np.uint8)
    out = np.zeros(12, dtype=np.uint8)
    lib().dcqo_pack_scale_min_k4(_p(ls), _p(lm), _p(out))
    return out


# ---------------------------------------------------------------- SIMD CPU restatement (the timed baseline)
ISA_SCALAR, ISA_AVX2, ISA_AVX512VNNI = 0, 1, 2
ISA_NAMES = {ISA_SCALAR: "scalar", ISA_AVX2: "AVX2 (vpmaddubsw/vpmaddwd)",
             ISA_AVX512VNNI: "AVX-512 VNNI (vpdpbusd) for Q8_0, AVX2 for Q4_K/Q6_K"}


def simd_isa():
    """The widest int8 dot the host CPU supports (CPUID at run time)."""
    return int(lib().dcqs_isa())


def simd_vec_dot(isa, wt, k, w_row, xq_row):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    xq_row = np.ascontiguousarray(xq_row, dtype=np.uint8)
    return float(lib().dcqs_vec_dot(isa, wt, k, _p(w_row), _p(xq_row)))


def physical_cpus(limit=4096):
    """(logical CPUs to pin one worker per physical core, logical CPUs in the affinity mask)."""
    cpus = np.zeros(limit, dtype=np.int32)
    logical = ctypes.c_int(0)
    n = lib().dcqs_physical_cpus(_p(cpus), limit, ctypes.byref(logical))
    return (cpus[:max(n, 0)].tolist(), logical.value)


def simd_mul_mat(wt, wq, x, nthreads=1, cpus=None, isa=-1):
    """The timed CPU baseline: quantize every X row once, then row-partitioned SIMD vec_dots on
    nthreads workers (pinned to `cpus` when given). Y [m, n] float32."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    n = wq.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    cp = np.ascontiguousarray(cpus, dtype=np.int32) if cpus is not None else None
    rc = lib().dcqs_mul_mat(isa, wt, _p(wq), n, k, wq.shape[1], _p(x), m, k, _p(y), n, nthreads,
                            _p(cp) if cp is not None else None)
    assert rc == 0, rc
    return y
