"""GPU parity: libdcq (through its C ABI) against the CPU oracle on identical inputs.

Bars: quantized activation bytes and per-block int32 sums
bit-exact; fp32 outputs within |y - y_ref| <= 1e-4 * max(|y_ref|, L1), where L1
is the sum of the magnitudes of the fp32 terms the reference adds (|scale_b * int_b|
per Q8_0 / Q4_0 block; the eight per-superblock lane sums of Q4_K / Q5_K / Q6_K, plus the mins
term):
the magnitude the fp32 rounding of both summation orders scales with.
"""
import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 2, 8, 12, 13, 14, 15
RTOL = 1e-4


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_inputs(O, wt, M, N, K, seed, zero_blocks=True, outliers=0):
    w = synth.normal(N * K, 1000 + seed, 0.0, 0.02).reshape(N, K)
    if zero_blocks and N > 2:
        w[1, :K // 2] = 0.0  # zero blocks / superblocks on the weight side
    wq = O.quantize_matrix(wt, w)
    x = synth.normal(M * K, 2000 + seed).reshape(M, K)
    if zero_blocks and M > 1:
        x[M - 1, :256] = 0.0  # an all-zero activation block
    if outliers:
        for m in range(M):
            synth.set_outliers(x[m], outliers, 20.0, 3000 + seed + m)
    return wq, x


# ---------------------------------------------------------------- activation quantization
@pytest.mark.parametrize("vdt", [Q8_0, Q8_K])
@pytest.mark.parametrize("M,K", [(1, 256), (3, 2560), (64, 2048), (2, 9728)])
def test_quantize_rows_bit_exact(O, dev, vdt, M, K):
    x = synth.normal(M * K, 77 + M + K).reshape(M, K)
    x[0, :256] = 0.0
    synth.set_outliers(x[-1], max(1, K // 100), 20.0, 5)
    # exact ties for Q8_0: amax 127 in a block makes id = 1
    t0 = 256 if K >= 512 else 0
    x[0, t0:t0 + 32] = np.arange(32, dtype=np.float32) - 15.5
    x[0, t0] = 127.0
    got = to_host(dc.quantize_rows(vdt, to_dev(x, dev)))
    want = O.quantize_rows(vdt, x, O.Q8_0_X86)
    assert np.array_equal(got, want)


def test_quantize_q8_K_ties_bit_exact(O, dev):
    """Q8_K's scale comes from the FIRST element of largest |x|: blocks whose maximum |x| is held
    by both signs (first occurrence negative, or positive, in different lanes of the 16-lane
    group and in the same lane), a single maximum, an all-zero block and exact .5 products."""
    K = 256 * 8
    x = synth.normal(4 * K, 4242).reshape(4, K) * np.float32(0.5)
    blk = lambda r, b: x[r, 256 * b:256 * (b + 1)]
    blk(0, 0)[[37, 200]] = [-3.0, 3.0]       # negative first, different lanes
    blk(0, 1)[[5, 250]] = [3.0, -3.0]        # positive first
    blk(0, 2)[[16, 17]] = [-3.0, 3.0]        # same lane
    blk(0, 3)[[255, 0]] = [-3.0, 3.0]        # last element negative, first positive
    blk(1, 0)[:] = 0.0                       # all zero
    blk(1, 1)[:] = 0.0
    blk(1, 1)[77] = -1.0                     # single non-zero
    blk(1, 2)[:] = np.float32(1.0)           # all equal
    blk(2, 0)[[3, 4, 5]] = [-127.0, 63.5, -0.5]  # iscale = 1: exact .5 ties round half even
    blk(2, 1)[[3, 4, 5]] = [127.0, 62.5, 1.5]
    got = to_host(dc.quantize_rows(Q8_K, to_dev(x, dev)))
    assert np.array_equal(got, O.quantize_rows(Q8_K, x))


def _planar_regions(vdt, M, K):
    """Byte layout of dcq_quantize_src1's workspace (planar_bytes in dcq_api.cpp): int8 qs [M][K],
    fp32 scales [K/bs][m_ld] with m_ld = M rounded up to 128 (rows >= M hold 0), then for Q8_K the
    int16 16-element sums [M][K/16]; each region starts on a 256-byte boundary."""
    up = lambda v, a: (v + a - 1) // a * a
    bs = 32 if vdt == Q8_0 else 256
    m_ld = up(M, 128)
    qs_b = up(M * K, 256)
    d_b = up((K // bs) * m_ld * 4, 256)
    return bs, m_ld, qs_b, d_b


@pytest.mark.parametrize("wt,M,K", [(Q8_0, 1, 96), (Q8_0, 33, 96), (Q8_0, 130, 1024), (Q4_K, 1, 256),
                                    (Q4_K, 17, 2560), (Q4_K, 130, 512)])
def test_quantize_src1_planar_bit_exact(O, dev, wt, M, K):
    """The planar activation the prefill, batch and MMQ kernels read, byte for byte against the
    oracle's row quantization: int8 values, scales (Q8_0's fp16 d widened to fp32), the Q8_K
    16-element sums, and zero scales on the padding rows. Covers an odd block count per row
    (K = 96: three Q8_0 blocks) and row counts that leave part of a row tile empty."""
    import torch
    vdt = Q8_0 if wt == Q8_0 else Q8_K
    x = synth.normal(M * K, 500 + M + K).reshape(M, K)
    synth.set_outliers(x[-1], max(1, K // 100), 20.0, 7)
    ws = torch.full((dc.mul_mat_workspace_size(wt, M, K),), 0xAB, dtype=torch.uint8, device=dev)
    dc.quantize_src1(wt, to_dev(x, dev), ws)
    raw = to_host(ws)
    bs, m_ld, qs_b, d_b = _planar_regions(vdt, M, K)
    nb = K // bs
    qs = raw[:M * K].view(np.int8).reshape(M, K)
    d = raw[qs_b:qs_b + nb * m_ld * 4].view(np.float32).reshape(nb, m_ld)
    want = O.quantize_rows(vdt, x)
    if vdt == Q8_0:
        blocks = want.reshape(M, nb, 34)
        want_d = blocks[:, :, :2].copy().view(np.float16).reshape(M, nb).astype(np.float32)
        want_qs = blocks[:, :, 2:].copy().view(np.int8).reshape(M, K)
    else:
        blocks = want.reshape(M, nb, 292)
        want_d = blocks[:, :, :4].copy().view(np.float32).reshape(M, nb)
        want_qs = blocks[:, :, 4:260].copy().view(np.int8).reshape(M, K)
        want_bs = blocks[:, :, 260:].copy().view(np.int16).reshape(M, K // 16)
        got_bs = raw[qs_b + d_b:qs_b + d_b + M * (K // 16) * 2].view(np.int16).reshape(M, K // 16)
        assert np.array_equal(got_bs, want_bs)
    assert np.array_equal(qs, want_qs)
    assert np.array_equal(d[:, :M].T, want_d)
    assert np.all(d[:, M:] == 0.0)


def test_quantize_rows_strided_input(O, dev):
    import torch
    x = synth.normal(4 * 1024, 91).reshape(4, 1024)
    big = torch.zeros((4, 1024 + 64), dtype=torch.float32, device=dev)
    big[:, :1024] = to_dev(x, dev)
    got = to_host(dc.quantize_rows(Q8_K, big[:, :1024]))
    assert np.array_equal(got, O.quantize_rows(Q8_K, x))


# ---------------------------------------------------------------- mul_mat: outputs and block sums
CASES = [
    (Q8_0, 1, 96, 1024), (Q8_0, 3, 70, 2048), (Q8_0, 1, 33, 96), (Q8_0, 2, 40, 160), (Q8_0, 40, 100, 512),
    (Q8_0, 130, 257, 256),
    # the prefill kernel's unguarded variant (M and N multiples of its 128 x 128 tile), and more
    # m-tiles: full, then ragged M and N
    (Q8_0, 256, 384, 1024), (Q8_0, 512, 256, 512), (Q8_0, 700, 300, 640),
    (Q4_K, 1, 97, 2560), (Q4_K, 2, 64, 256), (Q4_K, 5, 40, 512), (Q4_K, 64, 96, 2048), (Q4_K, 70, 33, 768),
    # the Q4_K prefill kernel (M > 128): unguarded 128 x 128 tiles, ragged M and N, one superblock
    (Q4_K, 256, 384, 1024), (Q4_K, 200, 300, 2048), (Q4_K, 130, 129, 256),
    # single-row decode at full width: 5-wave workgroups (rows spread evenly over the CUs)
    (Q4_K, 1, 9728, 2560), (Q4_K, 1, 2570, 4096), (Q4_K, 1, 2561, 9728),
    (Q6_K, 1, 50, 9728), (Q6_K, 1, 3, 256), (Q6_K, 8, 64, 512), (Q6_K, 33, 65, 1024), (Q6_K, 3, 17, 768),
    (Q6_K, 2, 9, 16384), (Q6_K, 1, 5, 16896),
    # the Q6_K prefill kernel (M > 32, an even number of superblocks): unguarded 128 x 128 tiles,
    # ragged M and N, one superblock pair; an odd count (K = 768) takes the generic kernel
    (Q6_K, 256, 384, 1024), (Q6_K, 200, 300, 2048), (Q6_K, 130, 129, 512), (Q6_K, 40, 50, 768),
    # Q6_K decode with the activation quantized in the workgroup (M <= 2, K <= 4096)
    (Q6_K, 1, 1000, 2560), (Q6_K, 2, 70, 4096),
    # fused Q4_K decode at the concatenated Q/K/V rows of Qwen3-4B and at twice the ffn width
    (Q4_K, 1, 6144, 2560), (Q4_K, 1, 12288, 2560),
    # fused Q6_K beyond K = 4096: one 8..12-wave workgroup per CU (rows per CU 8, 10, 12), the
    # activation staged by the first four waves in up to 4 passes; two rows at K = 9728 exceed
    # the 4 passes and take the separate quantize
    (Q6_K, 1, 2048, 9728), (Q6_K, 2, 2560, 9728), (Q6_K, 1, 3000, 5120),
    (Q6_K, 2, 2560, 8192), (Q6_K, 1, 2048, 12288),
    # the quantize tool's Q4_0 and Q5_K (core/src/quantize.cpp:71-78) on the generic GEMV and MFMA
    # kernels: Q4_0 in block pairs (K % 64 == 0, dword-aligned rows) and single blocks (K = 96,
    # 160: 54- and 90-byte rows), Qwen3-4B's ffn width, ragged tiles, several K-steps
    (Q4_0, 1, 96, 1024), (Q4_0, 3, 70, 2048), (Q4_0, 1, 33, 96), (Q4_0, 2, 40, 160), (Q4_0, 4, 41, 192),
    (Q4_0, 40, 100, 512), (Q4_0, 130, 257, 256), (Q4_0, 256, 384, 1024), (Q4_0, 1, 9728, 2560),
    (Q5_K, 1, 97, 2560), (Q5_K, 2, 64, 256), (Q5_K, 5, 40, 512), (Q5_K, 64, 96, 2048), (Q5_K, 70, 33, 768),
    (Q5_K, 256, 384, 1024), (Q5_K, 1, 9728, 2560), (Q5_K, 3, 2560, 9728),
    # the Q4_K / Q5_K batch kernel past 256 rows while the prefill tiles would not fill the CUs
    # (eight 64-row m-tiles, ragged last one), and the prefill kernel from 512 rows over 256+ tiles
    (Q4_K, 500, 320, 1024), (Q5_K, 384, 200, 512), (Q4_K, 512, 8192, 256),
]


@pytest.mark.parametrize("path", [dc.PATH_GEMV, dc.PATH_MMQ])
@pytest.mark.parametrize("wt,M,N,K", CASES)
def test_mul_mat_parity(O, dev, wt, M, N, K, path):
    import torch
    wq, x = make_inputs(O, wt, M, N, K, seed=M * 7 + N + K, outliers=2)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    per = dc.block_sums_per_row(wt, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    y = dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=path, block_sums=sums)
    O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"type {wt} M{M} N{N} K{K} path {path}")
    want = O.block_sums_matrix(wt, K, wq, O.quantize_rows(O.vec_dot_type(wt), x))
    assert np.array_equal(to_host(sums), want)
    # the same call without the integer dump takes the production kernels
    y2 = dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=path)
    O.assert_close(to_host(y2), y_ref, l1, RTOL, what="production kernel")


def _with_quantizer_ties(x, vdt):
    """Blocks whose scaled values hit exact .5 ties, an all-zero block and a single non-zero one."""
    K = x.shape[1]
    bs = 32 if vdt == Q8_0 else 256
    x[0, :bs] = np.float32(0.25) * (np.arange(bs, dtype=np.float32) - bs / 2)
    x[0, 0] = 127.0 if vdt == Q8_0 else -127.0  # scale 1: the .5 values are ties
    x[0, 1:6] = [0.5, 1.5, -2.5, 62.5, -0.5]
    if K >= 3 * bs:
        x[-1, bs:2 * bs] = 0.0
        x[-1, 2 * bs:3 * bs] = 0.0
        x[-1, 2 * bs + 7] = -3.0
    return x


# Shapes for the decode kernels that quantize the activation in the workgroup (M <= 8):
# Q8_0 lanes-per-row / pairs-per-lane shapes {16,1} (K 1024), {32,1} (2048), {64,1} (4096,
# and 3072 with idle lanes), {64,2} (8192); M tiles 1, 2, 4 and 8 rows; N not a multiple of
# the rows per workgroup. Q4_K for comparison on the same inputs. Q6_K beyond K = 4096: the
# 8..12-wave workgroups whose first four waves stage the activation (3 and 4 passes).
FUSED = [(Q8_0, 1, 96, 1024), (Q8_0, 8, 50, 1024), (Q8_0, 5, 37, 512), (Q8_0, 2, 41, 4096),
         (Q8_0, 1, 29, 3072), (Q8_0, 1, 70, 8192), (Q8_0, 3, 33, 2048), (Q4_K, 1, 45, 2560),
         (Q4_K, 7, 21, 1024), (Q4_K, 1, 2560, 9728),
         (Q6_K, 1, 2560, 9728), (Q6_K, 2, 2560, 8192), (Q6_K, 1, 3000, 5120),
         (Q4_0, 1, 96, 1024), (Q4_0, 5, 37, 512), (Q4_0, 1, 70, 8192), (Q4_0, 2, 2560, 9728),
         # shapes of 3 pairs per lane: 16 x 3 (Q4_0 at K = 2560), 32 x 3 (K = 5120)
         (Q4_0, 1, 300, 2560), (Q4_0, 3, 200, 5120), (Q8_0, 1, 300, 5120), (Q8_0, 2, 97, 3072),
         (Q5_K, 1, 45, 2560), (Q5_K, 7, 21, 1024), (Q5_K, 1, 2560, 9728), (Q5_K, 3, 9728, 2560)]


@pytest.mark.parametrize("wt,M,N,K", FUSED)
def test_decode_fused_quantization(O, dev, wt, M, N, K):
    """The fused decode path (dcq_mul_mat_ex without workspace at M <= 8): block sums bit-exact
    (so the in-workgroup activation bytes and scales equal the standalone quantizer's) and
    outputs within tolerance, including exact rounding ties."""
    import torch
    wq, x = make_inputs(O, wt, M, N, K, seed=31 + M + K, outliers=1)
    x = _with_quantizer_ties(x, O.vec_dot_type(wt))
    y_ref, l1 = O.mul_mat(wt, wq, x)
    per = dc.block_sums_per_row(wt, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    y = dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=dc.PATH_GEMV, block_sums=sums)
    O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"fused type {wt} M{M} N{N} K{K}")
    want = O.block_sums_matrix(wt, K, wq, O.quantize_rows(O.vec_dot_type(wt), x))
    assert np.array_equal(to_host(sums), want)
    y2 = dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=dc.PATH_GEMV)
    O.assert_close(to_host(y2), y_ref, l1, RTOL, what="fused production kernel")


# SwiGLU gate/up pair: the fused kernels (Q4_K, Q5_K, Q8_0, Q4_0 at M <= 4, shapes of both launch
# families) and the general path (Q6_K; larger M: the batched and prefill kernels plus the product
# kernel). The two 64 x 2048 x 8192 shapes split K (few weight rows, long K): both products then use
# the split-K room past the U temporary, one after the other.
GATE_UP = [(Q4_K, 1, 97, 2560), (Q4_K, 1, 9728, 2560), (Q4_K, 5, 40, 1024), (Q8_0, 1, 96, 1024), (Q8_0, 3, 41, 2048),
           (Q6_K, 1, 50, 1024), (Q6_K, 3, 17, 768), (Q4_K, 33, 64, 512), (Q8_0, 40, 100, 512),
           (Q8_0, 64, 2048, 8192), (Q6_K, 64, 2048, 8192),
           (Q4_0, 1, 96, 1024), (Q4_0, 1, 96, 2560), (Q4_0, 6, 41, 2048), (Q5_K, 1, 97, 2560), (Q5_K, 1, 9728, 2560), (Q5_K, 3, 40, 1024),
           (Q5_K, 40, 64, 512)]


@pytest.mark.parametrize("wt,M,N,K", GATE_UP)
def test_ffn_gate_up(O, dev, wt, M, N, K):
    """dcq_ffn_gate_up = silu(Wg x) * (Wu x) against the oracle's pair of mul_mats and float64
    silu, within the propagated mul_mat tolerance: without a workspace, with the full one (split-K
    room included) and with the minimal one (no split-K room)."""
    import torch
    wg, x = make_inputs(O, wt, M, N, K, seed=61 + M + K, outliers=1)
    wu, _ = make_inputs(O, wt, M, N, K, seed=62 + M + K)
    print(f"gate/up type {wt} M={M} N={N} K={K}", flush=True)
    y_ref, parts = O.ffn_gate_up(wt, wg, wu, x)
    wgd, wud, xd = to_dev(wg, dev), to_dev(wu, dev), to_dev(x, dev)
    y = dc.ffn_gate_up(wt, wgd, wud, N, K, xd)
    O.assert_close_gate_up(to_host(y), y_ref, parts, RTOL, what=f"gate/up type {wt} M{M} N{N} K{K}")
    full = dc.ffn_gate_up_workspace_size(wt, M, N, K)
    for nbytes in (full, full - _split_tail(M)):
        ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device=dev)
        y2 = dc.ffn_gate_up(wt, wgd, wud, N, K, xd, workspace=ws)
        O.assert_close_gate_up(to_host(y2), y_ref, parts, RTOL, what=f"gate/up with a workspace of {nbytes} B")


@pytest.mark.parametrize("wt,M", [(Q4_K, 9), (Q6_K, 3), (Q8_0, 2), (Q4_0, 3), (Q4_0, 12), (Q5_K, 2), (Q5_K, 9)])
def test_mul_mat_padded_strides_and_workspace(O, dev, wt, M):
    """Row strides larger than the data (ggml nb[1] > row size) and a caller workspace."""
    import torch
    N, K = 45, 512
    wq, x = make_inputs(O, wt, M, N, K, seed=5)
    rs = dc.row_size(wt, K)
    wpad = np.zeros((N, rs + 64), np.uint8)
    wpad[:, :rs] = wq
    xpad = np.zeros((M, K + 16), np.float32)
    xpad[:, :K] = x
    ws = torch.empty(dc.mul_mat_workspace_size(wt, M, K), dtype=torch.uint8, device=dev)
    ybig = torch.full((M, N + 3), -7.0, dtype=torch.float32, device=dev)
    xd = to_dev(xpad, dev)[:, :K]
    dc.mul_mat(wt, to_dev(wpad, dev), N, K, xd, y=ybig[:, :N], workspace=ws, w_row_bytes=rs + 64)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    yb = to_host(ybig)
    O.assert_close(yb[:, :N], y_ref, l1, RTOL, what="strided")
    assert np.all(yb[:, N:] == -7.0)  # nothing written past each output row


def test_auto_path_is_consistent(O, dev):
    wt, N, K = Q8_0, 64, 1024
    wq, x = make_inputs(O, wt, 24, N, K, seed=9)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    for M in (1, 8, 9, 24):
        y = dc.mul_mat(wt, to_dev(wq, dev), N, K, to_dev(x[:M], dev))
        O.assert_close(to_host(y), y_ref[:M], l1[:M], RTOL, what=f"auto M={M}")


# ---------------------------------------------------------------- dot_rows (ComputeDotProductBatch)
@pytest.mark.parametrize("wt,K", [(Q8_0, 1024), (Q8_0, 96), (Q4_K, 2560), (Q6_K, 1024), (Q4_0, 1024), (Q4_0, 96),
                                  (Q5_K, 2560)])
def test_dot_rows(O, dev, wt, K):
    N = 50
    wq, x = make_inputs(O, wt, 1, N, K, seed=K)
    xq = O.quantize_rows(O.vec_dot_type(wt), x)[0]
    for n0, n1 in ((0, N), (7, 31), (49, 50)):
        got = to_host(dc.dot_rows(wt, to_dev(wq, dev), to_dev(xq, dev), K, n0, n1))
        want = O.dot_rows(wt, wq, xq, K, n0, n1)
        l1 = np.array([O.vec_dot_l1(wt, K, wq[r], xq) for r in range(n0, n1)])
        O.assert_close(got, want, l1, RTOL, what=f"dot_rows {n0}:{n1}")


# ---------------------------------------------------------------- weights
@pytest.mark.parametrize("wt", [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K])
def test_quantize_weights_bit_exact(O, dev, wt):
    N, K = 64, 2048
    w = synth.normal(N * K, 313, 0.0, 0.02).reshape(N, K)
    w[3, :512] = 0.0
    w[5, 100] = 0.9
    got = to_host(dc.quantize_weights(wt, to_dev(w, dev)))
    assert np.array_equal(got, O.quantize_matrix(wt, w))


@pytest.mark.parametrize("wt", [Q8_0, Q4_0, Q4_K, Q5_K, Q6_K])
def test_dequantize_rows(O, dev, wt):
    N, K = 16, 1024
    w = synth.normal(N * K, 314, 0.0, 0.02).reshape(N, K)
    wq = O.quantize_matrix(wt, w)
    got = to_host(dc.dequantize_rows(wt, to_dev(wq, dev), N, K))
    want = np.stack([O.dequantize_row(wt, wq[r], K) for r in range(N)])
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)


# ---------------------------------------------------------------- BASELINE configurations
@pytest.mark.parametrize("cfg", dc.CONFIGS, ids=lambda c: f"cfg{c.index}")
def test_baseline_config_parity(O, dev, cfg):
    """Full-size configs, every output against the oracle (config 5: all 2048 x 8192 outputs, so
    every 128-row m-tile and every n-tile of the XCD band remap is covered)."""
    w = synth.normal(cfg.N * cfg.K, cfg.w_seed, 0.0, cfg.w_std).reshape(cfg.N, cfg.K)
    wq = O.quantize_matrix(cfg.wtype, w)
    x = synth.normal(cfg.M * cfg.K, cfg.x_seed).reshape(cfg.M, cfg.K)
    if cfg.n_outliers:
        for m in range(cfg.M):
            synth.set_outliers(x[m], cfg.n_outliers, cfg.outlier_value, cfg.x_seed + 17 * m)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    print(f"config {cfg.index}: {cfg.name} M={cfg.M} N={cfg.N} K={cfg.K}", flush=True)
    y = to_host(dc.mul_mat(cfg.wtype, wd, cfg.N, cfg.K, xd))
    y_ref, l1 = O.mul_mat(cfg.wtype, wq, x)
    O.assert_close(y, y_ref, l1, RTOL, what=cfg.name)
    # reported, not asserted: the plain relative error, which cancelling outputs may push past
    # 1e-4 inside the L1-guarded bound above
    st = O.relative_error_stats(y, y_ref, RTOL)
    print(f"config {cfg.index} plain relative error over {st['n']} outputs: p50 {st['p50']:.3g} "
          f"p99 {st['p99']:.3g} max {st['max']:.3g}; {st['n_above']} above {RTOL:g}", flush=True)
    # the GPU weight quantizer produces the same bytes as the oracle on the config shape
    if cfg.index in (1, 2, 3):
        assert np.array_equal(to_host(dc.quantize_weights(cfg.wtype, to_dev(w, dev))), wq)


def test_config5_block_sums_full_shape_corner(O, dev):
    """Config 5 at its full shape through dcq_mul_mat_ex with the per-block int32 sums dumped by
    the production prefill kernel (the same tiling and XCD band remap): the last 8 activation
    rows x the first and last 64 weight rows, bit for bit against the oracle's block sums."""
    import torch
    cfg = dc.by_index(5)
    w = synth.normal(cfg.N * cfg.K, cfg.w_seed, 0.0, cfg.w_std).reshape(cfg.N, cfg.K)
    wq = O.quantize_matrix(cfg.wtype, w)
    x = synth.normal(cfg.M * cfg.K, cfg.x_seed).reshape(cfg.M, cfg.K)
    per = dc.block_sums_per_row(cfg.wtype, cfg.K)
    sums = torch.zeros((cfg.M, cfg.N, per), dtype=torch.int32, device=dev)  # 4.3 GB
    y = dc.mul_mat_ex(cfg.wtype, to_dev(wq, dev), cfg.N, cfg.K, to_dev(x, dev), path=dc.PATH_AUTO, block_sums=sums)
    rows = np.arange(cfg.M - 8, cfg.M)
    cols = np.r_[0:64, cfg.N - 64:cfg.N]
    got = to_host(sums[rows[0]:, :, :])[:, cols, :]
    yc = to_host(y[rows[0]:, :])[:, cols]
    del sums
    torch.cuda.empty_cache()
    xq = O.quantize_rows(O.vec_dot_type(cfg.wtype), x[rows])
    want = O.block_sums_matrix(cfg.wtype, cfg.K, wq[cols], xq)
    assert np.array_equal(got, want)
    y_ref, l1 = O.mul_mat(cfg.wtype, wq[cols], x[rows])
    O.assert_close(yc, y_ref, l1, RTOL, what="config 5 corner")


# ---------------------------------------------------------------- split operator (shared quantization)
@pytest.mark.parametrize("path", [dc.PATH_AUTO, dc.PATH_GEMV, dc.PATH_MMQ])
@pytest.mark.parametrize("wt,M,N,K", [(Q8_0, 1, 70, 1024), (Q4_K, 1, 96, 2560), (Q4_K, 5, 64, 2048),
                                      (Q4_K, 8, 40, 768), (Q6_K, 3, 33, 1024), (Q4_0, 2, 70, 1024),
                                      (Q5_K, 6, 40, 768)])
def test_quantize_src1_then_mul_mat_q(O, dev, wt, M, N, K, path):
    """dcq_quantize_src1 once, then dcq_mul_mat_q for two weights sharing X (ffn gate and up):
    the planar-activation kernels, against the oracle."""
    import torch
    wq_a, x = make_inputs(O, wt, M, N, K, seed=11 + M)
    wq_b, _ = make_inputs(O, wt, M, N, K, seed=12 + M)
    ws = torch.empty(dc.mul_mat_workspace_size(wt, M, K), dtype=torch.uint8, device=dev)
    dc.quantize_src1(wt, to_dev(x, dev), ws)
    for wq in (wq_a, wq_b):
        y = dc.mul_mat_q(wt, to_dev(wq, dev), N, K, ws, M, path=path)
        y_ref, l1 = O.mul_mat(wt, wq, x)
        O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"split type {wt} M{M} path {path}")


# ---------------------------------------------------------------- GGUF ingest to HBM
def test_gguf_load_to_device_and_mul_mat(O, dev, tmp_path):
    """Tensors of a Q4_K_M-style file (Q4_K, Q6_K, Q8_0, F32) streamed into device memory
    byte-exact, including one larger than a 32 MB transfer chunk, and a loaded weight used by
    dcq_mul_mat directly (rows packed in the file as dcq_mul_mat reads them)."""
    import torch
    from gguf_writer import T_STR, write_gguf
    shapes = [("blk.0.ffn_up.weight", Q4_K, 96, 2560), ("blk.0.ffn_down.weight", Q6_K, 40, 1024),
              ("blk.0.attn_q.weight", Q8_0, 33, 512)]
    tensors, weights = [], {}
    for i, (name, wt, n, k) in enumerate(shapes):
        wq = O.quantize_matrix(wt, synth.normal(n * k, 700 + i, 0.0, 0.02).reshape(n, k))
        weights[name] = (wt, n, k, wq)
        tensors.append((name, wt, [k, n], wq.tobytes()))
    big = np.frombuffer(synth.normal(9 * 2 ** 20, 777).tobytes(), dtype=np.uint8)  # 36 MiB of F32
    tensors.append(("token_embd.weight", 0, [len(big) // 4], big.tobytes()))
    path = tmp_path / "model.gguf"
    write_gguf(path, [("general.architecture", T_STR, "qwen3")], tensors, alignment=32)
    with dc.GGUF(path) as g:
        assert g.get_str("general.architecture") == "qwen3"
        for name, t, ne, data in tensors:
            i = g.find(name)
            d = g.load(i, device=dev)
            assert np.array_equal(to_host(d), np.frombuffer(data, dtype=np.uint8)), name
        for name, (wt, n, k, wq) in weights.items():
            w_dev = g.load(g.find(name), device=dev).view(n, -1)
            x = synth.normal(3 * k, 800).reshape(3, k)
            y = dc.mul_mat(wt, w_dev, n, k, to_dev(x, dev))
            y_ref, l1 = O.mul_mat(wt, wq, x)
            O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"mul_mat on loaded {name}")


# ---------------------------------------------------------------- projections sharing X (Q/K/V)
@pytest.mark.parametrize("wt", [Q4_K, Q8_0])
def test_concatenated_projections_one_call(O, dev, tmp_path, wt):
    """The Q/K/V projections (core/src/inference.cpp:1128-1130) share X. Loaded back to back into
    one device buffer (same type and K, so the same row bytes), one dcq_mul_mat over the
    concatenated rows gives [Q | K | V] per activation row: each slice against the oracle's
    separate product. Loaded through the GGUF reader, as an integration would."""
    import torch
    from gguf_writer import write_gguf
    K = 2560 if wt == Q4_K else 1024
    parts = [("blk.0.attn_q.weight", 512), ("blk.0.attn_k.weight", 128), ("blk.0.attn_v.weight", 128)]
    wqs, tensors = [], []
    for i, (name, n) in enumerate(parts):
        wq = O.quantize_matrix(wt, synth.normal(n * K, 900 + i, 0.0, 0.02).reshape(n, K))
        wqs.append(wq)
        tensors.append((name, wt, [K, n], wq.tobytes()))
    path = tmp_path / "qkv.gguf"
    write_gguf(path, [], tensors)
    rb = dc.row_size(wt, K)
    n_all = sum(n for _, n in parts)
    buf = torch.empty((n_all, rb), dtype=torch.uint8, device=dev)
    with dc.GGUF(path) as g:
        r0 = 0
        for name, n in parts:
            g.load(g.find(name), dst=buf[r0:r0 + n])
            r0 += n
    for M in (1, 3):
        x = synth.normal(M * K, 950 + M).reshape(M, K)
        y = to_host(dc.mul_mat(wt, buf, n_all, K, to_dev(x, dev)))
        r0 = 0
        for (name, n), wq in zip(parts, wqs):
            y_ref, l1 = O.mul_mat(wt, wq, x)
            O.assert_close(y[:, r0:r0 + n], y_ref, l1, RTOL, what=f"{name} slice, M={M}")
            r0 += n


# ---------------------------------------------------------------- projection + residual / bias
# The shapes cover every kernel family the add rides on: the fused Q4_K (5-wave and 4-wave
# launches, several rows), Q8_0 and Q6_K decode kernels (add in the store), the Q6_K decode that
# quantizes first (K > 4096) and the batched / prefill MFMA kernels (add kernel after).
MUL_MAT_ADD = [(Q4_K, 1, 2560, 9728), (Q4_K, 1, 97, 2560), (Q4_K, 5, 40, 1024), (Q8_0, 1, 1024, 2048),
               (Q8_0, 3, 41, 2048), (Q6_K, 1, 1024, 2560), (Q6_K, 1, 2560, 9728), (Q6_K, 2, 70, 4096),
               (Q4_K, 64, 96, 512), (Q8_0, 130, 64, 1024), (Q6_K, 9, 33, 512),
               (Q4_0, 1, 1024, 2048), (Q4_0, 20, 64, 512), (Q5_K, 1, 2560, 9728), (Q5_K, 9, 33, 512)]


@pytest.mark.parametrize("mode", ["residual", "in_place", "bias"])
@pytest.mark.parametrize("wt,M,N,K", MUL_MAT_ADD)
def test_mul_mat_add(O, dev, wt, M, N, K, mode):
    """dcq_mul_mat_add = the same call's dcq_mul_mat output + R, one float32 add per element,
    bit for bit (the reference's ggml_add on the projection); the product itself within the
    oracle's tolerance. R is a separate [M, N] residual, Y itself, or a broadcast [N] bias."""
    import torch
    wq, x = make_inputs(O, wt, M, N, K, seed=71 + M + N, outliers=1)
    r = synth.normal((1 if mode == "bias" else M) * N, 72 + M, 0.0, 3.0).reshape(-1, N)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    y_mm = to_host(dc.mul_mat(wt, wd, N, K, xd))
    y_ref, l1 = O.mul_mat(wt, wq, x)
    O.assert_close(y_mm, y_ref, l1, RTOL, what=f"product type {wt} M{M} N{N} K{K}")
    want = (y_mm + r).astype(np.float32)  # float32 + float32, rounded once
    for ws in (None, torch.empty(dc.mul_mat_add_workspace_size(wt, M, N, K), dtype=torch.uint8, device=dev)):
        if mode == "in_place":
            y = to_dev(r, dev)
            dc.mul_mat_add(wt, wd, N, K, xd, y, y=y, workspace=ws)
        elif mode == "bias":
            y = dc.mul_mat_add(wt, wd, N, K, xd, to_dev(r[0], dev), workspace=ws)
        else:
            y = dc.mul_mat_add(wt, wd, N, K, xd, to_dev(r, dev), workspace=ws)
        got = to_host(y)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"{mode} type {wt} M{M} N{N} K{K} workspace={ws is not None}"


def test_mul_mat_add_strided_residual(O, dev):
    """Residual and output rows inside wider buffers: nothing written past each output row."""
    import torch
    wt, M, N, K = Q4_K, 3, 45, 512
    wq, x = make_inputs(O, wt, M, N, K, seed=80)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    y_mm = to_host(dc.mul_mat(wt, wd, N, K, xd))
    rbig = synth.normal(M * (N + 7), 81).reshape(M, N + 7)
    ybig = torch.full((M, N + 3), -7.0, dtype=torch.float32, device=dev)
    dc.mul_mat_add(wt, wd, N, K, xd, to_dev(rbig, dev)[:, :N], y=ybig[:, :N])
    yb = to_host(ybig)
    assert np.array_equal(yb[:, :N], (y_mm + rbig[:, :N]).astype(np.float32))
    assert np.all(yb[:, N:] == -7.0)


@pytest.mark.parametrize("wt,M,N,K", [(Q4_K, 520, 16400, 256), (Q6_K, 520, 16400, 256), (Q8_0, 30, 16400, 256),
                                      (Q5_K, 520, 16400, 256), (Q4_0, 520, 16400, 256)])
def test_mul_mat_large_tiles(O, dev, wt, M, N, K):
    """Shapes that take the large-tile kernels (64 x 256 workgroup tiles for Q4_K / Q6_K at
    >= 512 tiles; ragged M and N): the output against the oracle, and the exact per-block
    integer sums on a corner of rows and columns (the oracle's sums are slow at full size)."""
    import torch
    wq, x = make_inputs(O, wt, M, N, K, seed=90 + wt, outliers=1)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    per = dc.block_sums_per_row(wt, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    y = dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=dc.PATH_MMQ, block_sums=sums)
    O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"large tiles type {wt} M{M} N{N} K{K}")
    rows = np.r_[0:8, M - 8:M]
    cols = np.r_[0:64, N - 64:N]
    want = O.block_sums_matrix(wt, K, wq[cols], O.quantize_rows(O.vec_dot_type(wt), x[rows]))
    got = to_host(sums)[rows][:, cols]
    assert np.array_equal(got, want)
    y2 = dc.mul_mat(wt, to_dev(wq, dev), N, K, to_dev(x, dev))
    O.assert_close(to_host(y2), y_ref, l1, RTOL, what="production kernel")


# ---------------------------------------------------------------- the LM head (output projection)
def _random_blocks(wt, N, K, rng):
    """Valid weight rows of random quants with small positive fp16 scales (generating N(0, 0.02)
    floats and quantizing 150 k rows would dominate the test; the kernels see the same bytes
    either way)."""
    rb = dc.row_size(wt, K)
    q = rng.integers(0, 256, size=(N, rb), dtype=np.uint8)
    scale = np.frombuffer(np.float16(0.0004).tobytes(), dtype=np.uint8)
    if wt in (Q8_0, Q4_0):
        blk = q.reshape(N, K // 32, 34 if wt == Q8_0 else 18)
        blk[:, :, 0:2] = scale
    elif wt in (Q4_K, Q5_K):  # d, dmin, then 12 bytes of 6-bit scales and mins (random), (qh,) nibbles
        blk = q.reshape(N, K // 256, 144 if wt == Q4_K else 176)
        blk[:, :, 0:2] = scale
        blk[:, :, 2:4] = np.frombuffer(np.float16(0.0002).tobytes(), dtype=np.uint8)
    else:  # Q6_K: 16 int8 sub-scales (random), d last
        blk = q.reshape(N, K // 256, 210)
        blk[:, :, 208:210] = scale
    return q


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("wt,K", [(Q8_0, 1024), (Q6_K, 2560)])
def test_lm_head_parity(O, dev, wt, K, M):
    """The LM head, the largest weight stream of a decode step (ggml_mul_mat(output, cur),
    core/src/inference.cpp:1817): Qwen3's 151,936-token vocabulary at Qwen3-0.6B's width (Q8_0,
    K = 1024, 165 MB) and at Qwen3-4B's (Q6_K, the Q4_K_M type of output.weight, K = 2560, 319 MB),
    one and four tokens, every output against the oracle."""
    N = 151936
    rng = np.random.default_rng(151936 + K + M)
    wq = _random_blocks(wt, N, K, rng)
    x = synth.normal(M * K, 4000 + M + K).reshape(M, K)
    print(f"lm head type {wt} M={M} N={N} K={K}", flush=True)
    y = to_host(dc.mul_mat(wt, to_dev(wq, dev), N, K, to_dev(x, dev)))
    y_ref, l1 = O.mul_mat(wt, wq, x)
    O.assert_close(y, y_ref, l1, RTOL, what=f"lm head type {wt} M={M}")


# Tall Q6_K matrices (32768+ rows at K <= 4096): each wave streams 2, 4 or 8 rows through two LDS
# images, the next row's loads in flight while the current one computes. Rows not a multiple of
# the rows per workgroup (tails of every length), the fused kernel (M <= 2) and the one over a
# quantized activation (M = 3, M = 9: two tiles of rows), block sums and the residual add. The
# MFMA kernel for tall matrices splits each 32-row tile into two halves of its superblocks, summed
# in LDS, when the tiles are fewer than its waves (40003 rows at M = 9: 1251 tiles for 2048 waves);
# 70001+ rows keep whole tiles. One activation row over fewer than 65536 rows of up to 16
# superblocks (40001 x 1024) takes the fused LDS kernel instead.
TALL_Q6 = [(1, 40001, 1024), (2, 70003, 512), (3, 70001, 1024), (9, 40003, 512), (1, 139999, 1536)]


@pytest.mark.parametrize("M,N,K", TALL_Q6)
def test_q6k_rows_per_wave(O, dev, M, N, K):
    import torch
    rng = np.random.default_rng(N + K + M)
    wq = _random_blocks(Q6_K, N, K, rng)
    x = synth.normal(M * K, 500 + M + K).reshape(M, K)
    synth.set_outliers(x[0], max(1, K // 100), 20.0, 3)
    print(f"tall q6_k M={M} N={N} K={K}", flush=True)
    y_ref, l1 = O.mul_mat(Q6_K, wq, x)
    per = dc.block_sums_per_row(Q6_K, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    y = dc.mul_mat_ex(Q6_K, wd, N, K, xd, path=dc.PATH_GEMV, block_sums=sums)
    O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"tall q6_k M{M} N{N} K{K}")
    want = O.block_sums_matrix(Q6_K, K, wq, O.quantize_rows(Q8_K, x))
    assert np.array_equal(to_host(sums), want)
    y2 = to_host(dc.mul_mat(Q6_K, wd, N, K, xd))
    O.assert_close(y2, y_ref, l1, RTOL, what="tall q6_k production kernel")
    r = synth.normal(M * N, 700 + M, 0.0, 3.0).reshape(M, N)
    y3 = to_host(dc.mul_mat_add(Q6_K, wd, N, K, xd, to_dev(r, dev)))
    assert np.array_equal(y3.view(np.uint32), (y2 + r).astype(np.float32).view(np.uint32))


# K-quant prefill at config 5's shape (2048 x 8192 x 2048), the projection shape of a Q4_K_M
# prompt: every 128-row m-tile boundary row and interior rows against the oracle on all 8192
# outputs, and the per-superblock int32 sums of a full-shape corner bit for bit.
@pytest.mark.parametrize("wt", [Q4_K, Q6_K])
def test_kquant_prefill_full_shape(O, dev, wt):
    import torch
    M, N, K = 2048, 8192, 2048
    rng = np.random.default_rng(2048 + wt)
    wq = _random_blocks(wt, N, K, rng)
    x = synth.normal(M * K, 9000 + wt).reshape(M, K)
    for m in range(0, M, 97):
        synth.set_outliers(x[m], 20, 20.0, m)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    print(f"k-quant prefill type {wt} M={M} N={N} K={K}", flush=True)
    y = to_host(dc.mul_mat(wt, wd, N, K, xd))
    rows = np.unique(np.r_[np.arange(0, M, 128), np.arange(127, M, 128), 1, 500, 1000, 1234, 1999])
    y_ref, l1 = O.mul_mat(wt, wq, x[rows])
    O.assert_close(y[rows], y_ref, l1, RTOL, what=f"k-quant prefill type {wt}")
    per = dc.block_sums_per_row(wt, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    y2 = dc.mul_mat_ex(wt, wd, N, K, xd, path=dc.PATH_AUTO, block_sums=sums)
    corner = np.arange(M - 8, M)
    cols = np.r_[0:64, N - 64:N]
    got = to_host(sums[corner[0]:, :, :])[:, cols, :]
    del sums
    torch.cuda.empty_cache()
    want = O.block_sums_matrix(wt, K, wq[cols], O.quantize_rows(Q8_K, x[corner]))
    assert np.array_equal(got, want)
    assert np.array_equal(to_host(y2), y)  # the dump does not change the outputs


# Split-K: products whose 128 x 128 output tiles cannot occupy every CU (few weight rows, long K:
# ffn_down-like 2048 x 8192 at batch sizes) cut K into ranges whose partial tiles go to the
# workspace's split-K room and are summed in range order. Each case against the oracle on every
# output, with the full workspace (split) and with one that holds only the quantized activation
# (no split); repeated calls give the same bits.
SPLIT_K = [(Q8_0, 64, 2048, 8192), (Q6_K, 64, 2048, 8192), (Q4_K, 256, 2048, 8192), (Q8_0, 40, 1000, 4096),
           (Q6_K, 200, 384, 2048), (Q4_K, 130, 256, 4096), (Q8_0, 16, 2048, 8192), (Q6_K, 9, 2048, 8192),
           (Q8_0, 256, 8192, 2048), (Q4_0, 64, 2048, 8192), (Q4_0, 16, 2048, 8192), (Q4_0, 200, 384, 2048),
           (Q5_K, 64, 2048, 8192), (Q5_K, 256, 2048, 8192), (Q5_K, 130, 256, 4096)]


def _split_tail(M):
    return min(M, 128) * 128 * 1024 if M > 4 else 0


@pytest.mark.parametrize("wt,M,N,K", SPLIT_K)
def test_split_k_parity(O, dev, wt, M, N, K):
    import torch
    rng = np.random.default_rng(7000 + M + N)
    wq = _random_blocks(wt, N, K, rng)
    x = synth.normal(M * K, 7100 + N).reshape(M, K)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    full = dc.mul_mat_workspace_size(wt, M, K)
    print(f"split-K type {wt} M={M} N={N} K={K}", flush=True)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    outs = []
    for nbytes in (full, full - _split_tail(M), full):
        ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device=dev)
        y = to_host(dc.mul_mat(wt, wd, N, K, xd, workspace=ws))
        O.assert_close(y, y_ref, l1, RTOL, what=f"split-K type {wt} M={M} N={N} K={K} ws={nbytes}")
        outs.append(y)
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    # dcq_mul_mat_q only reads its workspace and never splits: the activation-only result's bits,
    # and the workspace past the quantized activation is left as it was
    ws = torch.full((full,), 0xAB, dtype=torch.uint8, device=dev)
    dc.quantize_src1(wt, xd, ws)
    yq = to_host(dc.mul_mat_q(wt, wd, N, K, ws, M))
    assert np.array_equal(yq.view(np.uint32), outs[1].view(np.uint32))
    assert bool((ws[full - _split_tail(M):] == 0xAB).all())


@pytest.mark.parametrize("wt,M,N,K", [(Q6_K, 64, 256, 4096), (Q8_0, 48, 384, 2048), (Q4_K, 160, 256, 2048),
                                      (Q4_0, 48, 384, 2048), (Q5_K, 160, 256, 2048), (Q5_K, 64, 256, 4096)])
def test_split_k_block_sums(O, dev, wt, M, N, K):
    """The per-block int32 sums dumped by split-K ranges: every block written once, bit-exact."""
    import torch
    rng = np.random.default_rng(7300 + wt)
    wq = _random_blocks(wt, N, K, rng)
    x = synth.normal(M * K, 7400 + wt).reshape(M, K)
    per = dc.block_sums_per_row(wt, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    ws = torch.empty(dc.mul_mat_workspace_size(wt, M, K), dtype=torch.uint8, device=dev)
    y = to_host(dc.mul_mat_ex(wt, to_dev(wq, dev), N, K, to_dev(x, dev), path=dc.PATH_AUTO, block_sums=sums,
                              workspace=ws))
    want = O.block_sums_matrix(wt, K, wq, O.quantize_rows(O.vec_dot_type(wt), x))
    assert np.array_equal(to_host(sums), want)
    y_ref, l1 = O.mul_mat(wt, wq, x)
    O.assert_close(y, y_ref, l1, RTOL, what=f"split-K sums type {wt}")


# Batched decode past four rows (Q6_K on matrices of 4096+ rows: past two): Q8_0, Q4_0 and Q6_K on
# their batch kernels (one or two 32-row m-tiles, K split over the waves and, with few weight rows,
# over workgroups), Q4_K and Q5_K on theirs (Q5_K: the extra MFMA of the fifth bits).
# Every output against the oracle, and the per-block int32 sums bit for bit.
BATCH_SMALL_M = [(Q8_0, 5, 100, 1024), (Q8_0, 8, 8192, 2048), (Q8_0, 16, 2048, 8192), (Q8_0, 32, 96, 256),
                 (Q8_0, 33, 130, 2048), (Q8_0, 64, 2048, 8192), (Q8_0, 64, 8192, 2048), (Q8_0, 7, 33, 4096),
                 (Q4_K, 6, 300, 2048), (Q4_K, 8, 2048, 8192), (Q4_K, 64, 2048, 8192), (Q4_K, 100, 1000, 4096),
                 (Q6_K, 5, 100, 1024), (Q6_K, 8, 8192, 2048), (Q6_K, 16, 2048, 8192), (Q6_K, 33, 130, 2048),
                 (Q6_K, 64, 2048, 8192), (Q6_K, 20, 77, 512), (Q6_K, 3, 4096, 1024), (Q6_K, 4, 8192, 2048),
                 (Q4_0, 5, 100, 1024), (Q4_0, 16, 2048, 8192), (Q4_0, 33, 130, 2048), (Q4_0, 64, 8192, 2048),
                 (Q5_K, 6, 300, 2048), (Q5_K, 8, 2048, 8192), (Q5_K, 64, 8192, 2048), (Q5_K, 100, 1000, 4096)]


@pytest.mark.parametrize("wt,M,N,K", BATCH_SMALL_M)
def test_batch_small_m(O, dev, wt, M, N, K):
    import torch
    rng = np.random.default_rng(7500 + M + N)
    wq = _random_blocks(wt, N, K, rng)
    x = synth.normal(M * K, 7600 + K).reshape(M, K)
    x[0, :32] = 0.0  # an all-zero block (scale 0)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    print(f"batch small M type {wt} M={M} N={N} K={K}", flush=True)
    ws = torch.full((dc.mul_mat_workspace_size(wt, M, K),), 0xAB, dtype=torch.uint8, device=dev)
    y = to_host(dc.mul_mat(wt, wd, N, K, xd, workspace=ws))
    y_ref, l1 = O.mul_mat(wt, wq, x)
    O.assert_close(y, y_ref, l1, RTOL, what=f"batch type {wt} M={M} N={N} K={K}")
    if N * K <= 2048 * 8192:
        per = dc.block_sums_per_row(wt, K)
        sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
        y2 = to_host(dc.mul_mat_ex(wt, wd, N, K, xd, path=dc.PATH_AUTO, block_sums=sums, workspace=ws))
        want = O.block_sums_matrix(wt, K, wq, O.quantize_rows(O.vec_dot_type(wt), x))
        assert np.array_equal(to_host(sums), want)
        O.assert_close(y2, y_ref, l1, RTOL, what=f"batch type {wt} with sums")
