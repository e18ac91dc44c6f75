"""GPU: row-split Q8_0 weights (DCQ_TYPE_Q8_0_RS, the load-time repack of Q8_0 rows).

The repack is a byte rearrangement, so its bytes are checked against the oracle's restatement, and
every product from the repacked rows against the oracle (the Q8_0 bar: block sums bit-exact,
outputs within 1e-4 * max(|y_ref|, L1)) and, bit for bit, against the same call on the Q8_0 rows:
the kernels and their arithmetic are the Q8_0 ones.
"""
import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, RS = dc.TYPE_Q8_0, dc.TYPE_Q8_0_RS
RTOL = 1e-4


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make(O, M, N, K, seed):
    w = synth.normal(N * K, 4000 + seed, 0.0, 0.02).reshape(N, K)
    if N > 2:
        w[1, :K // 2] = 0.0
    x = synth.normal(M * K, 5000 + seed).reshape(M, K)
    if M > 1:
        x[M - 1, :256] = 0.0
    return O.quantize_matrix(Q8_0, w), x


@pytest.mark.parametrize("N,K,pad_in,pad_out", [(3, 256, 0, 0), (70, 2048, 6, 16), (5, 9728, 0, 32)])
def test_repack_bytes(O, dev, N, K, pad_in, pad_out):
    import torch
    wq, _ = make(O, 1, N, K, N + K)
    rb = dc.row_size(Q8_0, K)
    src = np.zeros((N, rb + pad_in), dtype=np.uint8)
    src[:, :rb] = wq
    out = torch.full((N, dc.row_size(RS, K) + pad_out), 0xA5, dtype=torch.uint8, device=dev)
    dc.repack_weights(Q8_0, to_dev(src, dev), N, K, RS, out=out, w_row_bytes=rb + pad_in)
    got = to_host(out)
    assert np.array_equal(got[:, :dc.row_size(RS, K)], O.repack_q8_0_rs(wq, K))
    assert (got[:, dc.row_size(RS, K):] == 0xA5).all()  # the padding is not written
    d8 = to_host(dc.dequantize_rows(Q8_0, to_dev(wq, dev), N, K))
    dr = to_host(dc.dequantize_rows(RS, out, N, K, w_row_bytes=out.stride(0)))
    assert np.array_equal(d8, dr)


# decode (fused: 1..4 rows; the generic kernel past the fused LDS room), batched (5..64 rows, split
# K over workgroups for few weight rows), 128 x 128 tiles (ragged, full, split K)
SHAPES = [(1, 96, 1024), (3, 70, 2048), (4, 41, 4096), (2, 33, 8192), (8, 64, 16384), (5, 300, 1024),
          (16, 2048, 8192), (64, 96, 2048), (33, 130, 2048), (130, 257, 256), (256, 384, 1024), (200, 384, 2048)]


@pytest.mark.parametrize("path", [dc.PATH_AUTO, dc.PATH_GEMV, dc.PATH_MMQ])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_mul_mat_row_split(O, dev, M, N, K, path):
    import torch
    wq, x = make(O, M, N, K, M * 7 + N + K)
    wd = to_dev(wq, dev)
    wr = dc.repack_weights(Q8_0, wd, N, K, RS)
    xd = to_dev(x, dev)
    y_ref, l1 = O.mul_mat(Q8_0, wq, x)
    per = dc.block_sums_per_row(RS, K)
    sums = torch.zeros((M, N, per), dtype=torch.int32, device=dev)
    y = dc.mul_mat_ex(RS, wr, N, K, xd, path=path, block_sums=sums)
    O.assert_close(to_host(y), y_ref, l1, RTOL, what=f"row-split M{M} N{N} K{K} path {path}")
    want = O.block_sums_matrix(Q8_0, K, wq, O.quantize_rows(Q8_0, x))
    assert np.array_equal(to_host(sums), want)
    # the production kernels: the Q8_0 rows' bits
    y_rs = to_host(dc.mul_mat_ex(RS, wr, N, K, xd, path=path))
    y_q8 = to_host(dc.mul_mat_ex(Q8_0, wd, N, K, xd, path=path))
    assert np.array_equal(y_rs, y_q8)


@pytest.mark.parametrize("M,N,K", [(1, 96, 1024), (5, 300, 1024), (130, 257, 2048)])
def test_row_split_other_entry_points(O, dev, M, N, K):
    """mul_mat_q after quantize_src1, mul_mat_add, the allocation-free entry point and dot_rows give
    the Q8_0 rows' bits; the gate/up pair agrees with the Q8_0 pair to the fp32 tolerance."""
    import torch
    wq, x = make(O, M, N, K, 3 * M + N)
    wd, xd = to_dev(wq, dev), to_dev(x, dev)
    wr = dc.repack_weights(Q8_0, wd, N, K, RS)
    ws = torch.empty(dc.mul_mat_workspace_size(RS, M, K), dtype=torch.uint8, device=dev)
    dc.quantize_src1(RS, xd, ws)
    same = lambda a, b: np.array_equal(to_host(a), to_host(b))
    assert same(dc.mul_mat_q(RS, wr, N, K, ws, M), dc.mul_mat_q(Q8_0, wd, N, K, ws, M))
    r = torch.randn((M, N), device=dev)
    assert same(dc.mul_mat_add(RS, wr, N, K, xd, r), dc.mul_mat_add(Q8_0, wd, N, K, xd, r))
    y1 = torch.empty((M, N), dtype=torch.float32, device=dev)
    y2 = torch.empty((M, N), dtype=torch.float32, device=dev)
    assert same(dc.mul_mat_noalloc(RS, wr, N, K, xd, y1), dc.mul_mat_noalloc(Q8_0, wd, N, K, xd, y2))
    xq = dc.quantize_rows(Q8_0, xd[:1])
    assert same(dc.dot_rows(RS, wr, xq[0], K, 0, N), dc.dot_rows(Q8_0, wd, xq[0], K, 0, N))
    wq2, _ = make(O, M, N, K, 3 * M + N + 1)
    wd2 = to_dev(wq2, dev)
    wr2 = dc.repack_weights(Q8_0, wd2, N, K, RS)
    y_ref, parts = O.ffn_gate_up(Q8_0, wq, wq2, x)
    O.assert_close_gate_up(to_host(dc.ffn_gate_up(RS, wr, wr2, N, K, xd)), y_ref, parts, RTOL, what="row-split gate/up")


def test_config5_row_split_full_shape(O, dev):
    """Config 5's shape (M = 2048, N = 8192, K = 2048) on repacked rows: the Q8_0 rows' bits."""
    cfg = dc.by_index(5)
    import bench
    wq, x, _ = bench.make_config_inputs(cfg, dev)
    wr = dc.repack_weights(Q8_0, wq, cfg.N, cfg.K, RS)
    y_rs = to_host(dc.mul_mat(RS, wr, cfg.N, cfg.K, x))
    y_q8 = to_host(dc.mul_mat(Q8_0, wq, cfg.N, cfg.K, x))
    assert np.array_equal(y_rs, y_q8)
