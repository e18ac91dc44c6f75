"""The C ABI of libdcq without a GPU: symbols, type traits, argument validation.

Validation runs on the host before any device call, so every error path here is
exercised on the CPU; a well-formed call on a machine without a gfx950 device
must fail loudly with DCQ_ERR_NO_DEVICE (no CPU fallback).
"""
import ctypes
import os
import re

import pytest

import densecore_amd as dc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OK, INVALID, UNSUPPORTED, BAD_SHAPE, MISALIGNED, WORKSPACE, HIP, NO_DEVICE = 0, -1, -2, -3, -4, -5, -6, -7


def declared_symbols():
    inc = os.path.join(ROOT, "include")
    text = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dcq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = dc.lib()
    names = declared_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(dc._lib.SYMBOLS)


def test_version_and_status_strings():
    assert "gfx950" in dc.version()
    for s in (OK, INVALID, UNSUPPORTED, BAD_SHAPE, MISALIGNED, WORKSPACE, HIP, NO_DEVICE):
        assert dc._lib.status_string(s) != "unknown status"


def test_type_traits_match_gguf():
    assert [dc.block_size(t) for t in (0, 1, 2, 8, 12, 13, 14, 15, 3)] == [1, 1, 32, 32, 256, 256, 256, 256, 0]
    assert [dc.type_size(t) for t in (0, 1, 2, 8, 12, 13, 14, 15)] == [4, 2, 18, 34, 144, 176, 210, 292]
    assert dc.row_size(2, 2560) == 1440
    assert dc.row_size(13, 2560) == 1760
    assert dc.row_size(8, 1024) == 1088
    assert dc.row_size(12, 2560) == 1440
    assert dc.row_size(14, 9728) == 7980
    assert dc.row_size(15, 2560) == 2920
    assert dc.row_size(12, 100) == 0
    assert [dc.vec_dot_type(t) for t in (2, 8, 12, 13, 14)] == [8, 8, 15, 15, 15]
    assert dc.vec_dot_type(0) == UNSUPPORTED and dc.vec_dot_type(3) == UNSUPPORTED
    assert dc.supports_mul_mat(12, 0, 0) and not dc.supports_mul_mat(12, 1, 0) and not dc.supports_mul_mat(3, 0, 0)
    assert dc.supports_mul_mat(2, 0, 0) and dc.supports_mul_mat(13, 0, 0)
    assert dc.block_sums_per_row(8, 1024) == 32
    assert dc.block_sums_per_row(12, 2560) == 20
    assert dc.block_sums_per_row(14, 9728) == 38
    assert dc.block_sums_per_row(2, 1024) == 32
    assert dc.block_sums_per_row(13, 2560) == 20


def test_workspace_size():
    # planar: int8 [M][K] + fp32 scales [K/bs][roundup(M, 128)] (+ int16 bsums [M][K/16] for Q8_K),
    # then at M > 4 the split-K room, min(M, 128) * 128 KB
    assert dc.mul_mat_workspace_size(8, 1, 1024) == 1024 + 32 * 128 * 4
    assert dc.mul_mat_workspace_size(8, 4, 1024) == 4 * 1024 + 32 * 128 * 4
    assert dc.mul_mat_workspace_size(8, 8, 1024) == 8 * 1024 + 32 * 128 * 4 + 8 * 131072
    assert dc.mul_mat_workspace_size(8, 32, 1024) == 32 * 1024 + 32 * 128 * 4 + 32 * 131072
    assert dc.mul_mat_workspace_size(12, 64, 2048) == 64 * 2048 + 8 * 128 * 4 + 64 * 128 * 2 + 64 * 131072
    assert dc.mul_mat_workspace_size(8, 130, 1024) == 130 * 1024 + 32 * 256 * 4 + 128 * 131072
    assert dc.mul_mat_workspace_size(12, 1, 100) == 0


def _mm(wt=12, W=0x1000, N=16, K=256, wrb=None, X=0x2000, M=1, xs=None, Y=0x3000, ys=None, ws=None, wsb=0,
        path=0, sums=None):
    wrb = dc.row_size(wt, K) if wrb is None else wrb
    xs = K * 4 if xs is None else xs
    ys = N * 4 if ys is None else ys
    return dc.lib().dcq_mul_mat_ex(wt, W, N, K, wrb, X, M, xs, Y, ys, ws, wsb, path, sums, None)


def test_mul_mat_validation_order():
    """Argument errors are reported before any device call."""
    assert _mm(wt=3) == UNSUPPORTED  # Q4_1: not a weight type of this library
    assert _mm(W=None) == INVALID
    assert _mm(K=100) == BAD_SHAPE
    assert _mm(N=0) == BAD_SHAPE
    assert _mm(M=0) == BAD_SHAPE
    assert _mm(wrb=100) == INVALID
    assert _mm(xs=16) == INVALID
    assert _mm(W=0x1004) == MISALIGNED
    assert _mm(X=0x2004) == MISALIGNED
    assert _mm(wt=12, wrb=152) == MISALIGNED  # Q4_K rows must keep 16-byte alignment
    assert _mm(wt=13, wrb=184) == MISALIGNED  # so must Q5_K rows
    assert _mm(wt=2, wrb=145) == MISALIGNED   # odd row strides never
    assert _mm(path=7) == INVALID
    assert _mm(ws=0x4000, wsb=16) == WORKSPACE
    assert _mm(ws=0x4010, wsb=1 << 20) == MISALIGNED


def test_row_split_q8_0_traits_and_validation():
    """DCQ_TYPE_Q8_0_RS (108): Q8_0's block traits and activation type; rows K % 256 == 0 and 16-byte
    row strides; the repack takes Q8_0 -> row-split only, rejects overlap, all before any device call."""
    L = dc.lib()
    RS = dc.TYPE_Q8_0_RS
    assert RS == 108
    assert (dc.block_size(RS), dc.type_size(RS), dc.row_size(RS, 2048)) == (32, 34, 2176)
    assert dc.vec_dot_type(RS) == 8 and dc.supports_mul_mat(RS, 0, 0)
    assert dc.block_sums_per_row(RS, 2048) == 64
    assert dc.mul_mat_workspace_size(RS, 5, 2048) == dc.mul_mat_workspace_size(8, 5, 2048)
    assert _mm(wt=RS, K=96) == BAD_SHAPE           # K % 256
    assert _mm(wt=RS, K=1024, wrb=1096) == MISALIGNED  # row stride % 16
    assert L.dcq_dot_rows(RS, 0x1000, 1096, 0x2000, 1024, 0x3000, 0, 4, None) == MISALIGNED
    assert L.dcq_quantize_weights(RS, 0x1000, 1, 256, 0x2000, None) == UNSUPPORTED

    def rp(wt=8, W=0x1000, N=4, K=1024, wrb=None, out=RS, Wr=0x100000, wrrb=None):
        wrb = dc.row_size(8, K) if wrb is None else wrb
        wrrb = dc.row_size(RS, K) if wrrb is None else wrrb
        return L.dcq_repack_weights(wt, W, N, K, wrb, out, Wr, wrrb, None)
    assert rp(wt=12) == UNSUPPORTED and rp(out=8) == UNSUPPORTED
    assert rp(W=None) == INVALID
    assert rp(K=96) == BAD_SHAPE and rp(N=0) == BAD_SHAPE
    assert rp(wrb=1000) == INVALID and rp(wrrb=1000) == INVALID
    assert rp(W=0x1001) == MISALIGNED and rp(Wr=0x100008) == MISALIGNED and rp(wrrb=1096) == MISALIGNED
    assert rp(Wr=0x1000 + 1088) == INVALID  # overlaps the source rows
    import torch
    if not torch.cuda.is_available():  # well-formed calls reach the device check (no pointer is used)
        assert rp() == NO_DEVICE
        assert _mm(wt=RS, K=1024) == NO_DEVICE


def test_noalloc_validation_and_limit():
    """dcq_mul_mat_noalloc validates like dcq_mul_mat, and refuses a product whose activation
    workspace exceeds the static scratch (DCQ_ERR_SCRATCH_LIMIT), all before any device call."""
    L = dc.lib()
    SCRATCH_LIMIT = -11

    def na(wt=8, W=0x1000, N=16, K=1024, M=1, X=0x2000, Y=0x3000):
        return L.dcq_mul_mat_noalloc(wt, W, N, K, dc.row_size(wt, K), X, M, K * 4, Y, N * 4, None)
    assert na(wt=3) == UNSUPPORTED
    assert na(W=None) == INVALID
    assert na(K=100) == BAD_SHAPE
    assert na(X=0x2004) == MISALIGNED
    big_m = dc.NOALLOC_SCRATCH_BYTES // 1024 + 1
    assert dc.mul_mat_workspace_size(8, big_m, 1024) > dc.NOALLOC_SCRATCH_BYTES
    assert na(M=big_m) == SCRATCH_LIMIT
    assert "scratch" in dc._lib.status_string(SCRATCH_LIMIT)
    # config 5 (M = 2048, K = 2048, Q8_0): its quantized activation fits (int8 rows + fp32 scales;
    # the workspace size adds the optional split-K room)
    assert 2048 * 2048 + 64 * 2048 * 4 <= dc.NOALLOC_SCRATCH_BYTES
    import torch
    if not torch.cuda.is_available():
        assert na(M=2048, K=2048) == NO_DEVICE


def test_well_formed_call_without_gpu_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert _mm() == NO_DEVICE
    assert dc.lib().dcq_quantize_rows(8, 0x1000, 1, 64, 256, 0x2000, None) == NO_DEVICE


def test_dot_rows_and_quantize_validation():
    L = dc.lib()
    assert L.dcq_dot_rows(3, 0x1000, 64, 0x2000, 256, 0x3000, 0, 4, None) == UNSUPPORTED
    assert L.dcq_dot_rows(12, 0x1000, 144, 0x2000, 256, 0x3000, 4, 2, None) == BAD_SHAPE
    assert L.dcq_dot_rows(12, 0x1000, 144, 0x2000, 256, 0x3000, 3, 3, None) == OK  # empty range: no work
    assert L.dcq_quantize_rows(12, 0x1000, 1, 256, 1024, 0x2000, None) == UNSUPPORTED
    assert L.dcq_quantize_rows(15, 0x1000, 1, 100, 1024, 0x2000, None) == BAD_SHAPE
    assert L.dcq_quantize_rows(15, 0x1004, 1, 256, 1024, 0x2000, None) == MISALIGNED
    assert L.dcq_quantize_weights(15, 0x1000, 1, 256, 0x2000, None) == UNSUPPORTED
    assert L.dcq_dequantize_rows(3, 0x1000, 1, 256, 64, 0x2000, None) == UNSUPPORTED


def test_ffn_gate_up_workspace_and_validation():
    """The gate/up pair: workspace = the activation's + an fp32 [M][N] buffer; argument errors
    (the second weight included) come back before any device call."""
    L = dc.lib()
    assert dc.ffn_gate_up_workspace_size(12, 64, 100, 2048) == dc.mul_mat_workspace_size(12, 64, 2048) + 25600
    assert dc.ffn_gate_up_workspace_size(12, 1, 1, 2048) == dc.mul_mat_workspace_size(12, 1, 2048) + 256
    assert dc.ffn_gate_up_workspace_size(12, 1, 16, 100) == 0
    assert dc.ffn_gate_up_workspace_size(12, 1, 0, 256) == 0

    def ffn(wt=12, Wg=0x1000, Wu=0x5000, N=16, K=256, M=1, ws=None, wsb=0):
        return L.dcq_ffn_gate_up(wt, Wg, Wu, N, K, dc.row_size(wt, K), 0x2000, M, K * 4, 0x3000, N * 4, ws, wsb,
                                 None)
    assert ffn(wt=3) == UNSUPPORTED
    assert ffn(Wg=None) == INVALID
    assert ffn(Wu=None) == INVALID
    assert ffn(Wu=0x5004) == MISALIGNED
    assert ffn(K=100) == BAD_SHAPE
    assert ffn(ws=0x4000, wsb=16) == WORKSPACE
    import torch
    if not torch.cuda.is_available():
        assert ffn() == NO_DEVICE


def test_mul_mat_add_workspace_and_validation():
    """Projection + residual/bias: R is Y itself (same stride) or disjoint from Y's extent;
    a zero R stride broadcasts a bias row. Errors come back before any device call."""
    L = dc.lib()
    assert dc.mul_mat_add_workspace_size(8, 64, 100, 1024) == dc.mul_mat_workspace_size(8, 64, 1024) + 25600
    assert dc.mul_mat_add_workspace_size(12, 1, 16, 100) == 0

    def mma(R=0x8000, rs=64, Y=0x3000, ys=64, M=2, N=16, K=256, ws=None, wsb=0):
        return L.dcq_mul_mat_add(12, 0x1000, N, K, dc.row_size(12, K), 0x2000, M, K * 4, R, rs, Y, ys, ws, wsb,
                                 None)
    assert mma(R=None) == INVALID
    assert mma(rs=32) == INVALID                 # a residual row shorter than N
    assert mma(R=0x8002) == MISALIGNED
    assert mma(rs=66) == MISALIGNED
    assert mma(R=0x3000, rs=128) == INVALID      # R is Y with another stride
    assert mma(R=0x3040 - 4, rs=64) == INVALID   # R starts inside Y
    assert mma(R=0x3000 - 64, rs=64) == INVALID  # R's second row overlaps Y's first
    assert mma(R=0x3000 - 64, rs=0) != INVALID   # one bias row just below Y
    assert mma(ws=0x4000, wsb=16) == WORKSPACE
    import torch
    if not torch.cuda.is_available():
        assert mma() == NO_DEVICE
        assert mma(R=0x3000, rs=64) == NO_DEVICE  # in place
        assert mma(rs=0) == NO_DEVICE             # bias broadcast


def test_binding_checks_tensors_before_the_abi():
    """The ctypes wrappers pass raw pointers and row strides, so a tensor of the wrong dtype, rank,
    inner stride or device is refused before any call (a transposed or fp16 X would otherwise be
    read as other bytes)."""
    import torch
    need = dc._lib._need
    with pytest.raises(ValueError, match="dtype"):
        need("x", torch.zeros((1, 256), dtype=torch.float16), torch.float32, (2,), cuda=False)
    with pytest.raises(ValueError, match="stride"):
        need("x", torch.zeros((256, 2)).t(), torch.float32, (2,), cuda=False)
    with pytest.raises(ValueError, match="dimensions"):
        need("x", torch.zeros(256), torch.float32, (2,), cuda=False)
    need("x", torch.zeros((3, 256))[:, :128], torch.float32, (2,), cuda=False)  # padded rows are fine
    if not torch.cuda.is_available():
        with pytest.raises(ValueError, match="GPU"):
            need("x", torch.zeros((1, 256)), torch.float32, (2,))
    # every compute wrapper checks before calling the ABI
    w = torch.zeros((4, 144), dtype=torch.uint8)
    for bad in (torch.zeros((1, 256), dtype=torch.float16), torch.zeros((256, 2)).t(), torch.zeros(256)):
        for fn in (lambda x: dc.mul_mat(12, w, 4, 256, x), lambda x: dc.mul_mat_ex(12, w, 4, 256, x),
                   lambda x: dc.ffn_gate_up(12, w, w, 4, 256, x), lambda x: dc.quantize_rows(15, x),
                   lambda x: dc.mul_mat_add(12, w, 4, 256, x, torch.zeros(4))):
            with pytest.raises(ValueError):
                fn(bad)
    with pytest.raises(ValueError):
        dc.quantize_weights(12, torch.zeros((4, 256), dtype=torch.float64))
    cache = dc.PagedKVCache(8, 2, 1, 1, 64, device="cpu")
    q, kc, vc = torch.zeros((1, 64)), torch.zeros((1, 64)), torch.zeros((1, 128))[:, :64]
    with pytest.raises(ValueError, match="row stride"):
        cache.attention(0, torch.zeros(2, dtype=torch.int32), q, kc, vc, 0, 0.125)
    with pytest.raises(ValueError):
        cache.write("k", 0, torch.zeros(2, dtype=torch.int64), 0, torch.zeros((1, 64)))


def test_binding_raises_on_error():
    with pytest.raises(dc.DcqError):
        dc._lib._check("dcq_mul_mat", MISALIGNED)


def test_kv_slot_bytes_and_workspace():
    assert dc.kv_slot_bytes(8, 1024) == 1088 and dc.kv_slot_bytes(1, 1024) == 2048
    assert dc.kv_slot_bytes(0, 1024) == 4096
    assert dc.kv_slot_bytes(12, 1024) == 0 and dc.kv_slot_bytes(8, 1000) == 0
    # decode at a long context splits the keys (a workspace); a large prefill does not
    assert dc.kv_attention_workspace_size(32, 8, 128, 1, 4095) > 0
    assert dc.kv_attention_workspace_size(32, 8, 128, 2048, 0) == 0
    assert dc.kv_attention_workspace_size(32, 8, 96, 1, 100) == 0  # unsupported head_dim


def test_kv_validation_before_any_device_call():
    L = dc.lib()

    def write(ct=8, arena=0x1000, n_blocks=4, n_layer=2, layer=1, row=256, table=0x2000, n_table=4, pos0=0,
              src=0x3000, stride=1024, n=3):
        return L.dcq_kv_write(ct, arena, n_blocks, n_layer, layer, row, table, n_table, pos0, src, stride, n, None)
    assert write(ct=12) == UNSUPPORTED
    assert write(arena=None) == INVALID
    assert write(layer=2) == BAD_SHAPE
    assert write(row=100) == BAD_SHAPE
    assert write(pos0=62, n=3) == INVALID   # position 64 needs a 5th table entry
    assert write(stride=512) == INVALID
    assert write(src=0x3004) == MISALIGNED
    assert write(n=0) == OK                 # nothing to write

    def attn(ct=8, hd=128, n_head=32, n_kv=8, n=1, n_past=10, q=0x1000, qs=None, ws=0x100000, wsb=1 << 30,
             scale=0.1):
        qs = qs if qs is not None else n_head * hd * 4
        return L.dcq_kv_attention(ct, 0x10000, 0x20000, 4, 1, 0, 0x2000, 4, n_head, n_kv, hd, q, qs, 0x3000,
                                  0x4000, n_kv * hd * 4, n, n_past, scale, 0x5000, n_head * hd * 4, ws, wsb, None)
    assert attn(hd=96) == UNSUPPORTED
    assert attn(ct=14) == UNSUPPORTED
    assert attn(n_kv=5) == BAD_SHAPE
    assert attn(n=0) == BAD_SHAPE
    assert attn(q=None) == INVALID
    assert attn(qs=100) == INVALID
    assert attn(q=0x1008) == MISALIGNED
    assert attn(scale=float("nan")) == INVALID
    assert attn(n_past=4095, ws=None, wsb=0) == WORKSPACE   # the split decode needs its workspace
    assert attn(ws=0x100010) == MISALIGNED
    import torch
    if not torch.cuda.is_available():
        assert attn() == NO_DEVICE
        assert write() == NO_DEVICE
