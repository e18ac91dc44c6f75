"""Pins of the paged KV-cache oracle (oracle/kv.py): slot bytes and layout, the Q8_0 / F16 slot
encodings, the gather, and the attention against an independent library routine and closed
forms. CPU only."""
import numpy as np
import pytest

from densecore_amd import synth

Q8_0, F16, F32 = 8, 1, 0


@pytest.fixture(scope="module")
def KV(O):
    from oracle import kv
    return kv


# ---------------------------------------------------------------- slots
def test_slot_bytes(KV):
    """GetBytesPerSlot: head_dim * n_head_kv * type_size / block_size."""
    assert KV.slot_bytes(Q8_0, 8 * 128) == 8 * 128 // 32 * 34
    assert KV.slot_bytes(F16, 8 * 128) == 8 * 128 * 2
    assert KV.slot_bytes(F32, 4 * 64) == 4 * 64 * 4


def test_slot_layout_is_block_major_then_layer_then_slot(KV):
    """The arena viewed as [n_blocks][n_layer][16][slot_bytes] (a numpy reshape, independent of
    slot_offset) holds each written row at [block][layer][pos % 16]."""
    n_blocks, n_layer, row = 5, 3, 64
    sb = KV.slot_bytes(F32, row)
    arena = np.zeros(n_blocks * n_layer * 16 * sb, np.uint8)
    table = np.array([4, 0, 2], np.int32)
    rows = synth.normal(40 * row, 1).reshape(40, row)
    KV.write(F32, arena, n_layer, 2, table, 3, rows)
    view = arena.reshape(n_blocks, n_layer, 16, sb)
    for i in range(40):
        pos = 3 + i
        got = view[table[pos // 16], 2, pos % 16].view(np.float32)
        assert np.array_equal(got, rows[i])
    assert not view[:, :2].any() and not view[[1, 3]].any()


def test_write_skips_out_of_range_blocks(KV):
    arena = np.zeros(2 * 1 * 16 * KV.slot_bytes(F32, 32), np.uint8)
    KV.write(F32, arena, 1, 0, np.array([-1, 7], np.int32), 0, np.ones((32, 32), np.float32))
    assert not arena.any()


def test_q8_0_slot_is_the_ref_quantizer(KV, O):
    """Q8_0 slots use quantize_row_q8_0_ref: identical to the oracle's REF activation variant
    (whose ties and closed forms are pinned in test_oracle.py), and to an IEEE float32
    step-by-step recomputation in numpy: d = amax / 127, id = 1 / d, q = round half away."""
    x = synth.normal(32 * 64, 3)
    synth.set_outliers(x, 11, 30.0, 4)
    x[64:96] = 0.0
    got = KV.encode_row(Q8_0, x)
    assert np.array_equal(got, O.quantize_rows(Q8_0, x, O.Q8_0_REF)[0])
    blk = got.reshape(-1, 34)
    xb = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (xb * inv[:, None]).astype(np.float32)
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    assert np.array_equal(blk[:, :2].copy().view(np.float16)[:, 0], d.astype(np.float16))
    assert np.array_equal(blk[:, 2:].view(np.int8), q)


def test_f16_slot_is_ieee_rne(KV):
    x = synth.normal(4096, 5) * 1000
    x[:4] = [65504.0, 65520.0, 1e-8, -2.0 ** -25]
    got = KV.encode_row(F16, x).view(np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
    assert np.array_equal(KV.decode_row(F16, got.view(np.uint8), x.size), x.astype(np.float16).astype(np.float32))


def test_gather_history_then_current(KV):
    """History rows decode what was written; a position whose block is missing from the table
    (or out of range) reads zeros; the current rows are appended unquantized."""
    n_layer, row = 2, 64
    sb = KV.slot_bytes(Q8_0, row)
    arena = np.zeros(4 * n_layer * 16 * sb, np.uint8)
    table = np.array([3, 1, -1], np.int32)
    hist = synth.normal(40 * row, 6).reshape(40, row)
    KV.write(Q8_0, arena, n_layer, 1, table, 0, hist[:32])
    cur = synth.normal(3 * row, 7).reshape(3, row)
    g = KV.gather(Q8_0, arena, n_layer, 1, table, 40, cur)
    for t in range(32):
        assert np.array_equal(g[t], KV.decode_row(Q8_0, KV.encode_row(Q8_0, hist[t]), row))
    assert not g[32:40].any()
    assert np.array_equal(g[40:], cur)


# ---------------------------------------------------------------- attention
def _case(n, n_past, n_head, n_kv, hd, seed):
    q = synth.normal(n * n_head * hd, seed).reshape(n, n_head, hd)
    k = synth.normal((n_past + n) * n_kv * hd, seed + 1).reshape(n_past + n, n_kv, hd)
    v = synth.normal((n_past + n) * n_kv * hd, seed + 2).reshape(n_past + n, n_kv, hd)
    return q, k, v


@pytest.mark.parametrize("n,n_past,n_head,n_kv,hd", [(1, 37, 8, 2, 64), (5, 20, 4, 4, 32), (9, 0, 6, 3, 16),
                                                     (3, 100, 16, 1, 8)])
def test_attention_matches_torch_sdpa(KV, n, n_past, n_head, n_kv, hd):
    """torch's scaled_dot_product_attention in float64 on the CPU, with each KV head repeated
    for its query-head group and a boolean causal mask offset by n_past."""
    import torch
    import torch.nn.functional as F
    q, k, v = _case(n, n_past, n_head, n_kv, hd, 40 + n)
    scale = 1.0 / np.sqrt(hd)
    got, _ = KV.attention(q, k, v, n_past, scale)
    rep = n_head // n_kv
    qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(rep, dim=0)
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(rep, dim=0)
    mask = torch.arange(n_past + n)[None, :] <= (n_past + torch.arange(n))[:, None]
    want = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale).permute(1, 0, 2).numpy()
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_attention_closed_forms(KV):
    """The first query with n_past = 0 sees one key: its value row, whatever q and k are.
    Equal keys give equal scores: the mean of the visible value rows."""
    q, k, v = _case(4, 0, 4, 2, 16, 50)
    out, _ = KV.attention(q, k, v, 0, 0.25)
    rep = 2
    for h in range(4):
        assert np.allclose(out[0, h], v[0, h // rep], rtol=0, atol=1e-12)
    k[:] = k[0]
    out, _ = KV.attention(q, k, v, 0, 0.25)
    for i in range(4):
        for h in range(4):
            assert np.allclose(out[i, h], v[:i + 1, h // rep].astype(np.float64).mean(axis=0), atol=1e-12)


def test_attention_tolerance_catches_planted_mistakes(KV):
    """Each plausible mistake, planted in a copy of the computation, moves the output outside
    the fp32 tolerance; the float32 evaluation of the correct formula stays inside it."""
    n, n_past, n_head, n_kv, hd = 3, 50, 8, 2, 64
    q, k, v = _case(n, n_past, n_head, n_kv, hd, 60)
    scale = 1.0 / np.sqrt(hd)
    ref, parts = KV.attention(q, k, v, n_past, scale)

    def f32(q_, k_, v_, n_past_, scale_, mask_shift=0, group=lambda h, rep: h // rep):
        rep = n_head // n_kv
        out = np.zeros((n, n_head, hd), np.float32)
        for i in range(n):
            for h in range(n_head):
                g = group(h, rep)
                t_vis = n_past_ + i + 1 + mask_shift
                s = (k_[:t_vis, g].astype(np.float32) @ q_[i, h].astype(np.float32)) * np.float32(scale_)
                p = np.exp(s - s.max())
                out[i, h] = (p / p.sum()) @ v_[:t_vis, g].astype(np.float32)
        return out

    KV.assert_close_attention(f32(q, k, v, n_past, scale), ref, parts, what="float32 evaluation")
    planted = {
        "mask off by one (sees the next key)": f32(q, k, v, n_past, scale, mask_shift=1)[:2],
        "mask off by one (misses its own key)": f32(q, k, v, n_past, scale, mask_shift=-1),
        "K and V swapped": f32(q, v, k, n_past, scale),
        "scale dropped": f32(q, k, v, n_past, 1.0),
        "heads grouped by modulo": f32(q, k, v, n_past, scale, group=lambda h, rep: h % n_kv),
    }
    for what, bad in planted.items():
        r = ref[:bad.shape[0]]
        pa = tuple(x[:bad.shape[0]] for x in parts)
        with pytest.raises(AssertionError):
            KV.assert_close_attention(bad, r, pa, what=what)


def test_quantized_current_rows_fall_outside_the_tolerance(KV):
    """The batch's own K/V rows enter unquantized (inference.cpp:778-784); reading them back
    from a Q8_0 cache instead is a visible difference."""
    n, n_past, n_head, n_kv, hd = 4, 0, 4, 2, 64
    q, k, v = _case(n, n_past, n_head, n_kv, hd, 70)
    ref, parts = KV.attention(q, k, v, n_past, 1.0 / 8)
    kq = np.stack([KV.decode_row(Q8_0, KV.encode_row(Q8_0, r.ravel()), r.size).reshape(r.shape) for r in k])
    vq = np.stack([KV.decode_row(Q8_0, KV.encode_row(Q8_0, r.ravel()), r.size).reshape(r.shape) for r in v])
    bad, _ = KV.attention(q, kq, vq, n_past, 1.0 / 8)
    with pytest.raises(AssertionError):
        KV.assert_close_attention(bad, ref, parts)
