"""GPU parity of the paged KV cache and its attention (dcq_kv_*), through the C ABI, against the
CPU oracle (oracle/kv.py). Slot bytes and the gather are bit-exact; the attention output is
within |out - ref| <= A * (1e-4 + 1e-5 * B), A = sum_t p_t |v_t|, B = max_t scale sum |q k_t|."""
import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, F16, F32 = 8, 1, 0
CACHE_TYPES = [Q8_0, F16, F32]


@pytest.fixture(scope="module")
def KV(O):
    from oracle import kv
    return kv


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_table(n_pos, n_blocks, seed, holes=()):
    rng = np.random.default_rng(seed)
    need = (n_pos + 15) // 16
    table = rng.permutation(n_blocks)[:need].astype(np.int32)
    for h in holes:
        table[h] = -1
    return table


@pytest.mark.parametrize("ct", CACHE_TYPES)
def test_kv_write_bytes(KV, dev, ct):
    """Rows written at positions pos0 .. into a pre-filled arena: every byte equals the
    oracle's (including the slots left alone, and a table entry of -1 that is skipped)."""
    import torch
    n_layer, layer, row, n_blocks = 3, 1, 4 * 64, 9
    sb = KV.slot_bytes(ct, row)
    rng = np.random.default_rng(3)
    arena = rng.integers(0, 256, n_blocks * n_layer * 16 * sb, dtype=np.uint8)
    table = make_table(70, n_blocks, 4, holes=(2,))
    rows = synth.normal(45 * row, 5).reshape(45, row)
    synth.set_outliers(rows.reshape(-1), 30, 25.0, 6)
    rows[3, :64] = 0.0  # an all-zero Q8_0 block
    want = arena.copy()
    KV.write(ct, want, n_layer, layer, table, 25, rows)
    cache = dc.PagedKVCache(ct, n_blocks, n_layer, 4, 64, device=dev)
    cache.k.copy_(to_dev(arena, dev))
    cache.write("k", layer, to_dev(table, dev), 25, to_dev(rows, dev))
    assert np.array_equal(to_host(cache.k), want)
    assert not to_host(cache.v).any()
    del torch


@pytest.mark.parametrize("ct", CACHE_TYPES)
def test_kv_gather_exact(KV, dev, ct):
    """History decoded bit-exactly, missing blocks (short table, -1 entry) as zeros, the current
    rows appended as given."""
    n_layer, layer, row, n_blocks, n_past = 2, 0, 2 * 128, 8, 75
    sb = KV.slot_bytes(ct, row)
    arena = np.zeros(n_blocks * n_layer * 16 * sb, np.uint8)
    table = make_table(64, n_blocks, 8, holes=(1,))  # covers 4 of the 5 history blocks
    hist = synth.normal(n_past * row, 9).reshape(n_past, row)
    KV.write(ct, arena, n_layer, layer, table, 0, hist[:64])
    cur = synth.normal(3 * row, 10).reshape(3, row)
    want = KV.gather(ct, arena, n_layer, layer, table, n_past, cur)
    cache = dc.PagedKVCache(ct, n_blocks, n_layer, 2, 128, device=dev)
    cache.v.copy_(to_dev(arena, dev))
    got = cache.gather("v", layer, to_dev(table, dev), n_past, to_dev(cur, dev))
    assert np.array_equal(to_host(got).view(np.uint32), want.view(np.uint32))


ATTN = [
    # (cache type, n_tokens, n_past, n_head, n_head_kv, head_dim)
    (Q8_0, 1, 4095, 32, 8, 128),   # Qwen3-4B decode at a 4k context: keys split over workgroups
    (Q8_0, 1, 5, 32, 8, 128),      # a short history
    (Q8_0, 1, 0, 32, 8, 128),      # the first token: only its own row
    (Q8_0, 7, 100, 32, 8, 128),    # a chunk of prefill on top of history
    (Q8_0, 130, 0, 8, 8, 64),      # prefill, MHA, current rows over several chunks
    (Q8_0, 3, 300, 8, 1, 256),     # head_dim 256, multi-query (8 heads per KV head)
    (Q8_0, 2, 77, 32, 1, 128),     # 32 query heads per KV head: the group split over workgroups
    (Q8_0, 2, 50, 8, 4, 128),      # the 4-row workgroup with two tokens of two heads each
    (F16, 4, 20, 4, 4, 64),        # the 4-row workgroup with four tokens of one head
    (F16, 1, 4095, 32, 8, 128),
    # the split merge's forms: 17..64 splits, 97..128 (32 lanes per output), over 128 (a workgroup
    # per row)
    (Q8_0, 1, 2000, 32, 8, 128),   # 33 splits
    (Q8_0, 1, 7000, 32, 8, 128),   # 111 splits
    (F16, 1, 20000, 4, 4, 64),     # 158 splits
    (F16, 5, 33, 16, 4, 64),
    (F32, 1, 200, 8, 2, 128),
    (F32, 17, 40, 4, 2, 256),
    # prompts on the MFMA kernel (>= 64 tokens, query-head groups of 4k): two exact 32-token
    # tiles; a ragged last tile over a history that is not a multiple of 32 keys; head_dim 64
    # with 8 query heads per KV head; one KV head; a Qwen3-4B-sized prompt chunk
    (Q8_0, 64, 0, 32, 8, 128),
    (Q8_0, 100, 37, 8, 2, 128),
    (F16, 96, 50, 16, 2, 64),
    (F32, 70, 20, 4, 1, 128),
    (Q8_0, 256, 300, 32, 8, 128),
    # the MFMA kernel with its keys split over workgroups (few tokens over a long history)
    (Q8_0, 32, 700, 8, 2, 128),
    (F16, 40, 1000, 16, 4, 64),
]


@pytest.mark.parametrize("ct,n,n_past,n_head,n_kv,hd", ATTN)
def test_kv_attention(KV, dev, ct, n, n_past, n_head, n_kv, hd):
    n_layer, layer = 2, 1
    row = n_kv * hd
    n_blocks = (n_past + 15) // 16 + 3
    sb = KV.slot_bytes(ct, row)
    arena_k = np.zeros(n_blocks * n_layer * 16 * sb, np.uint8)
    arena_v = np.zeros_like(arena_k)
    table = make_table(max(n_past, 1), n_blocks, 11 + n)
    seed = 100 + n + n_past + hd
    hist_k = synth.normal(n_past * row, seed).reshape(n_past, row)
    hist_v = synth.normal(n_past * row, seed + 1).reshape(n_past, row)
    KV.write(ct, arena_k, n_layer, layer, table, 0, hist_k)
    KV.write(ct, arena_v, n_layer, layer, table, 0, hist_v)
    q = synth.normal(n * n_head * hd, seed + 2, 0.0, 2.0).reshape(n, n_head * hd)
    k_cur = synth.normal(n * row, seed + 3).reshape(n, row)
    v_cur = synth.normal(n * row, seed + 4).reshape(n, row)
    scale = 1.0 / np.sqrt(hd)
    k_all = KV.gather(ct, arena_k, n_layer, layer, table, n_past, k_cur).reshape(-1, n_kv, hd)
    v_all = KV.gather(ct, arena_v, n_layer, layer, table, n_past, v_cur).reshape(-1, n_kv, hd)
    ref, parts = KV.attention(q.reshape(n, n_head, hd), k_all, v_all, n_past, np.float32(scale))

    cache = dc.PagedKVCache(ct, n_blocks, n_layer, n_kv, hd, device=dev)
    cache.k.copy_(to_dev(arena_k, dev))
    cache.v.copy_(to_dev(arena_v, dev))
    out = cache.attention(layer, to_dev(table, dev), to_dev(q, dev), to_dev(k_cur, dev), to_dev(v_cur, dev),
                          n_past, float(np.float32(scale)))
    KV.assert_close_attention(to_host(out).reshape(n, n_head, hd), ref, parts,
                              what=f"attention ct={ct} n={n} n_past={n_past} heads={n_head}/{n_kv} hd={hd}")


@pytest.mark.parametrize("n", [2, 80])  # the VALU kernel with key splits; the MFMA prompt kernel
def test_kv_attention_missing_blocks_read_as_zero_keys(KV, dev, n):
    """A history block absent from the table (-1, or past the table's end) is a zero K/V row,
    as in the reference's gathered K_all: score 0, value 0."""
    ct, n_past, n_head, n_kv, hd, n_layer = Q8_0, 90, 8, 2, 128, 1
    row = n_kv * hd
    n_blocks = 8
    sb = KV.slot_bytes(ct, row)
    arena_k = np.zeros(n_blocks * n_layer * 16 * sb, np.uint8)
    arena_v = np.zeros_like(arena_k)
    table = make_table(64, n_blocks, 12, holes=(2,))  # 4 entries for 6 history blocks
    KV.write(ct, arena_k, n_layer, 0, table, 0, synth.normal(64 * row, 13).reshape(64, row))
    KV.write(ct, arena_v, n_layer, 0, table, 0, synth.normal(64 * row, 14).reshape(64, row))
    q = synth.normal(n * n_head * hd, 15).reshape(n, n_head * hd)
    k_cur = synth.normal(n * row, 16).reshape(n, row)
    v_cur = synth.normal(n * row, 17).reshape(n, row)
    k_all = KV.gather(ct, arena_k, n_layer, 0, table, n_past, k_cur).reshape(-1, n_kv, hd)
    v_all = KV.gather(ct, arena_v, n_layer, 0, table, n_past, v_cur).reshape(-1, n_kv, hd)
    ref, parts = KV.attention(q.reshape(n, n_head, hd), k_all, v_all, n_past, 0.125)
    cache = dc.PagedKVCache(ct, n_blocks, n_layer, n_kv, hd, device=dev)
    cache.k.copy_(to_dev(arena_k, dev))
    cache.v.copy_(to_dev(arena_v, dev))
    out = cache.attention(0, to_dev(table, dev), to_dev(q, dev), to_dev(k_cur, dev), to_dev(v_cur, dev), n_past,
                          0.125)
    KV.assert_close_attention(to_host(out).reshape(n, n_head, hd), ref, parts, what="missing blocks")


def test_kv_decode_steps_write_then_attend(KV, dev):
    """Decode loop: each step attends with its own row in fp32, then writes that row into the
    cache for the next step (the reference's write-then-gather order within one call gives the
    same attention input). Eight steps against the oracle doing the same."""
    ct, n_head, n_kv, hd, n_layer, layer = Q8_0, 16, 4, 128, 2, 0
    row = n_kv * hd
    n_blocks = 6
    sb = KV.slot_bytes(ct, row)
    arena_k = np.zeros(n_blocks * n_layer * 16 * sb, np.uint8)
    arena_v = np.zeros_like(arena_k)
    table = make_table(80, n_blocks, 20)
    n_past0 = 60
    KV.write(ct, arena_k, n_layer, layer, table, 0, synth.normal(n_past0 * row, 21).reshape(n_past0, row))
    KV.write(ct, arena_v, n_layer, layer, table, 0, synth.normal(n_past0 * row, 22).reshape(n_past0, row))
    cache = dc.PagedKVCache(ct, n_blocks, n_layer, n_kv, hd, device=dev)
    cache.k.copy_(to_dev(arena_k, dev))
    cache.v.copy_(to_dev(arena_v, dev))
    tdev = to_dev(table, dev)
    for step in range(8):
        n_past = n_past0 + step
        q = synth.normal(n_head * hd, 30 + step).reshape(1, -1)
        kc = synth.normal(row, 40 + step).reshape(1, -1)
        vc = synth.normal(row, 50 + step).reshape(1, -1)
        k_all = KV.gather(ct, arena_k, n_layer, layer, table, n_past, kc).reshape(-1, n_kv, hd)
        v_all = KV.gather(ct, arena_v, n_layer, layer, table, n_past, vc).reshape(-1, n_kv, hd)
        ref, parts = KV.attention(q.reshape(1, n_head, hd), k_all, v_all, n_past, 0.08838834764831845)
        kd, vd = to_dev(kc, dev), to_dev(vc, dev)
        out = cache.attention(layer, tdev, to_dev(q, dev), kd, vd, n_past, 0.08838834764831845)
        cache.write("k", layer, tdev, n_past, kd)
        cache.write("v", layer, tdev, n_past, vd)
        KV.write(ct, arena_k, n_layer, layer, table, n_past, kc)
        KV.write(ct, arena_v, n_layer, layer, table, n_past, vc)
        KV.assert_close_attention(to_host(out).reshape(1, n_head, hd), ref, parts, what=f"decode step {step}")
    assert np.array_equal(to_host(cache.k), arena_k) and np.array_equal(to_host(cache.v), arena_v)
