"""CPU restatement of DenseCore's paged KV cache (F32 / F16 / Q8_0 slots) and of the attention
that reads it, in numpy.

TEST INFRASTRUCTURE ONLY: imported by tests/ and by bench.py's cpu_baseline leg as the checker.
The product library never imports it.

What it restates (reference file:line):
  - slot bytes: row_size(cache_type, head_dim * n_head_kv)            core/src/kv_cache.cpp:341-351
  - slot address: arena + ((block_id * n_layer + layer) * 16 + slot)
    * slot_bytes, 16 slots (tokens) per block                         core/src/kv_cache.cpp:353-409,
                                                                      core/include/kv_cache.h:17
  - write: F32 copy, F16 round-to-nearest-even, Q8_0 with
    ggml_quantize_chunk (quantize_row_q8_0_ref: d = amax / 127,
    id = 1 / d, q = roundf(x * id), d stored as fp16)                 core/src/kv_cache.cpp:565-598
  - read: F16 -> F32, Q8_0 -> d * q                                   core/src/kv_cache.cpp:600-629
  - gather: history [0, n_past) read from the cache (zeros where the
    block table has no block), then the batch's own rows appended
    in fp32, unquantized                                              core/src/inference.cpp:667-784
  - attention over the gathered K/V, grouped-query heads h -> h / n_rep:
    KQ = K_head . Q, * scale, causal mask (key t visible to query i
    iff t <= n_past + i), softmax over keys, V . softmax             core/src/inference.cpp:1577-1746

Parity pins (tests/test_oracle.py):
  - q8_0_ref_row: closed forms (zero block, integer-valued blocks, ties rounding away from zero,
    |x - d q| <= d/2, max |q| = 127) and an IEEE float32 step-by-step recomputation;
  - F16 slots: numpy float16 (IEEE RNE);
  - attention: torch.nn.functional.scaled_dot_product_attention in float64 on the CPU with the
    K/V heads repeated per group, and closed forms (one visible key returns its value row;
    equal keys return the mean of the visible value rows); planted mistakes (mask off by one,
    K/V swapped, scale dropped, head grouping by modulo, quantized current rows) must fail the
    tolerance.
"""
import numpy as np

from . import oracle as O

KV_BLOCK = 16
CACHE_TYPES = (O.TYPE_F32, O.TYPE_F16, O.TYPE_Q8_0)


def slot_bytes(ct, row_elems):
    """core/src/kv_cache.cpp:341-347."""
    assert ct in CACHE_TYPES, ct
    rs = O.row_size(ct, row_elems)
    assert rs > 0, (ct, row_elems)
    return rs


def slot_offset(block_id, layer, n_layer, slot, sb):
    """core/src/kv_cache.cpp:353-409: [row, BLOCK_SIZE, num_blocks * n_layer] with block index
    block_id * n_layer + layer."""
    return ((block_id * n_layer + layer) * KV_BLOCK + slot) * sb


def q8_0_ref_row(x):
    """quantize_row_q8_0_ref (the quantizer ggml_quantize_chunk uses for Q8_0; called for KV
    slots at core/src/kv_cache.cpp:578, 594). Same bytes as O.quantize_matrix(TYPE_Q8_0)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(1, -1)
    return O.quantize_matrix(O.TYPE_Q8_0, x)[0]


def encode_row(ct, x):
    """WriteKSlot / WriteVSlot (core/src/kv_cache.cpp:565-598): one token row to slot bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if ct == O.TYPE_F32:
        return x.view(np.uint8).copy()
    if ct == O.TYPE_F16:
        return O.fp32_to_fp16(x).view(np.uint8).copy()
    return q8_0_ref_row(x)


def decode_row(ct, b, n):
    """ReadKSlot / ReadVSlot (core/src/kv_cache.cpp:600-629): slot bytes to fp32."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    if ct == O.TYPE_F32:
        return b.view(np.float32)[:n].copy()
    if ct == O.TYPE_F16:
        return O.fp16_to_fp32(b.view(np.uint16)[:n])
    return O.dequantize_row(O.TYPE_Q8_0, b, n)


def write(ct, arena, n_layer, layer, table, pos0, rows):
    """Write rows [N, row_elems] for positions pos0 .. pos0 + N - 1 of one sequence into arena
    (uint8, modified in place). A block id outside [0, n_blocks) is skipped, as the reference's
    null slot pointer is (core/src/kv_cache.cpp:566-568)."""
    rows = np.asarray(rows, dtype=np.float32)
    n_tok, row_elems = rows.shape
    sb = slot_bytes(ct, row_elems)
    n_blocks = arena.size // (sb * KV_BLOCK * n_layer)
    for i in range(n_tok):
        pos = pos0 + i
        blk = int(table[pos // KV_BLOCK])
        if not 0 <= blk < n_blocks:
            continue
        off = slot_offset(blk, layer, n_layer, pos % KV_BLOCK, sb)
        arena[off:off + sb] = encode_row(ct, rows[i])


def gather(ct, arena, n_layer, layer, table, n_past, cur):
    """cb_kv_update_and_gather's output (core/src/inference.cpp:748-784): [n_past + N, row]
    fp32, history read from the cache and the current rows appended as given."""
    cur = np.asarray(cur, dtype=np.float32)
    row_elems = cur.shape[1]
    sb = slot_bytes(ct, row_elems)
    n_blocks = arena.size // (sb * KV_BLOCK * n_layer)
    out = np.zeros((n_past + cur.shape[0], row_elems), dtype=np.float32)
    for t in range(n_past):
        lb = t // KV_BLOCK
        blk = int(table[lb]) if lb < len(table) else -1
        if 0 <= blk < n_blocks:
            off = slot_offset(blk, layer, n_layer, t % KV_BLOCK, sb)
            out[t] = decode_row(ct, arena[off:off + sb], row_elems)
    out[n_past:] = cur
    return out


def attention(q, k_all, v_all, n_past, scale):
    """The standard-path attention of core/src/inference.cpp:1577-1746 in float64.

    q [N, n_head, hd], k_all / v_all [T, n_head_kv, hd] with T = n_past + N. Returns
    (out [N, n_head, hd], (A, B)) where A[i, h, d] = sum_t p_t |v_t[d]| and
    B[i, h] = max over visible t of scale * sum_d |q_d k_t[d]|, the quantities the fp32 error
    of the device result is bounded by (assert_close_attention)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k_all, dtype=np.float64)
    v = np.asarray(v_all, dtype=np.float64)
    n, n_head, hd = q.shape
    t_all, n_kv, _ = k.shape
    assert t_all == n_past + n and n_head % n_kv == 0
    rep = n_head // n_kv
    kh = np.repeat(k, rep, axis=1)          # [T, n_head, hd]: head h reads KV head h // rep
    vh = np.repeat(v, rep, axis=1)
    s = np.einsum("ihd,thd->iht", q, kh) * scale
    sa = np.einsum("ihd,thd->iht", np.abs(q), np.abs(kh)) * scale
    visible = np.arange(t_all)[None, :] <= (n_past + np.arange(n))[:, None]   # [N, T]
    s = np.where(visible[:, None, :], s, -np.inf)
    p = np.exp(s - s.max(axis=2, keepdims=True))
    p /= p.sum(axis=2, keepdims=True)
    out = np.einsum("iht,thd->ihd", p, vh)
    a = np.einsum("iht,thd->ihd", p, np.abs(vh))
    b = np.where(visible[:, None, :], sa, 0.0).max(axis=2)
    return out, (a, b)


def assert_close_attention(out, ref, parts, rtol=1e-4, what=""):
    """fp32 tolerance of the attention output.

    A score carries the fp32 dot error, at most about hd * 2^-24 * B; the softmax weight p_t
    moves by the same relative amount, so the output moves by at most that times
    A = sum_t p_t |v_t|, plus the fp32 rounding of the weighted sum itself (relative to A).
    Bound: |out - ref| <= A * (rtol + 1e-5 * B)."""
    a, b = (np.asarray(x, dtype=np.float64) for x in parts)
    out = np.asarray(out, dtype=np.float64).reshape(ref.shape)
    bound = a * (rtol + 1e-5 * b[:, :, None]) + 1e-30
    err = np.abs(out - ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} outside the bound; worst at {i}: "
                             f"got {out[i]} want {ref[i]} bound {bound[i]}")
    return float(np.max(err / bound))
