"""GGUF ingest (dcq_gguf_*) on the host: the tensor table, metadata and error paths.

There is no GGUF file or reader among the reference's files, so the parser is pinned by a file
whose every byte and offset is written out by hand here, by round trips through the test
writer (tests/gguf_writer.py), and by malformed files it must reject without reading out of
bounds: every truncated prefix of a valid file, impossible counts and lengths, unaligned or
out-of-file tensor data, unknown types.
"""
import struct

import numpy as np
import pytest

import densecore_amd as dc
from densecore_amd import synth

from gguf_writer import (T_ARR, T_BOOL, T_F32, T_F64, T_I16, T_I32, T_I64, T_I8, T_STR, T_U16, T_U32, T_U64, T_U8,
                         build_gguf, write_gguf)

FORMAT, IO, NOT_FOUND, UNSUPPORTED = -8, -9, -10, -2
F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30


def status_of(path):
    h = __import__("ctypes").c_void_p()
    rc = dc.lib().dcq_gguf_open(str(path).encode(), __import__("ctypes").byref(h))
    if rc == 0:
        dc.lib().dcq_gguf_close(h)
    return rc


def test_minimal_file_by_hand(tmp_path):
    """One F32 tensor "a" of 4 elements, no metadata: the header is 24 bytes, the tensor info
    8 + 1 + 4 + 8 + 4 + 8 = 33, so the data section starts at 64 (alignment 32)."""
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    info = struct.pack("<Q", 1) + b"a" + struct.pack("<IQIQ", 1, 4, F32, 0)
    assert len(head) == 24 and len(info) == 33
    data = np.arange(4, dtype=np.float32).tobytes()
    blob = head + info + b"\0" * (64 - 57) + data
    p = tmp_path / "min.gguf"
    p.write_bytes(blob)
    with dc.GGUF(p) as g:
        assert len(g) == 1 and g.find("a") == 0 and g.find("b") == -1
        assert g.info(0) == {"name": "a", "type": F32, "ne": [4], "file_offset": 64, "nbytes": 16}
    # the test writer produces the same bytes
    assert build_gguf([], [("a", F32, [4], data)])[0] == blob


def quant_tensor(wt, n, k, seed):
    from oracle import oracle as O
    return O.quantize_matrix(wt, synth.normal(n * k, seed, 0.0, 0.02).reshape(n, k)).tobytes()


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_round_trip_mixed_types_and_metadata(tmp_path, alignment):
    kvs = [("general.architecture", T_STR, "qwen3"), ("a.u8", T_U8, 200), ("a.i8", T_I8, -5),
           ("a.u16", T_U16, 65000), ("a.i16", T_I16, -300), ("a.u32", T_U32, 4000000000), ("a.i32", T_I32, -7),
           ("a.u64", T_U64, 1 << 40), ("a.i64", T_I64, -(1 << 40)), ("a.bool", T_BOOL, 1), ("a.f32", T_F32, 1.5),
           ("a.f64", T_F64, 2.5), ("tok.list", T_ARR, (T_STR, ["x", "yy", ""])), ("a.arr", T_ARR, (T_I32, [1, 2, 3]))]
    if alignment != 32:
        kvs.append(("general.alignment", T_U32, alignment))
    tensors = [("blk.0.ffn_gate.weight", Q4_K, [512, 3], quant_tensor(Q4_K, 3, 512, 1)),
               ("blk.0.ffn_down.weight", Q6_K, [256, 2], quant_tensor(Q6_K, 2, 256, 2)),
               ("blk.0.attn_q.weight", Q8_0, [64, 5], quant_tensor(Q8_0, 5, 64, 3)),
               ("output_norm.weight", F32, [7], np.arange(7, dtype=np.float32).tobytes()),
               ("x.bf16", BF16, [16, 2], bytes(range(64)))]
    p = tmp_path / "mix.gguf"
    start, offsets = write_gguf(p, kvs, tensors, alignment)
    raw = p.read_bytes()
    with dc.GGUF(p) as g:
        assert len(g) == len(tensors)
        for i, ((name, t, ne, data), off) in enumerate(zip(tensors, offsets)):
            assert g.find(name) == i
            info = g.info(i)
            assert info == {"name": name, "type": t, "ne": ne, "file_offset": start + off, "nbytes": len(data)}
            assert info["file_offset"] % alignment == 0
            assert raw[info["file_offset"]:info["file_offset"] + info["nbytes"]] == data
        assert g.get_str("general.architecture") == "qwen3"
        for key, want in [("a.u8", 200), ("a.i8", -5), ("a.u16", 65000), ("a.i16", -300), ("a.u32", 4000000000),
                          ("a.i32", -7), ("a.u64", 1 << 40), ("a.i64", -(1 << 40)), ("a.bool", 1)]:
            assert g.get_int(key) == want, key
        with pytest.raises(dc.DcqError) as e:
            g.get_int("missing.key")
        assert e.value.status == NOT_FOUND
        for key in ("a.f32", "general.architecture", "a.arr"):
            with pytest.raises(dc.DcqError) as e:
                g.get_int(key)
            assert e.value.status == FORMAT
        with pytest.raises(dc.DcqError):
            g.get_str("a.u8")


def valid_blob():
    return build_gguf([("general.architecture", T_STR, "llama"), ("n", T_U32, 3)],
                      [("w", Q4_K, [256, 2], quant_tensor(Q4_K, 2, 256, 9)), ("b", F32, [3], bytes(12))])[0]


def test_every_truncated_prefix_is_rejected(tmp_path):
    blob = valid_blob()
    p = tmp_path / "t.gguf"
    p.write_bytes(blob)
    assert status_of(p) == 0
    for n in range(len(blob)):
        p.write_bytes(blob[:n])
        assert status_of(p) in (FORMAT, IO), n


def test_malformed_headers_and_tables(tmp_path):
    p = tmp_path / "bad.gguf"

    def rc(blob):
        p.write_bytes(blob)
        return status_of(p)
    good = valid_blob()
    assert rc(b"GGUX" + good[4:]) == FORMAT                                  # magic
    assert rc(good[:4] + struct.pack("<I", 1) + good[8:]) == FORMAT           # version 1
    assert rc(good[:4] + struct.pack("<I", 4) + good[8:]) == FORMAT           # version 4
    assert rc(good[:8] + struct.pack("<Q", 1 << 60) + good[16:]) == FORMAT    # tensor count
    assert rc(good[:16] + struct.pack("<Q", 1 << 60) + good[24:]) == FORMAT   # kv count
    # a string length past the end of the file
    assert rc(good[:24] + struct.pack("<Q", 1 << 50) + good[32:]) == FORMAT
    data = bytes(16)
    assert rc(build_gguf([], [("a", 99, [4], data)])[0]) == UNSUPPORTED        # unknown type
    assert rc(build_gguf([], [("a", Q8_0, [40], bytes(68))])[0]) == FORMAT     # ne[0] % 32
    assert rc(build_gguf([], [("a", F32, [], data)])[0]) == FORMAT             # n_dims 0
    assert rc(build_gguf([], [("a", F32, [1, 1, 1, 1, 4], data)])[0]) == FORMAT  # n_dims 5
    assert rc(build_gguf([], [("a", F32, [0], b"")])[0]) == FORMAT             # empty dim
    assert rc(build_gguf([], [("a", F32, [4], data), ("a", F32, [4], data)])[0]) == FORMAT  # duplicate
    assert rc(build_gguf([], [("a", F32, [4], data)], offsets=[4])[0]) == FORMAT       # unaligned
    blob, start, _ = build_gguf([], [("a", F32, [4], data)])
    assert rc(blob[:-1]) == FORMAT                                             # data past the end
    assert rc(build_gguf([("general.alignment", T_U32, 48)], [("a", F32, [4], data)])[0]) == FORMAT
    assert rc(build_gguf([("general.alignment", T_STR, "32")], [("a", F32, [4], data)])[0]) == FORMAT
    unknown_kv = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13) + bytes(8)
    assert rc(unknown_kv) == FORMAT                                            # unknown value type
    assert rc(build_gguf([("k", T_ARR, (T_STR, ["a"]))], [])[0]) == 0
    # a metadata key given twice
    assert rc(build_gguf([("k", T_U32, 1), ("k", T_U32, 2)], [("a", F32, [4], data)])[0]) == FORMAT
    assert rc(build_gguf([("k", T_U32, 1), ("k2", T_U32, 2)], [("a", F32, [4], data)])[0]) == 0
    assert status_of(tmp_path / "does_not_exist.gguf") == IO
    assert status_of(tmp_path) == IO                                           # a directory: no mapping


def test_load_needs_room_and_an_index(tmp_path):
    p = tmp_path / "v.gguf"
    p.write_bytes(valid_blob())
    with dc.GGUF(p) as g:
        L = dc.lib()
        assert L.dcq_gguf_load_tensor(g._h, 5, 0x1000, 1 << 20, None) == -1
        assert L.dcq_gguf_load_tensor(g._h, 0, 0x1000, 10, None) == -1
        assert L.dcq_gguf_load_tensor(g._h, 0, None, 1 << 20, None) == -1
        assert L.dcq_gguf_tensor_info(g._h, -1, None, None, None, None, None, None) == -1
