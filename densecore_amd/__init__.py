"""densecore_amd — MI355X (gfx950) backend for DenseCore's quantized mul_mat.

The product is the C ABI in include/dcq.h, implemented by densecore_amd/libdcq.so
(HIP kernels for gfx950). This package is a thin ctypes binding of that ABI
plus helpers that pass torch device tensors (torch is only used for device
memory and streams). There is no CPU fallback: every compute entry point calls
the HIP library, and importing the binding fails loudly when libdcq.so is
missing.
"""
from .configs import (CONFIGS, TYPE_F16, TYPE_F32, TYPE_NAMES, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q5_K,  # noqa: F401
                      TYPE_Q6_K, TYPE_Q8_0, TYPE_Q8_0_RS, TYPE_Q8_K, Config, by_index)
from ._lib import (GGUF, KV_BLOCK_SIZE, PagedKVCache, kv_attention_workspace_size, kv_slot_bytes,  # noqa: F401
                   DcqError, LIB_PATH, block_size, block_sums_per_row, build, dequantize_rows,  # noqa: F401
                   dot_rows, ffn_gate_up, ffn_gate_up_workspace_size, lib, mul_mat, mul_mat_add,
                   mul_mat_add_workspace_size, mul_mat_ex, mul_mat_noalloc, NOALLOC_SCRATCH_BYTES, probe_stream_read,
                   mul_mat_workspace_size, PATH_AUTO, PATH_GEMV, PATH_MMQ,
                   quantize_rows, quantize_src1, mul_mat_q, quantize_weights, repack_weights, row_size,
                   supports_mul_mat, type_size, vec_dot_type, version)

__all__ = [
    "CONFIGS", "Config", "by_index", "GGUF", "DcqError", "LIB_PATH", "lib", "build", "version", "block_size", "type_size",
    "row_size", "vec_dot_type", "supports_mul_mat", "block_sums_per_row", "mul_mat_workspace_size",
    "quantize_rows", "quantize_src1", "mul_mat_q", "mul_mat", "mul_mat_ex", "mul_mat_noalloc",
    "NOALLOC_SCRATCH_BYTES", "probe_stream_read", "mul_mat_add",
    "mul_mat_add_workspace_size", "dot_rows", "ffn_gate_up",
    "ffn_gate_up_workspace_size", "quantize_weights", "repack_weights", "dequantize_rows", "PATH_AUTO",
    "PATH_GEMV", "PATH_MMQ", "TYPE_F32", "TYPE_F16", "TYPE_Q4_0", "TYPE_Q8_0", "TYPE_Q4_K", "TYPE_Q5_K",
    "TYPE_Q6_K", "TYPE_Q8_K", "TYPE_Q8_0_RS",
    "TYPE_NAMES", "KV_BLOCK_SIZE", "PagedKVCache", "kv_slot_bytes", "kv_attention_workspace_size",
]
