"""ctypes binding of libdcq (include/dcq.h) with torch-tensor conveniences.

Every function maps 1:1 onto an extern "C" entry point. Non-zero status codes
raise DcqError carrying dcq_status_string(). Device tensors are passed as raw
pointers; the stream is torch's current stream unless one is given.
"""
import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdcq.so")
SYMBOLS = [
    "dcq_version", "dcq_status_string", "dcq_block_size", "dcq_type_size", "dcq_row_size", "dcq_vec_dot_type",
    "dcq_supports_mul_mat", "dcq_quantize_rows", "dcq_mul_mat_workspace_size", "dcq_mul_mat", "dcq_mul_mat_ex",
    "dcq_block_sums_per_row", "dcq_dot_rows", "dcq_quantize_weights", "dcq_repack_weights", "dcq_dequantize_rows",
    "dcq_quantize_src1", "dcq_mul_mat_q", "dcq_mul_mat_add_workspace_size", "dcq_mul_mat_add",
    "dcq_ffn_gate_up_workspace_size", "dcq_ffn_gate_up", "dcq_mul_mat_noalloc",
    "dcq_gguf_open", "dcq_gguf_close", "dcq_gguf_tensor_count", "dcq_gguf_find_tensor", "dcq_gguf_tensor_info",
    "dcq_gguf_get_int", "dcq_gguf_get_str", "dcq_gguf_load_tensor",
    "dcq_kv_slot_bytes", "dcq_kv_write", "dcq_kv_gather", "dcq_kv_attention_workspace_size", "dcq_kv_attention",
    "dcq_probe_stream_read",  # include/dcq_probe.h: measurement aid
]

KV_BLOCK_SIZE = 16

PATH_AUTO, PATH_GEMV, PATH_MMQ = 0, 1, 2

_lib = None


class DcqError(RuntimeError):
    def __init__(self, fn, status):
        self.status = status
        super().__init__(f"{fn} failed: status {status} ({status_string(status)})")


def build():
    """Compile libdcq.so for gfx950 in-tree (hipcc cross-compiles without a GPU)."""
    subprocess.check_call(["make", "-s", "-j8", "-C", os.path.join(HERE, "csrc")])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with densecore_amd.build() "
                              "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
        sig = {
            "dcq_version": (ctypes.c_char_p, []),
            "dcq_status_string": (ctypes.c_char_p, [i32]),
            "dcq_block_size": (i64, [i32]),
            "dcq_type_size": (i64, [i32]),
            "dcq_row_size": (sz, [i32, i64]),
            "dcq_vec_dot_type": (i32, [i32]),
            "dcq_supports_mul_mat": (i32, [i32, i32, i32]),
            "dcq_quantize_rows": (i32, [i32, vp, i64, i64, sz, vp, vp]),
            "dcq_mul_mat_workspace_size": (sz, [i32, i64, i64]),
            "dcq_mul_mat": (i32, [i32, vp, i64, i64, sz, vp, i64, sz, vp, sz, vp, sz, vp]),
            "dcq_mul_mat_ex": (i32, [i32, vp, i64, i64, sz, vp, i64, sz, vp, sz, vp, sz, i32, vp, vp]),
            "dcq_block_sums_per_row": (i64, [i32, i64]),
            "dcq_dot_rows": (i32, [i32, vp, sz, vp, i64, vp, i64, i64, vp]),
            "dcq_quantize_weights": (i32, [i32, vp, i64, i64, vp, vp]),
            "dcq_dequantize_rows": (i32, [i32, vp, i64, i64, sz, vp, vp]),
            "dcq_repack_weights": (i32, [i32, vp, i64, i64, sz, i32, vp, sz, vp]),
            "dcq_quantize_src1": (i32, [i32, vp, i64, i64, sz, vp, sz, vp]),
            "dcq_mul_mat_q": (i32, [i32, vp, i64, i64, sz, vp, sz, i64, vp, sz, i32, vp]),
            "dcq_mul_mat_add_workspace_size": (sz, [i32, i64, i64, i64]),
            "dcq_mul_mat_add": (i32, [i32, vp, i64, i64, sz, vp, i64, sz, vp, sz, vp, sz, vp, sz, vp]),
            "dcq_ffn_gate_up_workspace_size": (sz, [i32, i64, i64, i64]),
            "dcq_ffn_gate_up": (i32, [i32, vp, vp, i64, i64, sz, vp, i64, sz, vp, sz, vp, sz, vp]),
            "dcq_mul_mat_noalloc": (i32, [i32, vp, i64, i64, sz, vp, i64, sz, vp, sz, vp]),
            "dcq_gguf_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            "dcq_gguf_close": (None, [vp]),
            "dcq_gguf_tensor_count": (i64, [vp]),
            "dcq_gguf_find_tensor": (i64, [vp, ctypes.c_char_p]),
            "dcq_gguf_tensor_info": (i32, [vp, i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32),
                                           ctypes.POINTER(i32), ctypes.POINTER(i64), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64)]),
            "dcq_gguf_get_int": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(i64)]),
            "dcq_gguf_get_str": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
            "dcq_gguf_load_tensor": (i32, [vp, i64, vp, sz, vp]),
            "dcq_kv_slot_bytes": (sz, [i32, i64]),
            "dcq_kv_write": (i32, [i32, vp, i64, i32, i32, i64, vp, i64, i64, vp, sz, i64, vp]),
            "dcq_kv_gather": (i32, [i32, vp, i64, i32, i32, i64, vp, i64, i64, vp, sz, i64, vp, sz, vp]),
            "dcq_kv_attention_workspace_size": (sz, [i32, i32, i32, i64, i64]),
            "dcq_kv_attention": (i32, [i32, vp, vp, i64, i32, i32, vp, i64, i32, i32, i32, vp, sz, vp, vp, sz,
                                       i64, i64, ctypes.c_float, vp, sz, vp, sz, vp]),
            "dcq_probe_stream_read": (i32, [vp, sz, i32, i32, vp, vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def status_string(s):
    return lib().dcq_status_string(s).decode()


def _check(fn, status):
    if status != 0:
        raise DcqError(fn, status)


def version():
    return lib().dcq_version().decode()


def block_size(t):
    return int(lib().dcq_block_size(t))


def type_size(t):
    return int(lib().dcq_type_size(t))


def row_size(t, k):
    return int(lib().dcq_row_size(t, k))


def vec_dot_type(t):
    return int(lib().dcq_vec_dot_type(t))


def supports_mul_mat(wt, xt=0, yt=0):
    return bool(lib().dcq_supports_mul_mat(wt, xt, yt))


def block_sums_per_row(wt, k):
    return int(lib().dcq_block_sums_per_row(wt, k))


def mul_mat_workspace_size(wt, m, k):
    return int(lib().dcq_mul_mat_workspace_size(wt, m, k))


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(name, t, dtype, ndim=(1, 2), cuda=True):
    """Raise ValueError unless t is a tensor of `dtype` with a dimension count in `ndim`, on a GPU
    (when `cuda`), whose last dimension is contiguous: the ABI takes raw pointers and row strides,
    so anything else would be read as the wrong bytes."""
    import torch
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a torch tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if t.dim() not in ndim:
        raise ValueError(f"{name}: {t.dim()} dimensions, expected {' or '.join(map(str, ndim))}")
    if t.numel() > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name}: last dimension has stride {t.stride(-1)}, expected 1")
    if cuda and not t.is_cuda:
        raise ValueError(f"{name}: tensor on {t.device}, expected a GPU tensor")


def _f32(name, t, ndim=(2,)):
    import torch
    _need(name, t, torch.float32, ndim)


def _u8(name, t, ndim=(1, 2)):
    import torch
    _need(name, t, torch.uint8, ndim)


def quantize_rows(vdt, x, out=None, stream=None):
    """x: float32 cuda [M, K] -> uint8 cuda [M, row_size(vdt, K)] in ggml block layout."""
    import torch
    _f32("x", x)
    m, k = x.shape
    if out is None:
        out = torch.empty((m, row_size(vdt, k)), dtype=torch.uint8, device=x.device)
    _u8("out", out)
    _check("dcq_quantize_rows", lib().dcq_quantize_rows(vdt, _ptr(x), m, k, x.stride(0) * 4, _ptr(out),
                                                        _stream(stream)))
    return out


def mul_mat_ex(wt, wq, n, k, x, y=None, workspace=None, path=PATH_AUTO, block_sums=None, w_row_bytes=None,
               stream=None):
    """Y[M, N] = W[N, K] (quantized rows, uint8 cuda) x X[M, K]^T (float32 cuda)."""
    import torch
    _u8("wq", wq)
    _f32("x", x)
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _f32("y", y)
    if block_sums is not None:
        _need("block_sums", block_sums, torch.int32, (1, 2, 3))
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("dcq_mul_mat_ex", lib().dcq_mul_mat_ex(
        wt, _ptr(wq), n, k, wrb, _ptr(x), m, x.stride(0) * 4, _ptr(y), y.stride(0) * 4, _ptr(workspace), ws_bytes,
        path, _ptr(block_sums), _stream(stream)))
    return y


def mul_mat(wt, wq, n, k, x, y=None, workspace=None, w_row_bytes=None, stream=None):
    import torch
    _u8("wq", wq)
    _f32("x", x)
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _f32("y", y)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("dcq_mul_mat", lib().dcq_mul_mat(
        wt, _ptr(wq), n, k, wrb, _ptr(x), m, x.stride(0) * 4, _ptr(y), y.stride(0) * 4, _ptr(workspace), ws_bytes,
        _stream(stream)))
    return y


NOALLOC_SCRATCH_BYTES = 8 << 20  # DCQ_NOALLOC_SCRATCH_BYTES


def mul_mat_noalloc(wt, wq, n, k, x, y, w_row_bytes=None, stream=None):
    """dcq_mul_mat_noalloc: dcq_mul_mat with the library's static device scratch as workspace
    (no allocation on the library side; y must be given)."""
    _u8("wq", wq)
    _f32("x", x)
    _f32("y", y)
    m = x.shape[0]
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _check("dcq_mul_mat_noalloc", lib().dcq_mul_mat_noalloc(
        wt, _ptr(wq), n, k, wrb, _ptr(x), m, x.stride(0) * 4, _ptr(y), y.stride(0) * 4, _stream(stream)))
    return y


def mul_mat_add_workspace_size(wt, m, n, k):
    return lib().dcq_mul_mat_add_workspace_size(wt, m, n, k)


def mul_mat_add(wt, wq, n, k, x, r, y=None, workspace=None, w_row_bytes=None, stream=None):
    """Y[M, N] = W x + R: a projection and its residual (R [M, N], may be y itself) or bias (R [N],
    broadcast over the rows)."""
    import torch
    _u8("wq", wq)
    _f32("x", x)
    _f32("r", r, (1, 2))
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _f32("y", y)
    r_stride = 0 if r.dim() == 1 else r.stride(0) * 4
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("dcq_mul_mat_add", lib().dcq_mul_mat_add(
        wt, _ptr(wq), n, k, wrb, _ptr(x), m, x.stride(0) * 4, _ptr(r), r_stride, _ptr(y), y.stride(0) * 4,
        _ptr(workspace), ws_bytes, _stream(stream)))
    return y


def ffn_gate_up_workspace_size(wt, m, n, k):
    return lib().dcq_ffn_gate_up_workspace_size(wt, m, n, k)


def ffn_gate_up(wt, wg, wu, n, k, x, y=None, workspace=None, w_row_bytes=None, stream=None):
    """Y[M, N] = silu(Wg x) * (Wu x): the SwiGLU gate/up pair with one activation quantization."""
    import torch
    _u8("wg", wg)
    _u8("wu", wu)
    _f32("x", x)
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _f32("y", y)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("dcq_ffn_gate_up", lib().dcq_ffn_gate_up(
        wt, _ptr(wg), _ptr(wu), n, k, wrb, _ptr(x), m, x.stride(0) * 4, _ptr(y), y.stride(0) * 4, _ptr(workspace),
        ws_bytes, _stream(stream)))
    return y


class GGUF:
    """A GGUF weight file (dcq_gguf_*): tensor table and metadata parsed on the host, tensors
    streamed into device memory in the block layout dcq_mul_mat takes."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check("dcq_gguf_open", lib().dcq_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().dcq_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        return lib().dcq_gguf_tensor_count(self._h)

    def find(self, name):
        return lib().dcq_gguf_find_tensor(self._h, name.encode())

    def info(self, i):
        name, typ, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        ne = (ctypes.c_int64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _check("dcq_gguf_tensor_info", lib().dcq_gguf_tensor_info(
            self._h, i, ctypes.byref(name), ctypes.byref(typ), ctypes.byref(nd), ne, ctypes.byref(off),
            ctypes.byref(nb)))
        return {"name": name.value.decode(), "type": typ.value, "ne": list(ne[:nd.value]),
                "file_offset": off.value, "nbytes": nb.value}

    def get_int(self, key):
        v = ctypes.c_int64()
        _check("dcq_gguf_get_int", lib().dcq_gguf_get_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key):
        v = ctypes.c_char_p()
        _check("dcq_gguf_get_str", lib().dcq_gguf_get_str(self._h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def load(self, i, dst=None, device="cuda:0", stream=None):
        """The tensor's bytes as a uint8 device tensor (rows packed: [ne[1]*..., row bytes])."""
        import torch
        meta = self.info(i)
        if dst is None:
            dst = torch.empty(meta["nbytes"], dtype=torch.uint8, device=device)
        _check("dcq_gguf_load_tensor", lib().dcq_gguf_load_tensor(
            self._h, i, _ptr(dst), dst.numel() * dst.element_size(), _stream(stream)))
        return dst


def dot_rows(wt, wq, xq_row, k, n0, n1, y=None, w_row_bytes=None, stream=None):
    """ComputeDotProductBatch: y[r - n0] = vec_dot(W row r, xq_row), xq_row pre-quantized (ggml layout)."""
    import torch
    _u8("wq", wq)
    _u8("xq_row", xq_row)
    if y is None:
        y = torch.empty((max(n1 - n0, 0),), dtype=torch.float32, device=wq.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _check("dcq_dot_rows", lib().dcq_dot_rows(wt, _ptr(wq), wrb, _ptr(xq_row), k, _ptr(y), n0, n1,
                                              _stream(stream)))
    return y


def quantize_weights(wt, w, out=None, stream=None):
    """w: float32 cuda [N, K] -> uint8 cuda [N, row_size(wt, K)] (ggml_quantize_chunk)."""
    import torch
    _f32("w", w)
    if not w.is_contiguous():
        raise ValueError("w: rows must be packed (contiguous)")
    n, k = w.shape
    if out is None:
        out = torch.empty((n, row_size(wt, k)), dtype=torch.uint8, device=w.device)
    _check("dcq_quantize_weights", lib().dcq_quantize_weights(wt, _ptr(w), n, k, _ptr(out), _stream(stream)))
    return out


def repack_weights(wt, wq, n, k, out_type, out=None, w_row_bytes=None, stream=None):
    """Load-time repack (dcq_repack_weights): N rows of `wt` (uint8 cuda) -> uint8 cuda [N, row_size(out_type, K)]
    rows of out_type (Q8_0 -> row-split Q8_0)."""
    import torch
    _u8("wq", wq)
    if out is None:
        out = torch.empty((n, row_size(out_type, k)), dtype=torch.uint8, device=wq.device)
    _u8("out", out)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    orb = out.stride(0) if out.dim() == 2 else row_size(out_type, k)
    _check("dcq_repack_weights", lib().dcq_repack_weights(wt, _ptr(wq), n, k, wrb, out_type, _ptr(out), orb,
                                                          _stream(stream)))
    return out


def dequantize_rows(t, wq, n, k, y=None, w_row_bytes=None, stream=None):
    import torch
    _u8("wq", wq)
    if y is None:
        y = torch.empty((n, k), dtype=torch.float32, device=wq.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(t, k)
    _check("dcq_dequantize_rows", lib().dcq_dequantize_rows(t, _ptr(wq), n, k, wrb, _ptr(y), _stream(stream)))
    return y


def quantize_src1(wt, x, workspace, stream=None):
    """Quantize X [M, K] once into `workspace` (uint8 cuda, mul_mat_workspace_size bytes)."""
    _f32("x", x)
    _u8("workspace", workspace, (1,))
    m, k = x.shape
    _check("dcq_quantize_src1", lib().dcq_quantize_src1(wt, _ptr(x), m, k, x.stride(0) * 4, _ptr(workspace),
                                                        workspace.numel(), _stream(stream)))
    return workspace


def mul_mat_q(wt, wq, n, k, workspace, m, y=None, path=PATH_AUTO, w_row_bytes=None, stream=None):
    """Y[M, N] from W and activations already quantized by quantize_src1 into `workspace`."""
    import torch
    _u8("wq", wq)
    _u8("workspace", workspace, (1,))
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=wq.device)
    wrb = w_row_bytes if w_row_bytes is not None else row_size(wt, k)
    _check("dcq_mul_mat_q", lib().dcq_mul_mat_q(wt, _ptr(wq), n, k, wrb, _ptr(workspace), workspace.numel(), m,
                                                _ptr(y), y.stride(0) * 4, path, _stream(stream)))
    return y


# ---------------------------------------------------------------- paged KV cache
def kv_slot_bytes(cache_type, row_elems):
    return int(lib().dcq_kv_slot_bytes(cache_type, row_elems))


class PagedKVCache:
    """K and V arenas of DenseCore's paged KV cache in device memory (layout of the reference's
    PagedKVCache, core/src/kv_cache.cpp:341-409): n_blocks blocks of 16 token slots per layer,
    each slot one token's row of n_head_kv * head_dim values in cache_type (F32, F16, Q8_0).
    Block tables are int32 device tensors mapping position // 16 to an arena block."""

    def __init__(self, cache_type, n_blocks, n_layer, n_head_kv, head_dim, device="cuda"):
        import torch
        self.cache_type, self.n_blocks, self.n_layer = cache_type, n_blocks, n_layer
        self.n_head_kv, self.head_dim = n_head_kv, head_dim
        self.row_elems = n_head_kv * head_dim
        self.slot_bytes = kv_slot_bytes(cache_type, self.row_elems)
        if self.slot_bytes == 0:
            raise DcqError("dcq_kv_slot_bytes", -2)
        nbytes = n_blocks * n_layer * KV_BLOCK_SIZE * self.slot_bytes
        self.k = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        self.v = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    def _arena(self, which):
        return self.k if which == "k" else self.v

    def write(self, which, layer, table, pos0, rows, stream=None):
        """WriteKSlot / WriteVSlot for rows [N, row_elems] at positions pos0 .. pos0 + N - 1."""
        import torch
        _f32("rows", rows, (1, 2))
        _need("table", table, torch.int32, (1,))
        _check("dcq_kv_write", lib().dcq_kv_write(
            self.cache_type, _ptr(self._arena(which)), self.n_blocks, self.n_layer, layer, self.row_elems,
            _ptr(table), table.numel(), pos0, _ptr(rows), rows.stride(0) * 4 if rows.dim() == 2 else 0,
            rows.shape[0], _stream(stream)))

    def gather(self, which, layer, table, n_past, cur, out=None, stream=None):
        """[n_past + N, row_elems] fp32: history from the cache, then cur (cb_kv_update_and_gather)."""
        import torch
        _f32("cur", cur)
        if table is not None:
            _need("table", table, torch.int32, (1,))
        n = cur.shape[0]
        if out is None:
            out = torch.empty((n_past + n, self.row_elems), dtype=torch.float32, device=cur.device)
        _f32("out", out)
        _check("dcq_kv_gather", lib().dcq_kv_gather(
            self.cache_type, _ptr(self._arena(which)), self.n_blocks, self.n_layer, layer, self.row_elems,
            _ptr(table), table.numel() if table is not None else 0, n_past, _ptr(cur), cur.stride(0) * 4, n,
            _ptr(out), out.stride(0) * 4, _stream(stream)))
        return out

    def attention(self, layer, table, q, k_cur, v_cur, n_past, scale, out=None, workspace=None, stream=None):
        """q [N, n_head * head_dim] fp32 -> out [N, n_head * head_dim]: causal attention of the N
        batch tokens (positions n_past ..) over the cached history and their own k_cur / v_cur rows."""
        import torch
        if k_cur.stride(0) != v_cur.stride(0):
            raise ValueError(f"k_cur and v_cur must share a row stride (the ABI takes one): "
                             f"{k_cur.stride(0)} != {v_cur.stride(0)}")
        for name, t in (("q", q), ("k_cur", k_cur), ("v_cur", v_cur)):
            _f32(name, t)
        if table is not None:
            _need("table", table, torch.int32, (1,))
        n = q.shape[0]
        n_head = q.shape[1] // self.head_dim
        if out is None:
            out = torch.empty((n, n_head * self.head_dim), dtype=torch.float32, device=q.device)
        _f32("out", out)
        need = kv_attention_workspace_size(n_head, self.n_head_kv, self.head_dim, n, n_past)
        if workspace is None and need:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
        _check("dcq_kv_attention", lib().dcq_kv_attention(
            self.cache_type, _ptr(self.k), _ptr(self.v), self.n_blocks, self.n_layer, layer, _ptr(table),
            table.numel() if table is not None else 0, n_head, self.n_head_kv, self.head_dim, _ptr(q),
            q.stride(0) * 4, _ptr(k_cur), _ptr(v_cur), k_cur.stride(0) * 4, n, n_past, scale, _ptr(out),
            out.stride(0) * 4, _ptr(workspace), ws_bytes, _stream(stream)))
        return out


def kv_attention_workspace_size(n_head, n_head_kv, head_dim, n_tokens, n_past):
    return int(lib().dcq_kv_attention_workspace_size(n_head, n_head_kv, head_dim, n_tokens, n_past))


# ---------------------------------------------------------------- measurement aid (include/dcq_probe.h)
def probe_stream_read(src, nbytes, per_lane, max_workgroups, sink, stream=None):
    """Read nbytes of the device tensor src with the pure streaming kernel (no result)."""
    _check("dcq_probe_stream_read", lib().dcq_probe_stream_read(_ptr(src), nbytes, per_lane, max_workgroups,
                                                                _ptr(sink), _stream(stream)))
