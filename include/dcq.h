/*
 * dcq.h — C ABI of libdcq, the MI355X (gfx950) quantized mul_mat backend.
 *
 * It replaces the compute behind ggml's MUL_MAT for GGUF Q8_0 / Q4_K / Q6_K
 * weights (and the quantize tool's Q4_0 / Q5_K, core/src/quantize.cpp:71-78)
 * times fp32 activations with fp32 output, the operator DenseCore's
 * graph emits for every FFN / attention projection:
 *   core/src/inference.cpp:1063, 1794-1797, 1817 (ggml_mul_mat call sites),
 *   core/src/worker.cpp:544 (ggml_backend_graph_compute executes them),
 *   core/src/inference.cpp:840-948 (cb_gemv_custom, the M == 1 custom op).
 * Paths in citations are relative to the DenseCore source tree.
 *
 * Conventions
 *   - Plain C types only. `stream` is a hipStream_t passed as void* (NULL =
 *     the null stream). Every call is stream-ordered and asynchronous.
 *   - All data pointers are device pointers owned by the caller; nothing is
 *     freed across the ABI.
 *   - Type ids are ggml's: F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12,
 *     Q5_K = 13, Q6_K = 14, Q8_K = 15; and one layout of this library's own,
 *     DCQ_TYPE_Q8_0_RS (Q8_0 rows repacked at load time, see dcq_repack_weights).
 *   - Dimensions: W is [N][K] (N output rows, K reduction), row r starts at
 *     W + r * w_row_bytes. X is [M][K] fp32 with row stride x_stride_bytes.
 *     Y is [M][N] fp32 with row stride y_stride_bytes:
 *       Y[m][n] = vec_dot(W row n, quantize_{vec_dot_type}(X row m)).
 *   - Status: 0 on success, a negative DCQ_ERR_* otherwise. Arguments are
 *     validated before any device work, so an error never leaves a partial
 *     result (unlike the reference's silent zero-fill / early return,
 *     core/src/inference.cpp:842-879, core/src/simd_ops.cpp:193-196).
 *   - The quantized activation bytes are bit-exact with ggml's from_float
 *     for the vec_dot_type (Q8_0: x86 SIMD semantics, round-half-even with
 *     id = 127/amax; Q8_K: quantize_row_q8_K_ref); the per-block int32 sums
 *     are exact; fp32 outputs differ from a CPU vec_dot only by summation
 *     order.
 */
#ifndef DCQ_H
#define DCQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids */
#define DCQ_TYPE_F32 0
#define DCQ_TYPE_F16 1
#define DCQ_TYPE_Q4_0 2
#define DCQ_TYPE_Q8_0 8
#define DCQ_TYPE_Q4_K 12
#define DCQ_TYPE_Q5_K 13
#define DCQ_TYPE_Q6_K 14
#define DCQ_TYPE_Q8_K 15
/* Row-split Q8_0 (not a ggml type): a row of K elements holds its K int8 quants first (block b's 32
 * at byte 32b), then its K/32 fp16 scales (block b's at byte K + 2b): Q8_0's 34 bytes per block and
 * values, split into two planes so that every 16-byte piece of quants is 16-byte aligned. Written by
 * dcq_repack_weights; K % 256 == 0 and row strides multiples of 16 bytes. */
#define DCQ_TYPE_Q8_0_RS 108

/* status codes */
#define DCQ_OK 0
#define DCQ_ERR_INVALID_ARG (-1)     /* null pointer, negative size, bad stride */
#define DCQ_ERR_UNSUPPORTED (-2)     /* type (or type pair) not supported */
#define DCQ_ERR_BAD_SHAPE (-3)       /* K not a multiple of the block size, empty dims */
#define DCQ_ERR_MISALIGNED (-4)      /* pointer / stride alignment the kernels need */
#define DCQ_ERR_WORKSPACE (-5)       /* workspace smaller than dcq_mul_mat_workspace_size */
#define DCQ_ERR_HIP (-6)             /* a HIP runtime call failed */
#define DCQ_ERR_NO_DEVICE (-7)       /* no usable gfx950 device */
#define DCQ_ERR_FORMAT (-8)          /* malformed GGUF file */
#define DCQ_ERR_IO (-9)              /* file could not be opened or read */
#define DCQ_ERR_NOT_FOUND (-10)      /* GGUF metadata key not present */
#define DCQ_ERR_SCRATCH_LIMIT (-11)  /* needs more than DCQ_NOALLOC_SCRATCH_BYTES (dcq_mul_mat_noalloc) */

/* kernel path selection for dcq_mul_mat_ex */
#define DCQ_PATH_AUTO 0
#define DCQ_PATH_GEMV 1 /* wave-per-row-group int8 dot (sdot4), any M (tiled by 8) */
#define DCQ_PATH_MMQ 2  /* int8 MFMA tiles, any M */

/* Library version string, e.g. "dcq 0.1.0 gfx950". */
const char* dcq_version(void);
/* Human-readable text for a status code. */
const char* dcq_status_string(int status);

/* ---- type traits (ggml_type_traits / ggml_row_size equivalents) ---- */
/* Elements per block: Q4_0/Q8_0 32, Q4_K/Q5_K/Q6_K/Q8_K 256, F32/F16 1; 0 if unknown. */
int64_t dcq_block_size(int type);
/* Bytes per block: Q4_0 18, Q8_0 34, Q4_K 144, Q5_K 176, Q6_K 210, Q8_K 292, F32 4, F16 2;
 * 0 if unknown. */
int64_t dcq_type_size(int type);
/* Bytes of one row of K elements (ggml_row_size, core/src/inference.cpp:977); 0 if K is not
 * a multiple of the block size. */
size_t dcq_row_size(int type, int64_t k);
/* vec_dot_type of a weight type (core/src/inference.cpp:970-984, core/include/simd_ops.h:
 * 3298-3305): Q8_0 -> Q8_0, Q4_K/Q5_K/Q6_K -> Q8_K; and Q4_0 -> Q8_0, ggml's trait for the type
 * the reference's quantize tool emits by default (core/src/quantize.cpp:71-72, 90);
 * DCQ_ERR_UNSUPPORTED otherwise. */
int dcq_vec_dot_type(int wtype);
/* 1 if MUL_MAT(src0 = wtype, src1 = xtype) -> ytype is computed by this library, else 0
 * (the check a ggml backend's supports_op answers). */
int dcq_supports_mul_mat(int wtype, int xtype, int ytype);

/* ---- activation quantization: from_float of the vec_dot_type ----
 * Replaces type_traits_cpu(vec_dot_type)->from_float (core/src/inference.cpp:889-892).
 * Quantizes M rows of K floats into the ggml block layout, rows packed
 * (row r at Xq + r * dcq_row_size(vec_dot_type, K)). vec_dot_type: Q8_0 or Q8_K. */
int dcq_quantize_rows(int vec_dot_type, const float* X, int64_t M, int64_t K, size_t x_stride_bytes,
                      void* Xq, void* stream);

/* ---- the operator ----
 * GGML_OP_MUL_MAT for src0 = W (wtype in {Q8_0, Q4_K, Q6_K}, and the quantize tool's Q4_0 and
 * Q5_K, core/src/quantize.cpp:71-78), src1 = X (F32), dst = Y (F32):
 * quantizes X once into the workspace, then computes every (m, n) dot
 * (replaces the quantize + chunked vec_dot of ggml's CPU MUL_MAT, executed from
 * core/src/worker.cpp:544, and cb_gemv_custom, core/src/inference.cpp:840-948).
 * Requirements: K % block_size(wtype) == 0; W 16-byte aligned; w_row_bytes >= row_size, even, and
 * a multiple of 16 for Q4_K and Q5_K; X 16-byte aligned with x_stride_bytes % 16 == 0; Y 4-byte aligned
 * with y_stride_bytes % 4 == 0.
 * workspace may be NULL (the library then takes stream-ordered scratch); otherwise it must be
 * 256-byte aligned and should hold dcq_mul_mat_workspace_size(wtype, M, K) bytes: the quantized
 * activation, and at M > 4 room for split-K partial sums (M * 128 KB, at most 16 MB) that the
 * MFMA kernels use when the output tiles cannot occupy every CU (few weight rows, long K). A
 * workspace that holds only the quantized activation is accepted and runs without split-K
 * (smaller returns DCQ_ERR_WORKSPACE). The split count depends on the shape, the device's CU
 * count and that room; for a given one the result bits are fixed. */
size_t dcq_mul_mat_workspace_size(int wtype, int64_t M, int64_t K);
int dcq_mul_mat(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X,
                int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes, void* workspace,
                size_t workspace_bytes, void* stream);

/* dcq_mul_mat with an explicit kernel path and, optionally, the per-block int32 sums the
 * kernel scaled (block_sums != NULL: int32 [M][N][dcq_block_sums_per_row(wtype, K)], written
 * with atomics, so it must be zeroed by the caller; a debugging aid — slower). */
int dcq_mul_mat_ex(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes,
                   const float* X, int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes,
                   void* workspace, size_t workspace_bytes, int path, int32_t* block_sums,
                   void* stream);
/* Number of int32 block sums per (m, n): Q8_0 K/32 (I_b = sum qw*qa over a 32-block); Q4_0
 * K/32 (I_b = sum (qw - 8)*qa); Q4_K and Q5_K 2*K/256 (per superblock: sum_j sc_j*I_j, then
 * sum_j m_j*S_j); Q6_K K/256 (per superblock: sum_g sc_g*I_g). 0 if unsupported. */
int64_t dcq_block_sums_per_row(int wtype, int64_t k);

/* ---- the operator in two halves (ggml MUL_MAT's wdata step made explicit) ----
 * dcq_quantize_src1 quantizes X once into `workspace` (the library's planar layout, sized by
 * dcq_mul_mat_workspace_size(wtype, M, K)); dcq_mul_mat_q then computes Y from W and that
 * workspace. One quantization can feed several weights that share X (ffn gate and up,
 * core/src/inference.cpp:1794-1797). The workspace must not be written between the two calls.
 * dcq_mul_mat_q only reads the workspace, so several calls that share one quantization may run
 * concurrently on different streams. It therefore never splits K (split-K writes partial sums
 * into workspace room): its result equals dcq_mul_mat's with a workspace that holds only the
 * quantized activation, bit for bit; dcq_mul_mat with the full workspace may split and differ in
 * the last fp32 bits. */
int dcq_quantize_src1(int wtype, const float* X, int64_t M, int64_t K, size_t x_stride_bytes,
                      void* workspace, size_t workspace_bytes, void* stream);
int dcq_mul_mat_q(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes,
                  const void* workspace, size_t workspace_bytes, int64_t M, float* Y,
                  size_t y_stride_bytes, int path, void* stream);

/* ---- the operator without allocation ----
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * stream capture, serving loops or harnesses that forbid hipMalloc). Same arguments, result and
 * kernels as dcq_mul_mat with workspace = NULL, except that the workspace is a static device
 * array that the library holds on each GPU it runs on until the process ends, instead of
 * stream-ordered scratch: DCQ_NOALLOC_SCRATCH_BYTES (8 MiB) for the quantized activation and
 * 16 MiB of split-K room after it. No hipMalloc, hipFree or other allocating call is made. A
 * product whose quantized activation exceeds DCQ_NOALLOC_SCRATCH_BYTES returns
 * DCQ_ERR_SCRATCH_LIMIT before any device work (M*K up to about 7.4 M elements).
 * Every call on one GPU shares that GPU's array: calls on one stream are ordered, but calls that
 * overlap on one GPU (different streams, or host threads without ordering) race on it. */
#define DCQ_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int dcq_mul_mat_noalloc(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X,
                        int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes, void* stream);

/* Activation rows up to which dcq_mul_mat's automatic path (and dcq_mul_mat_add and
 * dcq_ffn_gate_up) takes the decode GEMV kernels: 4 in general; for Q6_K weights 8 when
 * N >= 32768 (LM heads), else 4 when N < 4096 or K/256 is 10..16, else 2; for Q8_0 and row-split
 * Q8_0 weights 8 when K <= 1024, 2 when K >= 4096 and N >= 4096; for Q4_K and Q5_K weights 2 when
 * K >= 4096 and N * K >= 2^25; 8 for other small matrices (Q4_0
 * with K <= 1024 and N <= 4096, Q4_K and Q5_K with N * K <= 2048 * 2048); for other Q4_0 weights 4
 * when K <= 2048, else 2. The eight-row cases hold where the GEMV quantizes the activation itself
 * (dcq_mul_mat_q, on a pre-quantized activation, keeps 4 there). Larger M goes to the batched and
 * prefill MFMA kernels. */
#define DCQ_DECODE_ROWS(wtype, N, K)                                                                 \
    ((wtype) == DCQ_TYPE_Q6_K                                                                        \
         ? ((N) >= 32768 ? 8 : ((N) < 4096 || ((K) / 256 >= 10 && (K) / 256 <= 16)) ? 4 : 2)         \
     : ((wtype) == DCQ_TYPE_Q8_0 || (wtype) == DCQ_TYPE_Q8_0_RS)                                     \
         ? ((K) <= 1024 ? 8 : ((K) >= 4096 && (N) >= 4096) ? 2 : 4)                                  \
     : ((wtype) == DCQ_TYPE_Q4_0 && (K) <= 1024 && (N) <= 4096) ||                                   \
             (((wtype) == DCQ_TYPE_Q4_K || (wtype) == DCQ_TYPE_Q5_K) && (int64_t)(N) * (K) <= 2048 * 2048) \
         ? 8                                                                                         \
     : (wtype) == DCQ_TYPE_Q4_0 ? ((K) <= 2048 ? 4 : 2)                                               \
     : (((wtype) == DCQ_TYPE_Q4_K || (wtype) == DCQ_TYPE_Q5_K) && (K) >= 4096 &&                      \
        (int64_t)(N) * (K) >= ((int64_t)1 << 25))                                                    \
         ? 2                                                                                         \
         : 4)

/* ---- a projection and its residual or bias ----
 * Y[m][n] = (sum_k W[n][k] x[m][k]) + R[m][n], one fp32 add per element after dcq_mul_mat's
 * product: the reference's residual connections cur = ggml_add(mul_mat(wo, .), inpL) and
 * ggml_add(mul_mat(w2, .), inpFF) (core/src/inference.cpp:1763-1764, 1799-1800), and the
 * projection biases bq/bk/bv/bo (core/src/inference.cpp:1133-1151, 1760-1761). Y equals
 * dcq_mul_mat's output plus R bit for bit. r_stride_bytes 0 broadcasts one bias row of N
 * floats; otherwise it is >= N*4. R may be Y itself (r_stride_bytes == y_stride_bytes: the
 * in-place residual) or must not overlap Y. R 4-byte aligned, strides multiples of 4; the rest
 * as dcq_mul_mat. Where the decode kernels serve the product (M <= DCQ_DECODE_ROWS(wtype, N))
 * the add is their store; otherwise the product goes to Y (or, when R is Y, a workspace
 * temporary) and one add kernel follows. workspace may
 * be NULL; otherwise it should hold dcq_mul_mat_add_workspace_size(wtype, M, N, K) bytes,
 * 256-byte aligned (the split-K room at its end is optional, as in dcq_mul_mat). */
size_t dcq_mul_mat_add_workspace_size(int wtype, int64_t M, int64_t N, int64_t K);
int dcq_mul_mat_add(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes,
                    const float* X, int64_t M, size_t x_stride_bytes, const float* R,
                    size_t r_stride_bytes, float* Y, size_t y_stride_bytes, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- the SwiGLU gate/up pair ----
 * Y[m][n] = silu(sum_k Wg[n][k] x[m][k]) * (sum_k Wu[n][k] x[m][k]), silu(g) = g / (1 + e^-g):
 * the reference FFN's w1 = mul_mat(W1, x), w3 = mul_mat(W3, x), ggml_mul(ggml_silu(w1), w3)
 * (core/src/inference.cpp:1794-1796) in one call. Both weights share wtype, shape and row
 * stride, and X's quantization. At M <= DCQ_DECODE_ROWS(wtype, N) (Q4_K, Q8_0) one fused kernel
 * streams both weight rows; otherwise (and for Q4_0, Q5_K, Q6_K) X is quantized once, both
 * projections run, then the product.
 * Requirements as dcq_mul_mat's, for both weights. workspace may be NULL; otherwise it should hold
 * dcq_ffn_gate_up_workspace_size(wtype, M, N, K) bytes, 256-byte aligned (the split-K room at its
 * end is optional, as in dcq_mul_mat). */
size_t dcq_ffn_gate_up_workspace_size(int wtype, int64_t M, int64_t N, int64_t K);
int dcq_ffn_gate_up(int wtype, const void* Wg, const void* Wu, int64_t N, int64_t K, size_t w_row_bytes,
                    const float* X, int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---- row-range dot with pre-quantized input ----
 * ComputeDotProductBatch (core/src/simd_ops.cpp:140-197): Y[r - n0] = vec_dot(K, W row r, Xq)
 * for r in [n0, n1); Xq is ONE row already quantized to the vec_dot_type (ggml layout, as
 * dcq_quantize_rows writes it). Unsupported types return DCQ_ERR_UNSUPPORTED instead of the
 * reference's zero-fill. */
int dcq_dot_rows(int wtype, const void* W, size_t w_row_bytes, const void* Xq, int64_t K, float* Y,
                 int64_t n0, int64_t n1, void* stream);

/* ---- weight quantization (ggml_quantize_chunk equivalent, core/src/quantize.cpp:285) ----
 * Quantizes an fp32 [N][K] matrix into wtype rows (packed, row stride dcq_row_size):
 * Q8_0 = quantize_row_q8_0_ref, Q4_0 = quantize_row_q4_0_ref, Q4_K = quantize_row_q4_K_ref,
 * Q5_K = quantize_row_q5_K_ref, Q6_K = quantize_row_q6_K_ref (no importance matrix). */
int dcq_quantize_weights(int wtype, const float* W, int64_t N, int64_t K, void* Wq, void* stream);

/* ---- load-time weight repack ----
 * The reference keeps GGUF blocks in plain host buffers (core/src/model_loader.cpp:103-105); a ggml
 * backend may instead store a tensor in its own layout when the loader hands it over (the role of
 * ggml's extra buffer types, e.g. the CPU backend's repacked weights). This converts N Q8_0 rows
 * (wtype = DCQ_TYPE_Q8_0) into DCQ_TYPE_Q8_0_RS rows (out_type) at Wr, row stride wr_row_bytes >=
 * dcq_row_size(DCQ_TYPE_Q8_0_RS, K), a multiple of 16; K % 256 == 0; W 2-byte aligned with an even
 * row stride, Wr 16-byte aligned, the two not overlapping. dcq_mul_mat (and _ex, _q, _add, _noalloc,
 * dcq_ffn_gate_up, dcq_dot_rows, dcq_dequantize_rows) take DCQ_TYPE_Q8_0_RS weights: the prefill MFMA
 * kernel then loads the quants straight into LDS (no register pass) and the other kernels read
 * aligned quants. The kernels and their arithmetic are the Q8_0 rows' (the same exact block sums
 * and fp32 steps), so dcq_mul_mat, _ex, _q, _add, _noalloc and dcq_dot_rows return the Q8_0 rows'
 * result bits; dcq_ffn_gate_up at M <= DCQ_DECODE_ROWS runs the pair as two products (the fused pair
 * kernel takes GGUF rows only), equal to the Q8_0 result up to summation order. */
int dcq_repack_weights(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, int out_type, void* Wr,
                       size_t wr_row_bytes, void* stream);

/* ---- dequantization (type_traits->to_float, core/src/inference.cpp:938-945) ----
 * Y[r][k] = value of element k of row r; N rows of K elements, Y rows packed. */
int dcq_dequantize_rows(int type, const void* Wq, int64_t N, int64_t K, size_t w_row_bytes, float* Y,
                        void* stream);

/* ---- GGUF weight ingest ----
 * The reference reads a model with ggml's gguf_init_from_file (no_alloc = false: every tensor's
 * bytes into host ggml buffers, core/src/model_loader.cpp:96-130), reads metadata with
 * gguf_find_key / gguf_get_val_* and maps tensors by name with ggml_get_tensor
 * (core/src/model_loader.cpp:294-402). Here the file is parsed on the host (GGUF v2/v3; every
 * count and length checked against the file size) and each tensor's bytes are streamed into
 * device memory the caller owns, in the block layout dcq_mul_mat takes (the tensor's ne[0] is K,
 * ne[1] is N, rows packed: w_row_bytes = dcq_row_size(type, K)). Real Q4_K_M files mix Q4_K,
 * Q6_K and F32 tensors; every ggml type with a fixed block size is accepted by the parser.
 *   dcq_gguf_open: DCQ_ERR_IO (open/read), DCQ_ERR_FORMAT (malformed), DCQ_ERR_UNSUPPORTED (a
 *     tensor type without a fixed block size).
 *   dcq_gguf_tensor_info: file_offset is the absolute byte offset of the tensor's data.
 *   dcq_gguf_get_int: any integer or bool value; dcq_gguf_get_str: string values (the pointer
 *     lives until dcq_gguf_close); DCQ_ERR_NOT_FOUND when the key is absent.
 *   dcq_gguf_load_tensor: copies nbytes to dst (device memory of at least nbytes) on `stream`
 *     through two pinned host chunks of up to 32 MB, which the handle's first load allocates and
 *     dcq_gguf_close frees; returns when the copy is complete. Loads on one handle share those
 *     chunks, so calls on one handle from several threads must not overlap. */
typedef struct dcq_gguf dcq_gguf;
int dcq_gguf_open(const char* path, dcq_gguf** out);
void dcq_gguf_close(dcq_gguf* g);
int64_t dcq_gguf_tensor_count(const dcq_gguf* g);
int64_t dcq_gguf_find_tensor(const dcq_gguf* g, const char* name);
int dcq_gguf_tensor_info(const dcq_gguf* g, int64_t i, const char** name, int* type, int* n_dims,
                         int64_t ne[4], uint64_t* file_offset, uint64_t* nbytes);
int dcq_gguf_get_int(const dcq_gguf* g, const char* key, int64_t* out);
int dcq_gguf_get_str(const dcq_gguf* g, const char* key, const char** out);
int dcq_gguf_load_tensor(const dcq_gguf* g, int64_t i, void* dst, size_t dst_bytes, void* stream);

/* ---- Paged KV cache: F32 / F16 / Q8_0 slots, and the attention that reads them ----
 * Arena layout, as the reference's PagedKVCache (core/src/kv_cache.cpp:341-409,
 * core/include/kv_cache.h:17): 16 token slots per block; slot (block, layer, s) at byte
 * ((block * n_layer + layer) * 16 + s) * dcq_kv_slot_bytes(type, row_elems), where a slot holds
 * one token's row of row_elems = n_head_kv * head_dim values, KV head h at h * head_dim.
 * n_blocks is the number of blocks the arena holds (its size is n_blocks * n_layer * 16 *
 * slot_bytes). block_table maps a sequence's logical block (position / 16) to an arena block;
 * it lives in device memory. Types: DCQ_TYPE_F32, DCQ_TYPE_F16, DCQ_TYPE_Q8_0; row_elems a
 * multiple of 32; arena, src, cur, dst, q, k_cur, v_cur 16-byte aligned with strides a multiple
 * of 16 bytes (out: 4). */
#define DCQ_KV_BLOCK_SIZE 16

/* bytes of one slot: PagedKVCache::GetBytesPerSlot (core/src/kv_cache.cpp:341-347); 0 when the
 * type is not a cache type or row_elems is not a multiple of 32. */
size_t dcq_kv_slot_bytes(int cache_type, int64_t row_elems);

/* Write n_tokens rows (positions pos0 .. pos0 + n_tokens - 1 of one sequence) into their slots:
 * PagedKVCache::WriteKSlot / WriteVSlot (core/src/kv_cache.cpp:565-598) as called per token by
 * cb_kv_update_and_gather (core/src/inference.cpp:711-745). Q8_0 is ggml_quantize_chunk's
 * quantize_row_q8_0_ref, F16 is round-to-nearest-even; bit-exact. A table entry outside
 * [0, n_blocks) is skipped, as the reference skips a null slot. The table must cover every
 * position written (DCQ_ERR_INVALID_ARG otherwise; the reference skips those tokens). */
int dcq_kv_write(int cache_type, void* arena, int64_t n_blocks, int n_layer, int layer, int64_t row_elems,
                 const int32_t* block_table, int64_t n_table, int64_t pos0, const float* src,
                 size_t src_stride_bytes, int64_t n_tokens, void* stream);

/* dst[n_past + n_tokens][row_elems] fp32: positions 0 .. n_past - 1 read from the arena, then the
 * n_tokens rows of cur as given, as cb_kv_update_and_gather leaves K_all / V_all
 * (core/src/inference.cpp:748-784; ReadKSlot at core/src/kv_cache.cpp:600-629). Positions whose
 * block is missing from the table, or outside [0, n_blocks), read as zeros. */
int dcq_kv_gather(int cache_type, const void* arena, int64_t n_blocks, int n_layer, int layer, int64_t row_elems,
                  const int32_t* block_table, int64_t n_table, int64_t n_past, const float* cur,
                  size_t cur_stride_bytes, int64_t n_tokens, float* dst, size_t dst_stride_bytes, void* stream);

/* The attention of one layer over the cache: the reference's standard path
 * (core/src/inference.cpp:1577-1746) on the K_all / V_all of dcq_kv_gather, fused: query
 * token i (position n_past + i) of q[n_tokens][n_head][head_dim] attends keys 0 .. n_past + i,
 * history from the arenas and the batch's own rows from k_cur / v_cur[n_tokens][n_head_kv]
 * [head_dim] in fp32; query head h uses KV head h / (n_head / n_head_kv);
 * out[i][h][:] = softmax_t(scale * q . k_t) . v_t, written as [n_tokens][n_head][head_dim].
 * head_dim 64, 128 or 256; n_head a multiple of n_head_kv; n_tokens <= 65535. The workspace
 * holds per-split partial results (dcq_kv_attention_workspace_size; 0 needs none). */
size_t dcq_kv_attention_workspace_size(int n_head, int n_head_kv, int head_dim, int64_t n_tokens, int64_t n_past);
int dcq_kv_attention(int cache_type, const void* k_arena, const void* v_arena, int64_t n_blocks, int n_layer,
                     int layer, const int32_t* block_table, int64_t n_table, int n_head, int n_head_kv,
                     int head_dim, const float* q, size_t q_stride_bytes, const float* k_cur, const float* v_cur,
                     size_t kv_stride_bytes, int64_t n_tokens, int64_t n_past, float scale, float* out,
                     size_t out_stride_bytes, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DCQ_H */
