/*
 * dcq_oracle.h — CPU oracle for the quantized mul_mat hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline). The product library (libdcq) never links or
 * calls it.
 *
 * What it restates. DenseCore's quantized mul_mat is executed by ggml (an
 * un-vendored, unpinned submodule: /root/reference/.gitmodules:1-3). The
 * reference's own files contribute only the call sites:
 *   - quantize X once with the weight type's vec_dot_type `from_float`, then a
 *     per-row `vec_dot` (core/src/inference.cpp:887-923);
 *   - vec_dot_type mapping Q4_K/Q5_K/Q6_K -> Q8_K, Q8_0 -> Q8_0
 *     (core/include/simd_ops.h:3298-3305); Q4_0 -> Q8_0 (ggml's trait for the
 *     quantize tool's default type, core/src/quantize.cpp:71-72, 90);
 *   - row-range contract with pre-quantized input (core/src/simd_ops.cpp:140-171).
 * The arithmetic below follows ggml's published algorithms for the GGUF block
 * formats Q8_0 / Q4_0 / Q4_K / Q5_K / Q6_K / Q8_K, restated from their definitions.
 *
 * Parity pins (each function lists its own in dcq_oracle.c):
 *   - fp16 conversion: numpy float16 (IEEE RNE) on 2^20+ values and all ties.
 *   - activation quantizers: closed forms (zero block, single non-zero, ties,
 *     max |q| = 127, dequant error <= d/2, bsums invariant).
 *   - integer block sums: brute force in int64 from the dequantized integers.
 *   - fp32 vec_dot: fp64 dequantize-and-dot brute force.
 *   - weight quantizers: each sub-block fit is the result of its grid search, recomputed
 *     independently in the tests; packing inverts; final quants are nearest grid points.
 * "parity unpinned" (only an import of ggml could pin them; ggml is absent):
 *   - the exact fp32 summation order of ggml's SIMD vec_dot;
 *   - the choice between the two Q8_0 from_float variants (x86 SIMD vs ref);
 *   - the Q8_K scale constant: iscale = -127/max (ggml's quantize_row_q8_K_ref in the
 *     type-traits-cpu API era the reference's calls imply; older ggml used -128);
 *   - the constants of the Q4_K / Q5_K / Q6_K weight quantizers' grid searches, and so their bytes
 *     against a ggml build — used only to generate inputs.
 */
#ifndef DCQ_ORACLE_H
#define DCQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (GGUF spec) */
enum {
    DCQO_TYPE_F32 = 0,
    DCQO_TYPE_F16 = 1,
    DCQO_TYPE_Q4_0 = 2,
    DCQO_TYPE_Q8_0 = 8,
    DCQO_TYPE_Q4_K = 12,
    DCQO_TYPE_Q5_K = 13,
    DCQO_TYPE_Q6_K = 14,
    DCQO_TYPE_Q8_K = 15,
};

/* Q8_0 from_float variants */
enum {
    DCQO_Q8_0_X86 = 0, /* ggml-cpu x86 SIMD: d = amax/127, id = 127/amax, round-half-even */
    DCQO_Q8_0_REF = 1, /* quantize_row_q8_0_ref: id = 1/d, roundf (half away from zero) */
};

/* ---- format helpers ---- */
int64_t dcqo_block_size(int type);       /* elements per block */
int64_t dcqo_type_size(int type);        /* bytes per block */
int64_t dcqo_row_size(int type, int64_t k);
int dcqo_vec_dot_type(int type);

/* ---- fp16 ---- */
uint16_t dcqo_fp32_to_fp16(float f);
float dcqo_fp16_to_fp32(uint16_t h);
void dcqo_fp32_to_fp16_array(const float* x, uint16_t* y, int64_t n);
void dcqo_fp16_to_fp32_array(const uint16_t* x, float* y, int64_t n);

/* ---- activation quantizers (from_float) ---- */
void dcqo_quantize_row_q8_0(const float* x, void* y, int64_t k, int variant);
void dcqo_quantize_row_q8_K(const float* x, void* y, int64_t k);
/* quantize rows: X is [m][k] with row stride x_stride floats; Y rows packed */
void dcqo_quantize_rows(int vec_dot_type, const float* x, int64_t m, int64_t k, int64_t x_stride,
                        void* y, int variant);

/* ---- weight quantizers (input generation only) ---- */
void dcqo_quantize_row_q8_0_weights(const float* x, void* y, int64_t k);
void dcqo_quantize_row_q4_0(const float* x, void* y, int64_t k);
void dcqo_quantize_row_q4_K(const float* x, void* y, int64_t k);
void dcqo_quantize_row_q5_K(const float* x, void* y, int64_t k);
void dcqo_quantize_row_q6_K(const float* x, void* y, int64_t k);
/* quantize an [n][k] fp32 matrix to `type`, rows packed; nthreads <= 0 -> auto */
int dcqo_quantize_matrix(int type, const float* x, int64_t n, int64_t k, void* y, int nthreads);

/* ---- test hooks into the weight quantizers ----
 * make_qkx2_quants (Q4_K, with the arguments ggml's quantize_row_q4_K_ref passes: nmax 15,
 * rmin -1, rdelta 0.1, nstep 20) and make_qx_quants (Q6_K: nmax 32), and the Q4_K 6-bit scale/min
 * packing. flags plant a mistake on purpose (DCQO_PLANT_*), so the tests can show that their
 * optimality checks reject it; the quantizers always pass 0. */
enum {
    DCQO_PLANT_NO_MIN_CLAMP = 1,  /* make_qkx2_quants: refitted min may stay > 0 */
    DCQO_PLANT_UNIT_WEIGHTS = 2,  /* make_qx_quants: weights 1 instead of x^2 */
    DCQO_PLANT_GRID_8 = 4,        /* make_qx_quants: grid is in [-8, 8] instead of [-9, 9] */
};
float dcqo_make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L, float* the_min,
                            float rmin, float rdelta, int nstep, int flags);
float dcqo_make_qx_quants(int n, int nmax, const float* x, int8_t* L, int flags);
void dcqo_pack_scale_min_k4(const uint8_t ls[8], const uint8_t lm[8], uint8_t s[12]);

/* ---- dequantization ---- */
int dcqo_dequantize_row(int type, const void* x, float* y, int64_t k);

/* ---- dot products ---- */
/* ggml-generic order vec_dot of one weight row with a pre-quantized activation row */
float dcqo_vec_dot(int wtype, int64_t k, const void* w, const void* xq);
/* fp64 brute force of the same quantity (dequantize both, sum in double) */
double dcqo_vec_dot_f64(int wtype, int64_t k, const void* w, const void* xq);
/* L1 magnitude of the per-block terms: sum_b |scale_b * int_b| (tolerance guard) */
double dcqo_vec_dot_l1(int wtype, int64_t k, const void* w, const void* xq);
/* number of int32 block sums per row that dcqo_block_sums emits */
int64_t dcqo_block_sums_per_row(int wtype, int64_t k);
/*
 * Per-block integer sums, the exact integers each vec_dot scales:
 *   Q8_0: I_b = sum_{32} qw*qa                          (k/32 values)
 *   Q4_0: I_b = sum_{32} (qw - 8)*qa                    (k/32 values)
 *   Q4_K, Q5_K: per superblock {sum_j sc_j*I_j, sum_j m_j*S_j} (2*k/256 values)
 *   Q6_K: per superblock sum_g sc_g*I_g                  (k/256 values)
 */
int dcqo_block_sums(int wtype, int64_t k, const void* w, const void* xq, int32_t* out);
/* the same, from first principles in int64 on dequantized integer fields */
int dcqo_block_sums_bruteforce(int wtype, int64_t k, const void* w, const void* xq, int64_t* out);

/* ComputeDotProductBatch semantics: y[r - n0] = vec_dot(row r), r in [n0, n1) */
int dcqo_dot_rows(int wtype, const void* w, size_t row_stride, const void* xq, int64_t k, float* y,
                  int64_t n0, int64_t n1);

/*
 * GGML_OP_MUL_MAT semantics: quantize every X row to vec_dot_type, then
 * Y[m*y_stride + n] = vec_dot(W row n, Xq row m). Strides in elements/bytes as named.
 * Also fills l1 (same shape as Y, may be NULL) with the tolerance guard.
 */
int dcqo_mul_mat(int wtype, const void* w, int64_t n, int64_t k, size_t w_row_bytes, const float* x,
                 int64_t m, int64_t x_stride, float* y, int64_t y_stride, float* l1, int variant,
                 int nthreads);

#ifdef __cplusplus
}
#endif
#endif
