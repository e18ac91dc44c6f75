// dcq_kernels.h — internal launcher declarations shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dcq_common.h"

namespace dcq {

// Weight formats of the Q8_0-block kernels: GGUF Q8_0 and Q4_0 rows, and row-split Q8_0
// (kTypeQ8_0_RS).
enum Q8Fmt { kFmtQ8_0 = 0, kFmtQ4_0 = 1, kFmtQ8_0RS = 2 };
inline int q8_fmt(int wtype) { return wtype == kTypeQ4_0 ? kFmtQ4_0 : wtype == kTypeQ8_0_RS ? kFmtQ8_0RS : kFmtQ8_0; }

// Planar quantized activations inside a workspace (see dcq_common.h for the layout).
struct PlanarBuffers {
    int8_t* qs;   // [M][K]
    float* d;     // [K/bs][m_ld]
    int16_t* bs;  // [M][K/16] (Q8_K) or nullptr
    int64_t m_ld;
};

// Workspace carve-up for `vdt` activations of M x K; returns total bytes (256-B granules).
size_t planar_bytes(int vdt, int64_t M, int64_t K, PlanarBuffers* pb, void* base);

hipError_t launch_quantize_ggml(int vdt, const float* X, int64_t x_stride, int64_t M, int64_t K, void* out,
                                int64_t out_row_bytes, hipStream_t st);
hipError_t launch_quantize_planar(int vdt, const float* X, int64_t x_stride, int64_t M, int64_t K,
                                  const PlanarBuffers& pb, hipStream_t st);
hipError_t launch_unpack_ggml_rows(int vdt, const void* in, int64_t in_row_bytes, int64_t M, int64_t K,
                                   const PlanarBuffers& pb, hipStream_t st);

// Decode GEMV / small-M: wave-per-row-group int8 dot products.
// Y[m*y_stride + n] for m < M, n in [n0, n1); block_sums optional (atomics, pre-zeroed).
// R (optional, indexed like Y, may be Y itself): Y = W x + R, added in the store of the
// LDS-staged Q4_K / Q5_K / Q6_K kernels; with R given and neither covering the shape, nothing is
// launched and the result is hipErrorNotSupported.
// compute units of the current device (cached per device)
int cu_count();

// Tuning overrides for measurements. The default build has a fixed dispatch rule: knob() is a
// constant that returns each knob's default (the measured choice), and the launchers' override
// branches fold away. Only a tuning build (make TUNING=1, which defines DCQ_TUNING) reads the
// DCQ_* variables below from the environment, once per process; -1 or 0 means "not set".
enum class Knob {
    Q4KShape,     // DCQ_Q4K_SHAPE: force a decode shape index (-1: launch rule)
    Q4KWaves,     // DCQ_Q4K_NW: 5 for 5-wave workgroups with a forced shape (default 4)
    NoFuse,       // DCQ_NO_FUSE: 1 disables the fused-activation decode kernels
    Q6KDecode,    // DCQ_Q6K_DECODE: 1 selects the lane-direct Q6_K decode kernel
    Q6KLdsOff,    // DCQ_Q6K_LDS_OFF: 1 disables the LDS-staged Q6_K kernels
    Q6KNoFuse,    // DCQ_Q6K_NO_FUSE: 1 disables the fused Q6_K decode
    Q6KFuseWaves, // DCQ_Q6K_FUSE_NW: force the fused Q6_K workgroup width (4, 8, 10, 12)
    Q8Shape,      // DCQ_Q8_SHAPE: force a Q8_0 / Q4_0 decode shape index (-1: launch rule)
    GemvGeneric,  // DCQ_GEMV_GENERIC: 1 forces the generic GEMV kernel
    GemvLanes,    // DCQ_GEMV_LG: log2 lanes per row of the generic GEMV (-1: rule)
    AttnNoMfma,   // DCQ_ATTN_NO_MFMA: 1 keeps prompts on the VALU attention kernel
    Q6KRows,      // DCQ_Q6K_RPW: rows per wave of the 4-wave Q6_K decode (-1: launch rule)
    Q6KMfma,      // DCQ_Q6K_MFMA: 0 keeps tall Q6_K matrices on the lane-per-superblock kernels
    SplitK,       // DCQ_SPLIT_K: force the K splits of the MFMA prefill kernels (-1: rule, 1: none)
    BatchTile,    // DCQ_BATCH_MTI: force the Q4_K batch kernel's 32-row m-tiles per workgroup (1 or 2)
    kCount
};
// defaults, in Knob order: the launchers' measured rules
constexpr int kKnobDefault[(int)Knob::kCount] = {-1, 4, 0, 0, 0, 0, -1, -1, 0, -1, 0, -1, 1, -1, -1};
#ifdef DCQ_TUNING
int knob(Knob k);
#else
constexpr int knob(Knob k) { return kKnobDefault[(int)k]; }
#endif

hipError_t launch_gemv(int wtype, const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                       const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                       int64_t sums_n_stride, hipStream_t st, const float* R = nullptr, int64_t r_stride = 0);

// LDS-staged decode kernels (M <= 8 per launch, tiled by 8). hipErrorNotSupported means the
// shape is outside what they cover and nothing was launched.
hipError_t launch_decode_kq(int wtype, const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                            const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                            int64_t sums_n_stride, hipStream_t st, const float* R = nullptr, int64_t r_stride = 0);

// SwiGLU gate/up pair at M <= 8 with the activation quantization fused in (Q4_K, Q5_K, Q8_0, Q4_0):
// Y = silu(Wg x) * (Wu x); hipErrorNotSupported when the fused kernels do not cover the shape.
hipError_t launch_decode_fused_glu(int wtype, const void* Wg, const void* Wu, int64_t w_row_bytes, int64_t N, int64_t K,
                                   const float* X, int64_t x_stride, int64_t M, float* Y, int64_t y_stride,
                                   hipStream_t st);
hipError_t launch_decode_fused_q8_0_glu(int fmt, const void* Wg, const void* Wu, int64_t w_row_bytes, int64_t N,
                                        int64_t K, const float* X, int64_t x_stride, int64_t M, float* Y,
                                        int64_t y_stride, hipStream_t st);
// Y[m][n] = silu(Y[m][n]) * U[m][n] (the SwiGLU product after two separate projections)
hipError_t launch_silu_mul(float* Y, int64_t y_stride, const float* U, int64_t u_stride, int64_t M, int64_t N,
                           hipStream_t st);
hipError_t launch_add_rows(float* Y, int64_t y_stride, const float* T, int64_t t_stride, const float* R,
                           int64_t r_stride, int64_t M, int64_t N, hipStream_t st);

// Q6_K decode with the weight rows staged in LDS by direct-to-LDS loads (K/256 even,
// w_row_bytes % 4 == 0); hipErrorNotSupported otherwise (nothing launched).
// Q6_K decode with the Q8_K activation quantization fused in (M <= 2, K % 512 == 0,
// K <= 16384, row stride a multiple of 4 bytes); hipErrorNotSupported otherwise.
hipError_t launch_decode_fused_q6k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const float* X,
                                   int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                                   hipStream_t st, const float* R = nullptr,
                                   int64_t r_stride = 0);
hipError_t launch_decode_q6k_lds(const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                                 const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                                 int64_t sums_n_stride, hipStream_t st, const float* R = nullptr,
                                 int64_t r_stride = 0);

// Decode with the activation quantization fused in (X fp32, no workspace): one launch per
// 8 rows of M. hipErrorNotSupported: the caller quantizes and uses launch_gemv.
hipError_t launch_decode_fused(int wtype, const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const float* X,
                               int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const float* R = nullptr,
                                   int64_t r_stride = 0);

// Q8_0, Q4_0 or row-split Q8_0 (fmt, a Q8Fmt) decode with the Q8_0 activation quantization fused in
// (K % 64 == 0, row stride a multiple of 4 bytes (row-split: 16), M*K*9/8 bytes of LDS per 8-row
// tile; the gate/up pair takes Q8_0 and Q4_0); hipErrorNotSupported otherwise.
hipError_t launch_decode_fused_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                                    const float* X, int64_t x_stride, int64_t M, float* Y, int64_t y_stride,
                                    int32_t* block_sums, hipStream_t st, const float* R = nullptr,
                                    int64_t r_stride = 0);

// Room for the partial tiles of a split-K product (fp32 planes of M x N); bytes == 0: no split.
struct SplitScratch {
    float* p = nullptr;
    size_t bytes = 0;
};

// Split-K for the 128 x 128-tile MFMA kernels when their tiles cannot fill the chip: the K stages
// are cut into `splits` ranges of `stps` stages (a multiple of `align`), each a workgroup per
// tile writing its partial tile to a plane of the scratch; then launch_sum_splits adds the planes
// in split order (deterministic). splits == 1: no split (stps = nstages).
struct SplitPlan {
    int splits, stps;
};
// us_per_stage: the estimated time of one stage of one workgroup (the cost model's unit)
SplitPlan plan_split_k(int64_t tiles, int nstages, int align, int64_t M, int64_t N, const SplitScratch& sc,
                       double us_per_stage = 2.0);
// Y[m][n] = sum over s (in order) of P[s][m][n], P planes of M x N floats.
hipError_t launch_sum_splits(const float* P, int splits, int64_t M, int64_t N, float* Y, int64_t y_stride,
                             hipStream_t st);

// Q8_0 / Q4_0 / row-split Q8_0 (fmt) prefill: LDS-staged 128 x 128 int8-MFMA tiles (K % 128 == 0,
// w_row_bytes % 4 == 0; row-split: % 16 == 0 and N * w_row_bytes < 4 GiB); hipErrorNotSupported
// otherwise (nothing launched).
hipError_t launch_prefill_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                               const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const SplitScratch& sc = SplitScratch());

// Q6_K prefill: the same tiling over the planar Q8_K activation (K % 512 == 0, w_row_bytes % 4
// == 0, m_ld % 128 == 0); hipErrorNotSupported otherwise (nothing launched).
hipError_t launch_prefill_q6_k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                               int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                               const SplitScratch& sc = SplitScratch());
// Q4_K (q5: Q5_K) prefill: the same tiling (K % 256 == 0, w_row_bytes % 16 == 0, m_ld % 128 == 0).
hipError_t launch_prefill_q4_k(bool q5, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                               const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const SplitScratch& sc = SplitScratch());

// Q4_K (q5: Q5_K) batched decode (M <= 128): 8-wave workgroups per 32 weight rows x 64 activation
// rows, K split over the waves (and over workgroups when the rows are few and sc has room);
// hipErrorNotSupported when the shape is outside it.
hipError_t launch_batch_q4k(bool q5, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                            const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                            hipStream_t st, const SplitScratch& sc = SplitScratch());

// Q8_0 / Q4_0 / row-split Q8_0 (fmt) batched decode (4 < M <= 64): 8-wave workgroups per 32 weight
// rows x 32 or 64 activation rows, K split over the waves (and over workgroups when the rows are few
// and sc has room); hipErrorNotSupported when the shape is outside it.
hipError_t launch_batch_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                             const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                             hipStream_t st, const SplitScratch& sc);

// Q6_K batched decode (4 < M <= 64, K % 512 == 0): the same launch shape, one int8 MFMA per
// 16-element scale group; hipErrorNotSupported when the shape is outside it.
hipError_t launch_batch_q6k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                            int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                            const SplitScratch& sc);

// Int8-MFMA tiles for any M; sc: room for split-K partial tiles (optional).
hipError_t launch_mmq(int wtype, const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                      int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                      const SplitScratch& sc = SplitScratch());

// Paged KV cache (arena layout of the reference's PagedKVCache; row_elems % 32 == 0, pointers
// and strides 16-byte aligned, checked by the caller).
hipError_t launch_kv_write(int ct, void* arena, int n_blocks, int n_layer, int layer, int64_t row_elems, int64_t sb,
                           const int32_t* table, int pos0, const float* src, int64_t src_stride, int n_tokens,
                           hipStream_t st);
hipError_t launch_kv_gather(int ct, const void* arena, int n_blocks, int n_layer, int layer, int64_t row_elems,
                            int64_t sb, const int32_t* table, int n_table, int n_past, const float* cur,
                            int64_t cur_stride, int n_tokens, float* dst, int64_t dst_stride, hipStream_t st);
// Attention over the arena (head_dim 64/128/256); workspace from attn_workspace_bytes (0 when
// the keys are not split). hipErrorNotSupported for another head_dim or cache type.
size_t attn_workspace_bytes(int hd, int n_head, int n_head_kv, int n_tokens, int n_past);
hipError_t launch_kv_attention(int ct, const void* k_arena, const void* v_arena, int n_blocks, int n_layer, int layer,
                               int64_t sb, const int32_t* table, int n_table, int n_head, int n_head_kv, int hd,
                               const float* q, int64_t q_stride, const float* k_cur, const float* v_cur,
                               int64_t kv_stride, int n_tokens, int n_past, float scale, float* out,
                               int64_t out_stride, void* ws, size_t ws_bytes, hipStream_t st);

// The current device's copy of the no-alloc scratch array (dcq_noalloc.hip): its device address,
// looked up on the device's first call, and its size. DCQ_OK, or DCQ_ERR_* if the lookup fails.
int noalloc_scratch(void** ptr, size_t* bytes);

hipError_t launch_quantize_weights(int wtype, const float* W, int64_t N, int64_t K, void* Wq, hipStream_t st);
hipError_t launch_dequantize(int type, const void* Wq, int64_t N, int64_t K, int64_t w_row_bytes, float* Y,
                             hipStream_t st);
// Q8_0 rows -> row-split rows (out rows 16-byte aligned, out_row_bytes >= 34 * K / 32)
hipError_t launch_repack_q8_0_rs(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, void* out,
                                 int64_t out_row_bytes, hipStream_t st);

}  // namespace dcq
