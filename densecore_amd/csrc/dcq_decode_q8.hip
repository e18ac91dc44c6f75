// dcq_decode_q8.hip — decode GEMV (M <= 8 per launch) for Q8_0 and Q4_0 weights with the
// activation's Q8_0 quantization fused in (one launch per decode step, no workspace).
//
// Replaces cb_gemv_custom's quantize-once-then-vec_dot-per-row (core/src/inference.cpp:
// 887-923) for Q8_0 weights (vec_dot_type Q8_0, core/src/inference.cpp:970-984) and ggml's
// CPU MUL_MAT at small M (core/src/inference.cpp:1063; executed at core/src/worker.cpp:544).
//
// Launch shape. A workgroup of NW waves owns NW * 64/G weight rows; G lanes stream a row,
// lane g holding the block pairs u = g + G*t, t < NS (68 bytes: two 34-byte blocks, dword
// aligned because K % 64 == 0 and the row stride is a multiple of 4; Q4_0: 36 bytes, two
// 18-byte blocks, their nibbles turned into signed q - 8 bytes as they are used; row-split Q8_0:
// the pair's 64 quants from the row's quants plane and its two scales from its scales plane).
// Every weight load of a lane is issued right after the activation loads, before any arithmetic.
//
// Activation. Each workgroup quantizes the M fp32 rows into LDS: 8 lanes per 32-element
// block, 4 floats per lane, the block's max |x| over the 8 lanes by DPP. The arithmetic is
// the standalone quantizer's (ggml-cpu x86 quantize_row_q8_0): d = amax/127 stored as fp16,
// id = amax ? 127/amax : 0, q = round-half-even(fl(x*id)) — the rounding done by adding
// 1.5*2^23 (exact for |x*id| <= 2^22; here |x*id| <= 127), so bytes and scales are
// bit-identical to dcq_quantize_rows.
// LDS: qs int8 [MT][K], then dA fp32 [MT][K/32] (the fp16 scale widened).
//
// Dot. Per block b, I_b = sum_k qw*qa exactly (8 v_dot4, int32), and
//   y += I_b * (dW_b * dA_b)          (vec_dot_q8_0_q8_0's per-block form)
// two blocks per lane per step; the G lanes of a row are reduced once at the end.
#include "dcq_common.h"
#include "dcq_kernels.h"

#include <stdlib.h>

namespace dcq {

namespace {

// max over the 8 lanes 8k .. 8k+7: quad swaps, then the half-row mirror
__device__ __forceinline__ float row8_max(float v) {
    v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
    return v;
}

// 68 bytes (two 34-byte blocks) at a dword aligned address into 17 dwords
__device__ __forceinline__ void load_pair(const uint8_t* p, uint32_t (&r)[17]) {
    const U32x4 a = ld4(p), b = ld4(p + 16), c = ld4(p + 32), d = ld4(p + 48);
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
    r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
    r[8] = c.x; r[9] = c.y; r[10] = c.z; r[11] = c.w;
    r[12] = d.x; r[13] = d.y; r[14] = d.z; r[15] = d.w;
    r[16] = ld1(p + 64);
}

// a row-split pair u (two 32-blocks): the 64 quants at row + 64u (16-byte aligned) into r[0..15],
// the two fp16 scales at row + K + 4u into r[16]
__device__ __forceinline__ void load_pair_rs(const uint8_t* row, int u, int K, uint32_t (&r)[17]) {
    const uint8_t* p = row + (int64_t)u * 64;
    const U32x4 a = ld4(p), b = ld4(p + 16), c = ld4(p + 32), d = ld4(p + 48);
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
    r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
    r[8] = c.x; r[9] = c.y; r[10] = c.z; r[11] = c.w;
    r[12] = d.x; r[13] = d.y; r[14] = d.z; r[15] = d.w;
    r[16] = ld1(row + K + (int64_t)u * 4);
}

// 36 bytes (two 18-byte Q4_0 blocks) at a dword aligned address into 9 dwords
__device__ __forceinline__ void load_pair(const uint8_t* p, uint32_t (&r)[9]) {
    const U32x4 a = ld4(p), b = ld4(p + 16);
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
    r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
    r[8] = ld1(p + 32);
}

// exact int32 sums of a block pair (w: 17 dwords, block 0's bytes start at byte 2, block 1's at
// byte 36) against 64 activation bytes
__device__ __forceinline__ void pair_sums(const uint32_t* w, uint4 a0, uint4 a1, uint4 a2, uint4 a3, int& i0,
                                          int& i1) {
    i0 = sdot4((int)align_bytes(w[1], w[0], 2), (int)a0.x, 0);
    i0 = sdot4((int)align_bytes(w[2], w[1], 2), (int)a0.y, i0);
    i0 = sdot4((int)align_bytes(w[3], w[2], 2), (int)a0.z, i0);
    i0 = sdot4((int)align_bytes(w[4], w[3], 2), (int)a0.w, i0);
    i0 = sdot4((int)align_bytes(w[5], w[4], 2), (int)a1.x, i0);
    i0 = sdot4((int)align_bytes(w[6], w[5], 2), (int)a1.y, i0);
    i0 = sdot4((int)align_bytes(w[7], w[6], 2), (int)a1.z, i0);
    i0 = sdot4((int)align_bytes(w[8], w[7], 2), (int)a1.w, i0);
    i1 = sdot4((int)w[9], (int)a2.x, 0);
    i1 = sdot4((int)w[10], (int)a2.y, i1);
    i1 = sdot4((int)w[11], (int)a2.z, i1);
    i1 = sdot4((int)w[12], (int)a2.w, i1);
    i1 = sdot4((int)w[13], (int)a3.x, i1);
    i1 = sdot4((int)w[14], (int)a3.y, i1);
    i1 = sdot4((int)w[15], (int)a3.z, i1);
    i1 = sdot4((int)w[16], (int)a3.w, i1);
}
// the pair's exact sums and its two weight scales, Q8_0 (17 dwords) or Q4_0 (9 dwords)
__device__ __forceinline__ void pair_terms(const uint32_t (&w)[17], uint4 a0, uint4 a1, uint4 a2, uint4 a3, int& i0,
                                           int& i1, float& dW0, float& dW1) {
    pair_sums(w, a0, a1, a2, a3, i0, i1);
    dW0 = half_bits_to_float(w[0] & 0xFFFFu);
    dW1 = half_bits_to_float(w[8] >> 16);
}
__device__ __forceinline__ void pair_terms(const uint32_t (&w)[9], uint4 a0, uint4 a1, uint4 a2, uint4 a3, int& i0,
                                           int& i1, float& dW0, float& dW1) {
    q4_0_pair(w, a0, a1, a2, a3, i0, i1, dW0, dW1);
}
// row-split pair (load_pair_rs): the quants need no re-slicing
__device__ __forceinline__ void pair_terms_rs(const uint32_t (&w)[17], uint4 a0, uint4 a1, uint4 a2, uint4 a3, int& i0,
                                              int& i1, float& dW0, float& dW1) {
    i0 = sdot4((int)w[0], (int)a0.x, 0);
    i0 = sdot4((int)w[1], (int)a0.y, i0);
    i0 = sdot4((int)w[2], (int)a0.z, i0);
    i0 = sdot4((int)w[3], (int)a0.w, i0);
    i0 = sdot4((int)w[4], (int)a1.x, i0);
    i0 = sdot4((int)w[5], (int)a1.y, i0);
    i0 = sdot4((int)w[6], (int)a1.z, i0);
    i0 = sdot4((int)w[7], (int)a1.w, i0);
    i1 = sdot4((int)w[8], (int)a2.x, 0);
    i1 = sdot4((int)w[9], (int)a2.y, i1);
    i1 = sdot4((int)w[10], (int)a2.z, i1);
    i1 = sdot4((int)w[11], (int)a2.w, i1);
    i1 = sdot4((int)w[12], (int)a3.x, i1);
    i1 = sdot4((int)w[13], (int)a3.y, i1);
    i1 = sdot4((int)w[14], (int)a3.z, i1);
    i1 = sdot4((int)w[15], (int)a3.w, i1);
    dW0 = half_bits_to_float(w[16] & 0xFFFFu);
    dW1 = half_bits_to_float(w[16] >> 16);
}

constexpr int kMaxStagePasses = 8;  // float4 registers of activation per thread

// (block, activation row) items staged per workgroup pass: 8 lanes each
__host__ __device__ constexpr int q8_stage_passes(int G, int NS, int MT, int NW) {
    return (MT * 2 * G * NS + 8 * NW - 1) / (8 * NW);
}


}  // namespace

// GLU: a second weight matrix W2 shares the activation; the output is silu(W x) * (W2 x).
// The arguments the first loads need come first: the first 56 bytes of arguments are preloaded
// into scalar registers at dispatch (-amdgpu-kernarg-preload-count), the rest take a dependent
// scalar load.
// FMT: Q8_0 (68-byte block pairs), Q4_0 (36-byte pairs) or row-split Q8_0 (64 quant bytes and 4 scale
// bytes from the row's two planes).
template <int G, int NS, int MT, int NW, bool DUMP, bool GLU = false, int FMT = kFmtQ8_0,
          int QC = q8_stage_passes(G, NS, MT, NW)>
__global__ void __launch_bounds__(64 * NW) decode_q8_0_kernel(const float* __restrict__ X, int64_t x_stride,
                                                           const uint8_t* __restrict__ W,
                                                           const uint8_t* __restrict__ W2, int64_t w_row_bytes,
                                                           int64_t N, int K, int M, float* Y,  // R may alias Y
                                                           int64_t y_stride, int32_t* __restrict__ sums,
                                                           int64_t sums_n_stride, const float* R, int64_t r_stride) {
    constexpr bool Q40 = FMT == kFmtQ4_0, RS = FMT == kFmtQ8_0RS;
    if constexpr (QC <= kMaxStagePasses) {
        extern __shared__ __align__(16) uint8_t smem[];
        constexpr int RPW = 64 / G;  // rows per wave
        const int nb = K / 32, U = K / 64;
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        int8_t* act_qs = reinterpret_cast<int8_t*>(smem);
        float* act_d = reinterpret_cast<float*>(smem + (size_t)MT * K);
        const int last_item = nb * MT - 1;

        // ---- 1. activation loads, issued first ----
        float4 xv[QC];
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            int it = (tid >> 3) + 8 * NW * i;
            it = it < last_item ? it : last_item;
            const int b = it / MT, m = it % MT;  // MT is a power of two
            xv[i] = *reinterpret_cast<const float4*>(X + (int64_t)(m < M ? m : M - 1) * x_stride + 32 * b +
                                                     4 * (tid & 7));
        }
        // loads retire in order: the staging below then waits for the activation only
        __builtin_amdgcn_sched_barrier(0);

        // ---- 2. every weight load of this lane ----
        const int64_t row = ((int64_t)blockIdx.x * NW + wave) * RPW + lane / G;
        const bool row_ok = row < N;
        const uint8_t* wrow = W + (row_ok ? row : N - 1) * w_row_bytes;
        const int g = lane % G;
        constexpr int kPairDw = Q40 ? 9 : 17, kPairBytes = 4 * kPairDw;
        uint32_t raw[NS][kPairDw], raw2[GLU ? NS : 1][kPairDw];
#pragma clang loop unroll(full)
        for (int t = 0; t < NS; ++t) {
            int u = g + G * t;
            u = u < U ? u : U - 1;
            if constexpr (RS)
                load_pair_rs(wrow, u, K, raw[t]);
            else
                load_pair(wrow + (int64_t)u * kPairBytes, raw[t]);
        }
        if constexpr (GLU) {
            const uint8_t* wrow2 = W2 + (row_ok ? row : N - 1) * w_row_bytes;
#pragma clang loop unroll(full)
            for (int t = 0; t < NS; ++t) {
                int u = g + G * t;
                u = u < U ? u : U - 1;
                if constexpr (RS)
                    load_pair_rs(wrow2, u, K, raw2[t]);
                else
                    load_pair(wrow2 + (int64_t)u * kPairBytes, raw2[t]);
            }
        }
        // keep the quantizer's first use of the activation (and its wait) behind the weight loads
        __builtin_amdgcn_sched_barrier(0);

        // ---- 3. quantize the activation into LDS ----
        {
#pragma clang fp contract(off)
#pragma unroll
            for (int i = 0; i < QC; ++i) {
                int it = (tid >> 3) + 8 * NW * i;
                it = it < last_item ? it : last_item;
                const int b = it / MT, m = it % MT;
                const float4 v = xv[i];
                const float amax =
                    row8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
                const float dA = half_bits_to_float(float_to_half_bits(amax / 127.f));
                const float id = amax != 0.0f ? 127.f / amax : 0.0f;
                // |x*id| <= 127: fl(x*id) + 1.5*2^23 is the half-even integer in the low byte
                const uint32_t u0 = __float_as_uint(v.x * id + 12582912.0f);
                const uint32_t u1 = __float_as_uint(v.y * id + 12582912.0f);
                const uint32_t u2 = __float_as_uint(v.z * id + 12582912.0f);
                const uint32_t u3 = __float_as_uint(v.w * id + 12582912.0f);
                // items past the end rewrite the last item with the values it already holds
                *reinterpret_cast<uint32_t*>(act_qs + m * K + 32 * b + 4 * (tid & 7)) = pack_low_bytes(u0, u1, u2, u3);
                if ((tid & 7) == 0) act_d[m * nb + b] = dA;
            }
        }
        __syncthreads();

        // ---- 4. exact block sums, one fp32 update per block ----
        float acc[MT], acc2[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) acc[mi] = acc2[mi] = 0.0f;
#pragma clang loop unroll(full)
        for (int t = 0; t < NS; ++t) {
            const int u_raw = g + G * t;
            const bool valid = u_raw < U;
            const int u = valid ? u_raw : U - 1;
            // all MT rows, also those >= M (never stored): a guard would let the compiler merge
            // the unrolled steps into one select-fed block
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                const int8_t* aq = act_qs + mi * K + 64 * u;
                const uint4 a0 = *reinterpret_cast<const uint4*>(aq);
                const uint4 a1 = *reinterpret_cast<const uint4*>(aq + 16);
                const uint4 a2 = *reinterpret_cast<const uint4*>(aq + 32);
                const uint4 a3 = *reinterpret_cast<const uint4*>(aq + 48);
                const float2 dA = *reinterpret_cast<const float2*>(act_d + mi * nb + 2 * u);
                int i0, i1;
                float dW0, dW1;
                if constexpr (RS)
                    pair_terms_rs(raw[t], a0, a1, a2, a3, i0, i1, dW0, dW1);
                else
                    pair_terms(raw[t], a0, a1, a2, a3, i0, i1, dW0, dW1);
                if (DUMP && valid && row_ok && mi < M) {
                    int32_t* srow = sums + ((int64_t)mi * sums_n_stride + row) * nb;
                    atomicAdd(srow + 2 * u, i0);
                    atomicAdd(srow + 2 * u + 1, i1);
                }
                const float v = fmaf((float)i1, dW1 * dA.y, (float)i0 * (dW0 * dA.x));
                acc[mi] = valid ? acc[mi] + v : acc[mi];
                if constexpr (GLU) {
                    int j0, j1;
                    float eW0, eW1;
                    if constexpr (RS)
                        pair_terms_rs(raw2[t], a0, a1, a2, a3, j0, j1, eW0, eW1);
                    else
                        pair_terms(raw2[t], a0, a1, a2, a3, j0, j1, eW0, eW1);
                    const float v2 = fmaf((float)j1, eW1 * dA.y, (float)j0 * (eW0 * dA.x));
                    acc2[mi] = valid ? acc2[mi] + v2 : acc2[mi];
                }
            }
        }
        // ---- 5. reduce the G lanes of each row ----
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            acc[mi] = lanes_sum<G>(acc[mi]);
            if constexpr (GLU) acc[mi] = silu(acc[mi]) * lanes_sum<G>(acc2[mi]);
        }
        if (g == 0 && row_ok) {
#pragma unroll
            for (int mi = 0; mi < MT; ++mi)
                if (mi < M)  // R (optional, may alias Y): Y = W x + R
                    Y[(int64_t)mi * y_stride + row] = R ? acc[mi] + R[(int64_t)mi * r_stride + row] : acc[mi];
        }
    }
}

namespace {

using DecodeQ8Fn = void (*)(const float*, int64_t, const uint8_t*, const uint8_t*, int64_t, int64_t, int, int,
                            float*, int64_t, int32_t*, int64_t, const float*, int64_t);

// (G lanes per row, NS pairs per lane): a row of U = K/64 pairs needs G*NS >= U
struct Q8Shape {
    int G, NS;
};
constexpr Q8Shape kQ8Shapes[] = {{16, 1}, {8, 2}, {32, 1}, {16, 2}, {64, 1}, {32, 2},
                                 {16, 4}, {64, 2}, {32, 4}, {64, 4}, {16, 3}, {32, 3}};
constexpr int kNumQ8Shapes = sizeof(kQ8Shapes) / sizeof(kQ8Shapes[0]);
static_assert(kNumQ8Shapes == 12, "pick_q8_shape covers every shape");

#ifndef DCQ_Q8_NW
#define DCQ_Q8_NW 4
#endif
constexpr int kQ8Waves = DCQ_Q8_NW;

template <int I, int MT, bool DUMP, bool GLU, int FMT>
DecodeQ8Fn q8_fn() {
    return decode_q8_0_kernel<kQ8Shapes[I].G, kQ8Shapes[I].NS, MT, kQ8Waves, DUMP, GLU, FMT>;
}
template <int I, bool DUMP, bool GLU, int FMT>
DecodeQ8Fn q8_pick_mt(int mt) {
    switch (mt) {
        case 1: return q8_fn<I, 1, DUMP, GLU, FMT>();
        case 2: return q8_fn<I, 2, DUMP, GLU, FMT>();
        case 4: return q8_fn<I, 4, DUMP, GLU, FMT>();
        default: return q8_fn<I, 8, DUMP, GLU, FMT>();
    }
}
template <bool DUMP, bool GLU, int FMT>
DecodeQ8Fn q8_pick_shape(int idx, int mt) {
    switch (idx) {
        case 0: return q8_pick_mt<0, DUMP, GLU, FMT>(mt);
        case 1: return q8_pick_mt<1, DUMP, GLU, FMT>(mt);
        case 2: return q8_pick_mt<2, DUMP, GLU, FMT>(mt);
        case 3: return q8_pick_mt<3, DUMP, GLU, FMT>(mt);
        case 4: return q8_pick_mt<4, DUMP, GLU, FMT>(mt);
        case 5: return q8_pick_mt<5, DUMP, GLU, FMT>(mt);
        case 6: return q8_pick_mt<6, DUMP, GLU, FMT>(mt);
        case 7: return q8_pick_mt<7, DUMP, GLU, FMT>(mt);
        case 8: return q8_pick_mt<8, DUMP, GLU, FMT>(mt);
        case 9: return q8_pick_mt<9, DUMP, GLU, FMT>(mt);
        case 10: return q8_pick_mt<10, DUMP, GLU, FMT>(mt);
        default: return q8_pick_mt<11, DUMP, GLU, FMT>(mt);
    }
}
template <int FMT>
DecodeQ8Fn q8_pick(bool glu, bool dump, int idx, int mt) {
    if constexpr (FMT == kFmtQ8_0RS) {
        // the gate/up pair takes GGUF rows only
        return dump ? q8_pick_shape<true, false, FMT>(idx, mt) : q8_pick_shape<false, false, FMT>(idx, mt);
    } else {
        return glu ? q8_pick_shape<false, true, FMT>(idx, mt)
                   : (dump ? q8_pick_shape<true, false, FMT>(idx, mt) : q8_pick_shape<false, false, FMT>(idx, mt));
    }
}

// The shape for U pairs per row. Measured on MI355X (fused, M = 1, W rotated over 1 GiB; us):
//   Q8_0  9728 x 2560: {32,2} 6.47  {16,3} 6.88  {64,1} 8.19     4096 x 4096: {32,2} 5.00  {64,1} 5.34
//        13824 x 5120: {32,3} 15.75 {64,2} 20.31                 2048 x 8192: {64,2} 5.39  {32,4} 5.80
//   Q4_0  9728 x 2560: {16,3} 5.17  {16,4} 5.74  {32,2} 5.86  {64,1} 7.44
//         8192 x 3072: {16,3} 4.61  {16,4} 5.12  {32,2} 5.37   2048 x 8192: {32,4} 4.30  {64,2} 4.71
// Rows of at most 32 lanes win, with a lane's weight bytes in flight up to about 140 (Q8_0: 2
// pairs of 68 B, then 3; Q4_0: 4 pairs of 36 B): within those limits the shape with the fewest idle
// pair slots, then the fewest steps. Past them (long rows), the fewest steps whose idle slots stay
// within a quarter, then any shape that fits. DCQ_Q8_SHAPE=<index> forces one (tuning).
int choose_q8_shape(int U, bool q40) {
    const int forced = knob(Knob::Q8Shape);
    if (forced >= 0 && forced < kNumQ8Shapes && kQ8Shapes[forced].G * kQ8Shapes[forced].NS >= U) return forced;
    const int tiers = q40 ? 1 : 2;
    for (int t = 0; t < tiers; ++t) {
        const int ns_max = q40 ? 4 : 2 + t;
        int best = -1, best_waste = 1 << 30, best_ns = 1 << 30;
        for (int i = 0; i < kNumQ8Shapes; ++i) {
            const int cap = kQ8Shapes[i].G * kQ8Shapes[i].NS;
            if (cap < U || kQ8Shapes[i].G > 32 || kQ8Shapes[i].NS > ns_max) continue;
            const int waste = cap - U;
            if (waste < best_waste || (waste == best_waste && kQ8Shapes[i].NS < best_ns)) {
                best = i;
                best_waste = waste;
                best_ns = kQ8Shapes[i].NS;
            }
        }
        if (best >= 0) return best;
    }
    int best = -1;
    for (int pass = 0; pass < 2 && best < 0; ++pass) {
        int best_ns = 1 << 30, best_waste = 1 << 30;
        for (int i = 0; i < kNumQ8Shapes; ++i) {
            const int cap = kQ8Shapes[i].G * kQ8Shapes[i].NS;
            if (cap < U) continue;
            const int waste = cap - U;
            if (pass == 0 && 4 * waste > cap) continue;
            if (kQ8Shapes[i].NS < best_ns || (kQ8Shapes[i].NS == best_ns && waste < best_waste)) {
                best = i;
                best_ns = kQ8Shapes[i].NS;
                best_waste = waste;
            }
        }
    }
    return best;
}

}  // namespace

namespace {

// W2 != nullptr: the gate/up pair (no block sums), Y = silu(W x) * (W2 x). q40: Q4_0 weights.
hipError_t launch_q8(int fmt, const void* W, const void* W2, int64_t w_row_bytes, int64_t N, int64_t K,
                     const float* X, int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                     hipStream_t st, const float* R = nullptr, int64_t r_stride = 0) {
    if (K % 64 != 0 || w_row_bytes % 4 != 0 || x_stride % 4 != 0) return hipErrorNotSupported;
    if (W2 && (block_sums || fmt == kFmtQ8_0RS)) return hipErrorNotSupported;
    if (fmt == kFmtQ8_0RS && w_row_bytes % 16 != 0) return hipErrorNotSupported;
    const int U = (int)(K / 64);
    const int idx = choose_q8_shape(U, fmt == kFmtQ4_0);
    if (idx < 0) return hipErrorNotSupported;
    const int G = kQ8Shapes[idx].G, NS = kQ8Shapes[idx].NS;
    // validate every M tile before launching anything
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        if (q8_stage_passes(G, NS, mt, kQ8Waves) > kMaxStagePasses) return hipErrorNotSupported;
        if ((size_t)mt * K * 9 / 8 > 64 * 1024) return hipErrorNotSupported;
    }
    const int rows_per_block = kQ8Waves * (64 / G);
    const unsigned grid = (unsigned)((N + rows_per_block - 1) / rows_per_block);
    const int64_t per_row_sums = K / 32;
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const size_t lds = (size_t)mt * K * 9 / 8;
        const bool glu = W2 != nullptr, dump = block_sums != nullptr;
        DecodeQ8Fn fn = fmt == kFmtQ4_0     ? q8_pick<kFmtQ4_0>(glu, dump, idx, mt)
                        : fmt == kFmtQ8_0RS ? q8_pick<kFmtQ8_0RS>(glu, dump, idx, mt)
                                            : q8_pick<kFmtQ8_0>(glu, dump, idx, mt);
        hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * kQ8Waves), lds, st, X + m0 * x_stride, x_stride,
                           (const uint8_t*)W, (const uint8_t*)W2, w_row_bytes, N, (int)K, (int)mc, Y + m0 * y_stride,
                           y_stride,
                           block_sums ? block_sums + m0 * N * per_row_sums : nullptr, N,
                           R ? R + m0 * r_stride : nullptr, r_stride);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_fused_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                                    const float* X, int64_t x_stride, int64_t M, float* Y, int64_t y_stride,
                                    int32_t* block_sums, hipStream_t st, const float* R, int64_t r_stride) {
    return launch_q8(fmt, W, nullptr, w_row_bytes, N, K, X, x_stride, M, Y, y_stride, block_sums, st, R, r_stride);
}

hipError_t launch_decode_fused_q8_0_glu(int fmt, const void* Wg, const void* Wu, int64_t w_row_bytes, int64_t N,
                                        int64_t K, const float* X, int64_t x_stride, int64_t M, float* Y,
                                        int64_t y_stride, hipStream_t st) {
    return launch_q8(fmt, Wg, Wu, w_row_bytes, N, K, X, x_stride, M, Y, y_stride, nullptr, st);
}

}  // namespace dcq
