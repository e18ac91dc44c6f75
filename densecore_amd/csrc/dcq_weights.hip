// dcq_weights.hip — weight quantization (ggml_quantize_chunk without an importance
// matrix) and dequantization (type_traits->to_float).
//
// Weight quantization is the offline step before the hot path
// (core/src/quantize.cpp:214, 285 call ggml_quantize_chunk); dequantization is
// the reference GEMV's fallback (core/src/inference.cpp:938-945). The search is ggml's published
// algorithm (make_qkx2_quants for Q4_K and Q5_K, make_qx_quants with rmse_type 1 for Q6_K, roundf
// scaling for Q8_0, the max / -8 scale with truncation after + 8.5 for Q4_0), each fit's sums in
// their sequential order. Q8_0 and Q4_0 take one thread per block. The K-quants take one lane per
// independent fit: eight lanes per Q4_K / Q5_K superblock (a 32-element sub-block each), sixteen per
// Q6_K superblock (a 16-element group each), each fit on values in registers; what a superblock
// shares (its largest scale and min, Q6_K's first group of the largest |scale|, the packed scale
// bytes, bytes built from several fits' levels) comes from lane exchanges within the superblock's
// lanes. ggml's fits within a sub-block depend on each other (a better candidate moves the next
// candidates' offset), so they stay sequential in their lane. 9728 x 2560: Q4_K one thread per
// superblock with the sub-block fits in LDS 0.39 ms (2.36 ms with per-thread arrays in scratch
// memory); Q6_K one thread per superblock 0.33 ms. This file is compiled with -ffp-contract=off so
// each fp32 operation rounds on its own, as the CPU code does, and the bytes match a CPU build of
// the same algorithm exactly.
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

__device__ __forceinline__ int nearest_int(float v) {
    float t = v + 12582912.f;
    int32_t i;
    __builtin_memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

// ---- Q8_0: quantize_row_q8_0_ref (id = 1/d, roundf) ----
__global__ void __launch_bounds__(256) quantize_w_q8_0_kernel(const float* __restrict__ W, int64_t N, int64_t K,
                                                              uint8_t* __restrict__ out) {
    const int64_t nb = K / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= N * nb) return;
    const int64_t r = gid / nb, b = gid - (gid / nb) * nb;
    const float* x = W + r * K + b * QK8_0;
    float amax = 0.0f;
    for (int j = 0; j < QK8_0; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* blk = out + r * nb * 34 + b * 34;
    uint16_t* p16 = reinterpret_cast<uint16_t*>(blk);
    p16[0] = float_to_half_bits(d);
    for (int j = 0; j < QK8_0; j += 2) {
        float v0 = fminf(fmaxf(roundf(x[j] * id), -128.f), 127.f);
        float v1 = fminf(fmaxf(roundf(x[j + 1] * id), -128.f), 127.f);
        p16[1 + j / 2] = (uint16_t)(((uint32_t)(int32_t)v0 & 0xFFu) | (((uint32_t)(int32_t)v1 & 0xFFu) << 8));
    }
}

// ---- Q4_0: quantize_row_q4_0_ref (d = max / -8 for the first element of largest |x|,
// q = min(15, trunc(x / d + 8.5))) ----
__global__ void __launch_bounds__(256) quantize_w_q4_0_kernel(const float* __restrict__ W, int64_t N, int64_t K,
                                                              uint8_t* __restrict__ out) {
    const int64_t nb = K / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= N * nb) return;
    const int64_t r = gid / nb, b = gid - (gid / nb) * nb;
    const float* x = W + r * K + b * QK8_0;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < QK8_0; ++j) {
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            max = x[j];
        }
    }
    const float d = max / -8;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t* p16 = reinterpret_cast<uint16_t*>(out + r * nb * 18 + b * 18);  // blocks are 2-byte aligned
    // an all-zero block has d = 0 / -8 = -0.0, stored as fp16 -0.0 (0x8000). The compiler folds the
    // fp16 conversion of the product max * -0.125 into v_fma_mix with a +0 addend, which turns a
    // -0 product into +0, so the sign bit is taken from d itself (the product is exact, so the
    // fold changes nothing else).
    p16[0] = (uint16_t)(float_to_half_bits(d) | ((__float_as_uint(d) >> 16) & 0x8000u));
    for (int j = 0; j < QK8_0 / 2; j += 2) {
        uint32_t two = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            // the float -> int8 conversion truncates toward zero; x * id + 8.5 lies in [0, 17)
            const int q0 = (int)(x[j + t] * id + 8.5f), q1 = (int)(x[16 + j + t] * id + 8.5f);
            two |= (uint32_t)((q0 < 15 ? q0 : 15) | ((q1 < 15 ? q1 : 15) << 4)) << (8 * t);
        }
        p16[1 + j / 2] = (uint16_t)two;
    }
}

// ---- Q4_K and Q5_K ----
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

// One sub-block's fit for quantize_row_q4_K_ref: ggml's make_qkx2_quants with n = 32, nmax = 15,
// rmin = -1, rdelta = 0.1, nstep = 20 (the sub-block scale and min of the least weighted squared
// error over a grid of 21 inverse scales around nmax / (max - min), each refined by a least-squares
// fit, min clamped to <= 0), the same fp32 operations in the same order, on the sub-block held in
// registers. quantize_row_q5_K_ref's fit is the same search with nmax = 31, rmin = -0.5, nstep = 15. The chosen levels L are not stored: the (iscale, min) they were
// computed with are returned instead, so the caller recomputes them where it needs them.
struct Qkx2Fit {
    float scale, the_min;  // make_qkx2_quants' return value and *the_min
    float l_iscale, l_min;  // L_i = clamp(nearest_int(l_iscale * (x_i - l_min)), 0, 15)
    int zero;               // max == min: every L_i is 0
};

template <int NMAX>
__device__ __forceinline__ int clampq(int l) { return l < 0 ? 0 : (l > NMAX ? NMAX : l); }

template <bool Q5>
__device__ __forceinline__ Qkx2Fit qkx2_fit32(const float (&x)[32], float av_x) {
    constexpr int nmax = Q5 ? 31 : 15;
    const float rmin = Q5 ? -0.5f : -1.f, rdelta = 0.1f;
    const int nstep = Q5 ? 15 : 20;
    float w[32];  // the weights av_x + |x_i|, each computed once (the same fp32 value at every use)
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = av_x + fabsf(x[i]);
    float min = x[0], max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) return {0.f, -min, 0.f, 0.f, 1};
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    float l_iscale = iscale, l_min = min;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int l = clampq<nmax>(nearest_int(iscale * (x[i] - min)));
        const float diff = scale * (float)l + min - x[i];
        best_error += w[i] * (diff * diff);
    }
#pragma unroll 1
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        float lf[32];  // this candidate's levels, reused by its error sum
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            lf[i] = (float)clampq<nmax>(nearest_int(iscale * (x[i] - min)));
            sum_l += w[i] * lf[i];
            sum_l2 += w[i] * lf[i] * lf[i];
            sum_xl += w[i] * lf[i] * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const float diff = this_scale * lf[i] + this_min - x[i];
                mad += w[i] * (diff * diff);
            }
            if (mad < best_error) {
                l_iscale = iscale;
                l_min = min;
                best_error = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    return {scale, -min, l_iscale, l_min, 0};
}

// ---- Q4_K / Q5_K: quantize_row_q4_K_ref / quantize_row_q5_K_ref with eight lanes per superblock,
// one per 32-element sub-block. Each lane runs its sub-block's fit on its values in registers; the
// superblock's largest scale and min, and the packed scale bytes, come from exchanges within the
// eight lanes; each lane then forms its sub-block's final levels, and the even lane of a pair writes
// the pair's 32 nibble bytes. The maxima are exact in any order, so the bytes are those of ggml's
// sequential loop. ----
constexpr int kWqThreads = 256;
template <bool Q5>
__global__ void __launch_bounds__(kWqThreads) quantize_w_q4_K_kernel(const float* __restrict__ W, int64_t N,
                                                                     int64_t K, uint8_t* __restrict__ out) {
    constexpr int nmax = Q5 ? 31 : 15, kSb = Q5 ? 176 : 144, kQsDw = Q5 ? 12 : 4;
    const int64_t nsb = K / QK_K;
    const int64_t sg = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;  // superblock over [N][nsb]
    const int j = (int)(threadIdx.x & 7);                                       // its sub-block
    if (sg >= N * nsb) return;  // the eight lanes of a superblock leave together
    const int64_t r = sg / nsb, sbi = sg - r * nsb;
    float x[32];
    {
        const float4* p = reinterpret_cast<const float4*>(W + r * K + sbi * QK_K + 32 * j);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = p[q];
            x[4 * q] = v.x, x[4 * q + 1] = v.y, x[4 * q + 2] = v.z, x[4 * q + 3] = v.w;
        }
    }
    float sum_x2 = 0;
#pragma unroll
    for (int l = 0; l < 32; ++l) sum_x2 += x[l] * x[l];
    const float av_x = sqrtf(sum_x2 / 32);
    const Qkx2Fit f = qkx2_fit32<Q5>(x, av_x);
    // the superblock's largest scale and min, from 0 (ggml's running maxima)
    float max_scale = f.scale > 0 ? f.scale : 0.f, max_min = f.the_min > 0 ? f.the_min : 0.f;
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        const float a = __shfl_xor(max_scale, o, 8), c = __shfl_xor(max_min, o, 8);
        max_scale = a > max_scale ? a : max_scale;
        max_min = c > max_min ? c : max_min;
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    int ls = nearest_int(inv_scale * f.scale);
    int lm = nearest_int(inv_min * f.the_min);
    ls = ls < 63 ? ls : 63;
    lm = lm < 63 ? lm : 63;
    const uint16_t dh = float_to_half_bits(max_scale / 63.f), dminh = float_to_half_bits(max_min / 63.f);
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + sg * kSb);
    // the 12 scale bytes (get_scale_min_k4's packing) from the eight lanes' (ls, lm)
    const int pk = (ls & 0xFFFF) | (lm << 16);
    uint32_t scw[3] = {0, 0, 0};
    auto put = [&](int byte, uint32_t v) { scw[byte >> 2] |= (v & 0xFFu) << (8 * (byte & 3)); };
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int v = __shfl(pk, k, 8);
        const int lsk = (int)(int16_t)(v & 0xFFFF), lmk = v >> 16;
        if (k < 4) {
            put(k, (uint32_t)lsk);
            put(k + 4, (uint32_t)lmk);
        } else {
            put(k + 4, (uint32_t)((lsk & 0xF) | ((lmk & 0xF) << 4)));
            put(k - 4, (uint32_t)((lsk >> 4) << 6));
            put(k, (uint32_t)((lmk >> 4) << 6));
        }
    }
    if (j == 0) {
        dst[0] = (uint32_t)dh | ((uint32_t)dminh << 16);
        dst[1] = scw[0];
        dst[2] = scw[1];
        dst[3] = scw[2];
    }
    // final levels: from the 6-bit scales, or, where the scale quantized to 0, the fit's own levels.
    // Sub-blocks 2c and 2c + 1 are the low and high nibbles of qs[32c .. 32c + 32); Q5_K: bit 4 of
    // element ii of sub-block j goes to bit j of qh[ii].
    const float d = half_bits_to_float(dh) * (float)(uint8_t)ls;
    const float dm = half_bits_to_float(dminh) * (float)(uint8_t)lm;
    const int h = j & 1;
    uint32_t nib[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    [[maybe_unused]] uint32_t hb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) {
        int l;
        if (d != 0.0f)
            l = clampq<nmax>(nearest_int((x[ii] + dm) / d));
        else
            l = f.zero ? 0 : clampq<nmax>(nearest_int(f.l_iscale * (x[ii] - f.l_min)));
        nib[ii >> 2] |= (uint32_t)(l & 0xF) << (8 * (ii & 3) + 4 * h);
        if constexpr (Q5) hb[ii >> 2] |= (uint32_t)(l >> 4) << (8 * (ii & 3) + j);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) nib[q] |= (uint32_t)__shfl_xor((int)nib[q], 1, 8);
    if (h == 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[kQsDw + 8 * (j >> 1) + q] = nib[q];
    }
    if constexpr (Q5) {
#pragma unroll
        for (int o = 1; o < 8; o <<= 1)
#pragma unroll
            for (int q = 0; q < 8; ++q) hb[q] |= (uint32_t)__shfl_xor((int)hb[q], o, 8);
        if (j == 0) {
#pragma unroll
            for (int q = 0; q < 8; ++q) dst[4 + q] = hb[q];
        }
    }
}

// ---- Q6_K: quantize_row_q6_K_ref with sixteen lanes per superblock, one per 16-element group ----
// make_qx_quants with n = 16, nmax = 32, rmse_type 1 on one group held in registers (the levels L
// are l + 32 in [0, 63]); the candidate loop is ggml's, in order.
__device__ __forceinline__ float qx_fit16(const float (&x)[16], int (&L)[16]) {
    constexpr int nmax = 32;
    float max = 0, amax = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = l + nmax;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    float w[16], wx[16];  // x_i^2 and x_i^2 * x_i, the first factors of the sums below
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        w[i] = x[i] * x[i];
        wx[i] = w[i] * x[i];
    }
#pragma unroll 1
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            sumlx += wx[i] * l;
            suml2 += w[i] * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = l + nmax;
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// Lane ib fits group ib; the superblock scale is the scale of the first group of the largest |scale|
// (ggml's strict running maximum), found by exchanges within the sixteen lanes; each lane forms its
// group's scale byte and final levels. In the 210-byte superblock, element 128 jh + 32 qd + l of half
// jh and quarter qd is the low (qd 0, 1) or high (qd 2, 3) nibble of ql[64 jh + 32 (qd & 1) + l] and
// bits 2 qd of qh[32 jh + l]: group ib = 8 jh + 2 qd + (l >> 4). The lanes of one ql byte (ib, ib ^ 4)
// and of one qh byte (ib, ib ^ 2, ib ^ 4, ib ^ 6) combine by exchange; superblocks are 2-byte aligned,
// so the bytes go out as 16-bit stores.
__global__ void __launch_bounds__(kWqThreads) quantize_w_q6_K_kernel(const float* __restrict__ W, int64_t N, int64_t K,
                                                                     uint8_t* __restrict__ out) {
    const int64_t nsb = K / QK_K;
    const int64_t sg = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;  // superblock over [N][nsb]
    const int ib = (int)(threadIdx.x & 15);                                      // its group
    if (sg >= N * nsb) return;  // the sixteen lanes of a superblock leave together
    const int64_t r = sg / nsb, sbi = sg - r * nsb;
    float x[16];
    {
        const float4* p = reinterpret_cast<const float4*>(W + r * K + sbi * QK_K + 16 * ib);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = p[q];
            x[4 * q] = v.x, x[4 * q + 1] = v.y, x[4 * q + 2] = v.z, x[4 * q + 3] = v.w;
        }
    }
    int L[16];
    const float scale = qx_fit16(x, L);
    // the first group of the largest |scale|
    float best_abs = fabsf(scale), best_scale = scale;
    int best_ib = ib;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        const float a = __shfl_xor(best_abs, o, 16), sc = __shfl_xor(best_scale, o, 16);
        const int i2 = __shfl_xor(best_ib, o, 16);
        if (a > best_abs || (a == best_abs && i2 < best_ib)) {
            best_abs = a;
            best_scale = sc;
            best_ib = i2;
        }
    }
    uint16_t* d16 = reinterpret_cast<uint16_t*>(out + sg * 210);
    if (best_abs < 1e-15f) {  // an all-zero superblock: 105 zero halfwords over the sixteen lanes
        for (int k = ib; k < 105; k += 16) d16[k] = 0;
        return;
    }
    const float iscale = -128.f / best_scale;
    const uint16_t dh = float_to_half_bits(1 / iscale);
    const int v = nearest_int(iscale * scale);
    const int sc8 = v < 127 ? v : 127;  // the group's int8 scale
    const float d = half_bits_to_float(dh) * (float)(int8_t)sc8;
    if (d != 0.0f) {
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(x[ii] / d);
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            L[ii] = l + 32;
        }
    }
    const int jh = ib >> 3, g = ib & 7, qd = g >> 1, l0 = 16 * (g & 1);
    uint32_t ql[4] = {0, 0, 0, 0}, qh[4] = {0, 0, 0, 0};
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
        ql[ii >> 2] |= (uint32_t)(L[ii] & 0xF) << (8 * (ii & 3) + 4 * (qd >> 1));
        qh[ii >> 2] |= (uint32_t)(L[ii] >> 4) << (8 * (ii & 3) + 2 * qd);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        ql[q] |= (uint32_t)__shfl_xor((int)ql[q], 4, 16);
        qh[q] |= (uint32_t)__shfl_xor((int)qh[q], 2, 16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) qh[q] |= (uint32_t)__shfl_xor((int)qh[q], 4, 16);
    if ((qd >> 1) == 0) {  // ql bytes 64 jh + 32 qd + l0 ..
        uint16_t* p = d16 + (64 * jh + 32 * qd + l0) / 2;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            p[2 * q] = (uint16_t)ql[q];
            p[2 * q + 1] = (uint16_t)(ql[q] >> 16);
        }
    }
    if (qd == 0) {  // qh bytes 128 + 32 jh + l0 ..
        uint16_t* p = d16 + (128 + 32 * jh + l0) / 2;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            p[2 * q] = (uint16_t)qh[q];
            p[2 * q + 1] = (uint16_t)(qh[q] >> 16);
        }
    }
    // scale bytes 192 + ib (pairs as halfwords), then d
    const int sc_pair = (sc8 & 0xFF) | ((__shfl_xor(sc8, 1, 16) & 0xFF) << 8);
    if ((ib & 1) == 0) d16[(192 + ib) / 2] = (uint16_t)sc_pair;
    if (ib == 0) d16[104] = dh;
}

// ---- dequantization: one thread per 32 output elements ----
__global__ void __launch_bounds__(256) dequantize_kernel(int type, const uint8_t* __restrict__ Wq, int64_t N,
                                                         int64_t K, int64_t w_row_bytes, float* __restrict__ Y) {
    const int64_t per_row = K / 32;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= N * per_row) return;
    const int64_t r = gid / per_row, c = gid - (gid / per_row) * per_row;  // chunk of 32 elements
    const uint8_t* row = Wq + r * w_row_bytes;
    float* y = Y + r * K + c * 32;
    if (type == kTypeQ8_0) {
        const uint8_t* b = row + c * 34;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b));
        for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
    } else if (type == kTypeQ8_0_RS) {
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(row + K + 2 * c));
        for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)row[32 * c + j] * d;
    } else if (type == kTypeQ4_K) {
        const uint8_t* b = row + (c / 8) * 144;
        const int j = (int)(c % 8);  // sub-block
        uint8_t sc, m;
        scale_min_k4(j, b + 4, &sc, &m);
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b)) * sc;
        const float dm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b + 2)) * m;
        const uint8_t* qs = b + 16 + 32 * (j / 2);
        for (int l = 0; l < 32; ++l) {
            const int q = (j & 1) ? (qs[l] >> 4) : (qs[l] & 0xF);
            y[l] = d * q - dm;
        }
    } else if (type == kTypeQ4_0) {
        const uint8_t* b = row + c * 18;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b));
        for (int j = 0; j < 16; ++j) {
            y[j] = (float)((int)(b[2 + j] & 0xF) - 8) * d;
            y[j + 16] = (float)((int)(b[2 + j] >> 4) - 8) * d;
        }
    } else if (type == kTypeQ5_K) {
        const uint8_t* b = row + (c / 8) * 176;
        const int j = (int)(c % 8);  // sub-block
        uint8_t sc, m;
        scale_min_k4(j, b + 4, &sc, &m);
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b)) * sc;
        const float dm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(b + 2)) * m;
        const uint8_t* qs = b + 48 + 32 * (j / 2);
        for (int l = 0; l < 32; ++l) {
            const int q = ((j & 1) ? (qs[l] >> 4) : (qs[l] & 0xF)) + 16 * ((b[16 + l] >> j) & 1);
            y[l] = d * q - dm;
        }
    } else if (type == kTypeQ6_K) {
        const uint8_t* b = row + (c / 8) * 210;
        const float d = half_bits_to_float((uint32_t)b[208] | ((uint32_t)b[209] << 8));
        for (int l = 0; l < 32; ++l) {
            const int e = (int)(c % 8) * 32 + l;
            const int h = e / 128, ep = e % 128, t = ep / 32, ll = ep % 32;
            const int lo = (b[64 * h + ll + 32 * (t & 1)] >> (4 * (t >> 1))) & 0xF;
            const int hi = (b[128 + 32 * h + ll] >> (2 * t)) & 3;
            y[l] = d * (float)(int8_t)b[192 + e / 16] * (float)((lo | (hi << 4)) - 32);
        }
    } else if (type == kTypeQ8_K) {
        const uint8_t* b = row + (c / 8) * 292;
        const float d = *reinterpret_cast<const float*>(b);
        for (int l = 0; l < 32; ++l) y[l] = d * (float)(int8_t)b[4 + (c % 8) * 32 + l];
    }
}

// ---- load-time repack: Q8_0 rows into row-split rows (quants plane, then scales plane) ----
// One thread per 32-element block: the block's 34 bytes (2-byte aligned) as 17 halfwords; the 32
// quants go out as two 16-byte stores (out rows 16-byte aligned), the scale as one halfword.
__global__ void __launch_bounds__(256) repack_q8_0_rs_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                             int64_t N, int64_t K, uint8_t* __restrict__ out,
                                                             int64_t out_row_bytes) {
    const int64_t nb = K / 32;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= N * nb) return;
    const int64_t r = gid / nb, b = gid - r * nb;
    const uint16_t* p = reinterpret_cast<const uint16_t*>(W + r * w_row_bytes + b * 34);
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
    uint8_t* o = out + r * out_row_bytes;
    *reinterpret_cast<uint4*>(o + 32 * b) = make_uint4(q[0], q[1], q[2], q[3]);
    *reinterpret_cast<uint4*>(o + 32 * b + 16) = make_uint4(q[4], q[5], q[6], q[7]);
    *reinterpret_cast<uint16_t*>(o + K + 2 * b) = p[0];
}

hipError_t launch_repack_q8_0_rs(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, void* out,
                                 int64_t out_row_bytes, hipStream_t st) {
    const int64_t t = N * (K / 32);
    hipLaunchKernelGGL(repack_q8_0_rs_kernel, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st,
                       (const uint8_t*)W, w_row_bytes, N, K, (uint8_t*)out, out_row_bytes);
    return hipGetLastError();
}

hipError_t launch_quantize_weights(int wtype, const float* W, int64_t N, int64_t K, void* Wq, hipStream_t st) {
    if (wtype == kTypeQ8_0) {
        const int64_t t = N * (K / QK8_0);
        hipLaunchKernelGGL(quantize_w_q8_0_kernel, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, W, N, K,
                           (uint8_t*)Wq);
    } else if (wtype == kTypeQ4_0) {
        const int64_t t = N * (K / QK8_0);
        hipLaunchKernelGGL(quantize_w_q4_0_kernel, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, W, N, K,
                           (uint8_t*)Wq);
    } else if (wtype == kTypeQ4_K || wtype == kTypeQ5_K) {
        const int64_t t = N * (K / QK_K);
        hipLaunchKernelGGL(wtype == kTypeQ5_K ? quantize_w_q4_K_kernel<true> : quantize_w_q4_K_kernel<false>,
                           dim3((unsigned)((8 * t + kWqThreads - 1) / kWqThreads)), dim3(kWqThreads), 0, st, W, N,
                           K, (uint8_t*)Wq);
    } else {
        const int64_t t = N * (K / QK_K);
        hipLaunchKernelGGL(quantize_w_q6_K_kernel, dim3((unsigned)((16 * t + kWqThreads - 1) / kWqThreads)),
                           dim3(kWqThreads), 0, st, W, N, K, (uint8_t*)Wq);
    }
    return hipGetLastError();
}

hipError_t launch_dequantize(int type, const void* Wq, int64_t N, int64_t K, int64_t w_row_bytes, float* Y,
                             hipStream_t st) {
    const int64_t t = N * (K / 32);
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, st, type,
                       (const uint8_t*)Wq, N, K, w_row_bytes, Y);
    return hipGetLastError();
}

}  // namespace dcq
