// dcq_quantize.hip — activation quantization (the vec_dot_type `from_float`).
//
// Replaces type_traits_cpu(vec_dot_type)->from_float at
// core/src/inference.cpp:889-892 (and the src1 quantization inside ggml's CPU
// MUL_MAT). Bit-exact semantics:
//   Q8_0 (ggml-cpu x86 SIMD form): amax = max|x|; d = amax/127 (fp32 divide,
//     correctly rounded) stored as fp16 (RNE); id = amax ? 127/amax : 0;
//     q = round-half-even(x*id) (v_rndne_f32 of the rounded product).
//   Q8_K (quantize_row_q8_K_ref): max = first element of largest |x|;
//     iscale = -127/max; q = min(127, round-half-even(iscale*x)); d = 1/iscale;
//     bsums[g] = sum of q[16g..16g+15]; an all-zero block is all zero. 16 lanes per
//     superblock, reduced with DPP (quantize_q8k_row16).
// Memory-bound: reads 4 B and writes ~1.06 B (Q8_0) / ~1.14 B (Q8_K) per element.
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

// ---- Q8_0: 4 lanes per 32-element block, 8 floats per lane ----
template <bool kPlanar>
__global__ void __launch_bounds__(256) quantize_q8_0_kernel(const float* __restrict__ X, int64_t x_stride,
                                                            int64_t M, int64_t K, int64_t m_ld,
                                                            int8_t* __restrict__ qs, float* __restrict__ dpl,
                                                            uint8_t* __restrict__ out, int64_t out_row_bytes) {
    const int64_t nb = K / QK8_0;
    const int q = (int)(threadIdx.x & 3);  // quarter of the block
    int64_t m, b;
    if (kPlanar) {
        // a 256-thread workgroup takes 32 rows x 2 blocks (lane group g: row g % 32, block g / 32),
        // so each block's 32 scales go out as one 128-byte run of the [nb][m_ld] scale array
        const int64_t tiles_b = (nb + 1) / 2, g = threadIdx.x >> 2;
        m = (int64_t)(blockIdx.x / tiles_b) * 32 + (g & 31);
        b = (int64_t)(blockIdx.x % tiles_b) * 2 + (g >> 5);
        if (b >= nb) return;            // whole groups of 4 lanes exit together
    } else {
        const int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 2;  // over [M][nb]
        m = blk / nb;
        b = blk - m * nb;
    }
    if (m >= m_ld) return;              // whole groups of 4 lanes exit together
    if (m >= M) {                       // planar padding rows: scale 0
        if (kPlanar && q == 0) dpl[b * m_ld + m] = 0.0f;
        return;
    }
    const float* xp = X + m * x_stride + b * QK8_0 + q * 8;
    const float4 v0 = *reinterpret_cast<const float4*>(xp);
    const float4 v1 = *reinterpret_cast<const float4*>(xp + 4);
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 4));
    const float d = amax / 127.f;
    const uint16_t dh = float_to_half_bits(d);
    const float id = amax != 0.0f ? 127.f / amax : 0.0f;
    const float xs[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float r = __builtin_rintf(xs[j] * id);
        r = fminf(fmaxf(r, -128.f), 127.f);
        const uint32_t byte = (uint32_t)(int32_t)r & 0xFFu;
        packed[j >> 2] |= byte << (8 * (j & 3));
    }
    if (kPlanar) {
        *reinterpret_cast<uint2*>(qs + m * K + b * QK8_0 + q * 8) = make_uint2(packed[0], packed[1]);
        if (q == 0) dpl[b * m_ld + m] = half_bits_to_float(dh);
    } else {
        uint8_t* blkp = out + m * out_row_bytes + b * (int64_t)sizeof(BlockQ8_0);
        uint16_t* qs16 = reinterpret_cast<uint16_t*>(blkp + 2 + q * 8);  // 2-byte aligned
        qs16[0] = (uint16_t)packed[0];
        qs16[1] = (uint16_t)(packed[0] >> 16);
        qs16[2] = (uint16_t)packed[1];
        qs16[3] = (uint16_t)(packed[1] >> 16);
        if (q == 0) *reinterpret_cast<uint16_t*>(blkp) = dh;
    }
}

// ---- Q8_K: 16 lanes (one DPP row) per 256-element superblock, 16 floats per lane ----
template <bool kPlanar>
__global__ void __launch_bounds__(256) quantize_q8_K_kernel(const float* __restrict__ X, int64_t x_stride,
                                                            int64_t M, int64_t K, int64_t m_ld,
                                                            int8_t* __restrict__ qs, int16_t* __restrict__ bsp,
                                                            float* __restrict__ dpl, uint8_t* __restrict__ out,
                                                            int64_t out_row_bytes) {
    const int64_t nsb = K / QK_K;
    const int g = threadIdx.x & 15;
    int64_t m, s;
    if (kPlanar) {
        // a 256-thread workgroup takes 16 rows of one superblock, so their scales go out as one
        // 64-byte run of the [nsb][m_ld] scale array
        m = (int64_t)(blockIdx.x / nsb) * 16 + (threadIdx.x >> 4);
        s = blockIdx.x % nsb;
    } else {
        const int64_t sbg = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;  // over [M][nsb]
        m = sbg / nsb;
        s = sbg - m * nsb;
    }
    if (m >= m_ld) return;  // whole 16-lane rows exit together
    if (m >= M) {
        if (kPlanar && g == 0) dpl[s * m_ld + m] = 0.0f;
        return;
    }
    const float4* xp = reinterpret_cast<const float4*>(X + m * x_stride + s * QK_K + 16 * g);
    float x[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = xp[i];
        x[4 * i] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
    }
    uint32_t packed[4];
    int bsum;
    float dval;
    quantize_q8k_row16(x, g, packed, bsum, dval);
    if (kPlanar) {
        *reinterpret_cast<uint4*>(qs + m * K + s * QK_K + 16 * g) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        bsp[m * (K / 16) + s * 16 + g] = (int16_t)bsum;
        if (g == 0) dpl[s * m_ld + m] = dval;
    } else {
        uint8_t* blkp = out + m * out_row_bytes + s * (int64_t)sizeof(BlockQ8_K);
        U32x4 w;
        w.x = packed[0];
        w.y = packed[1];
        w.z = packed[2];
        w.w = packed[3];
        *reinterpret_cast<U32x4*>(blkp + 4 + 16 * g) = w;  // 4-byte aligned block
        *reinterpret_cast<int16_t*>(blkp + 4 + QK_K + 2 * g) = (int16_t)bsum;
        if (g == 0) *reinterpret_cast<float*>(blkp) = dval;
    }
}

// ---- ggml block rows -> planar (used by dcq_dot_rows on pre-quantized input) ----
__global__ void __launch_bounds__(256) unpack_q8_0_rows_kernel(const uint8_t* __restrict__ in, int64_t in_row_bytes,
                                                               int64_t M, int64_t K, int8_t* __restrict__ qs,
                                                               float* __restrict__ dpl, int64_t m_ld) {
    const int64_t nb = K / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / nb, b = gid - (gid / nb) * nb;
    if (m >= m_ld) return;
    if (m >= M) {
        dpl[b * m_ld + m] = 0.0f;
        return;
    }
    const uint8_t* blkp = in + m * in_row_bytes + b * (int64_t)sizeof(BlockQ8_0);
    const uint16_t* q16 = reinterpret_cast<const uint16_t*>(blkp + 2);
    uint32_t* dst = reinterpret_cast<uint32_t*>(qs + m * K + b * QK8_0);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = (uint32_t)q16[2 * i] | ((uint32_t)q16[2 * i + 1] << 16);
    dpl[b * m_ld + m] = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blkp));
}

__global__ void __launch_bounds__(256) unpack_q8_K_rows_kernel(const uint8_t* __restrict__ in, int64_t in_row_bytes,
                                                               int64_t M, int64_t K, int8_t* __restrict__ qs,
                                                               float* __restrict__ dpl, int16_t* __restrict__ bsp,
                                                               int64_t m_ld) {
    const int64_t nsb = K / QK_K;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = gid / nsb, s = gid - (gid / nsb) * nsb;
    if (m >= m_ld) return;
    if (m >= M) {
        dpl[s * m_ld + m] = 0.0f;
        return;
    }
    const uint8_t* blkp = in + m * in_row_bytes + s * (int64_t)sizeof(BlockQ8_K);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(blkp + 4);
    uint32_t* dst = reinterpret_cast<uint32_t*>(qs + m * K + s * QK_K);
    for (int i = 0; i < QK_K / 4; ++i) dst[i] = src[i];
    const int16_t* bsrc = reinterpret_cast<const int16_t*>(blkp + 4 + QK_K);
    for (int g = 0; g < 16; ++g) bsp[m * (K / 16) + s * 16 + g] = bsrc[g];
    dpl[s * m_ld + m] = *reinterpret_cast<const float*>(blkp);
}

// ---- host launchers ----
// Block size: 256 threads, or 64 when that leaves fewer workgroups than two per CU, so that
// a small activation (a few rows) spreads over more CUs and L2 channels.
static int quant_block(int64_t threads) { return threads < 2 * 256 * (int64_t)cu_count() ? 64 : 256; }
hipError_t launch_quantize_ggml(int vdt, const float* X, int64_t x_stride, int64_t M, int64_t K, void* out,
                                int64_t out_row_bytes, hipStream_t st) {
    if (vdt == kTypeQ8_0) {
        const int64_t threads = M * (K / QK8_0) * 4;
        const int bs = quant_block(threads);
        const int64_t grid = (threads + bs - 1) / bs;
        hipLaunchKernelGGL(quantize_q8_0_kernel<false>, dim3((unsigned)grid), dim3(bs), 0, st, X, x_stride, M, K, M,
                           (int8_t*)nullptr, (float*)nullptr, (uint8_t*)out, out_row_bytes);
    } else {
        const int64_t threads = M * (K / QK_K) * 16;
        const int bs = quant_block(threads);
        const int64_t grid = (threads + bs - 1) / bs;
        hipLaunchKernelGGL(quantize_q8_K_kernel<false>, dim3((unsigned)grid), dim3(bs), 0, st, X, x_stride, M, K, M,
                           (int8_t*)nullptr, (int16_t*)nullptr, (float*)nullptr, (uint8_t*)out, out_row_bytes);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_planar(int vdt, const float* X, int64_t x_stride, int64_t M, int64_t K,
                                  const PlanarBuffers& pb, hipStream_t st) {
    // m_ld is a multiple of 128 (planar_bytes): whole 32-row (Q8_0) or 16-row (Q8_K) tiles
    if (pb.m_ld % 32) return hipErrorInvalidValue;
    if (vdt == kTypeQ8_0) {
        const int64_t grid = (pb.m_ld / 32) * ((K / QK8_0 + 1) / 2);
        if (grid > UINT32_MAX) return hipErrorInvalidValue;
        hipLaunchKernelGGL(quantize_q8_0_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, X, x_stride, M, K,
                           pb.m_ld, pb.qs, pb.d, (uint8_t*)nullptr, (int64_t)0);
    } else {
        const int64_t grid = (pb.m_ld / 16) * (K / QK_K);
        if (grid > UINT32_MAX) return hipErrorInvalidValue;
        hipLaunchKernelGGL(quantize_q8_K_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, X, x_stride, M, K,
                           pb.m_ld, pb.qs, pb.bs, pb.d, (uint8_t*)nullptr, (int64_t)0);
    }
    return hipGetLastError();
}

hipError_t launch_unpack_ggml_rows(int vdt, const void* in, int64_t in_row_bytes, int64_t M, int64_t K,
                                   const PlanarBuffers& pb, hipStream_t st) {
    if (vdt == kTypeQ8_0) {
        const int64_t threads = pb.m_ld * (K / QK8_0);
        hipLaunchKernelGGL(unpack_q8_0_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t*)in, in_row_bytes, M, K, pb.qs, pb.d, pb.m_ld);
    } else {
        const int64_t threads = pb.m_ld * (K / QK_K);
        hipLaunchKernelGGL(unpack_q8_K_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                           (const uint8_t*)in, in_row_bytes, M, K, pb.qs, pb.d, pb.bs, pb.m_ld);
    }
    return hipGetLastError();
}

}  // namespace dcq
