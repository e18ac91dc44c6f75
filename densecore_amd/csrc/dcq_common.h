// dcq_common.h — shared definitions of the gfx950 quantized mul_mat library.
//
// GGUF block layouts (little-endian, `half` = IEEE fp16), as the reference's
// ggml stores weights in host memory (core/src/model_loader.cpp:103-122) and
// DenseCore's own Metal shader restates for Q8_0
// (core/shaders/quantized_gemv.metal:85-88):
//   Q8_0 (32 elems, 34 B):  { half d; int8 qs[32]; }                 value = d*qs[i]
//   Q4_0 (32 elems, 18 B):  { half d; u8 qs[16]; }  elems i, i+16 = low, high nibble of qs[i];
//                                                   value = d*(q - 8)
//   Q4_K (256 elems, 144 B):{ half d; half dmin; u8 scales[12]; u8 qs[128]; }
//   Q5_K (256 elems, 176 B):{ half d; half dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]; }
//                           qs as Q4_K's nibbles; bit j of qh[l] = bit 4 of elem l of sub-block j
//   Q6_K (256 elems, 210 B):{ u8 ql[128]; u8 qh[64]; i8 scales[16]; half d; }
//   Q8_K (256 elems, 292 B):{ float d; i8 qs[256]; i16 bsums[16]; }
//
// Planar activation layout (library-internal, in the caller's workspace). The
// GPU kernels consume quantized activations in this split form rather than
// the ggml block array; dcq_quantize_rows still emits the ggml bytes.
//   qs : int8  [M][K]                 row m at qs + m*K (K % 32 == 0, so rows stay 16-B aligned)
//   d  : float [K/bs][M_ld]           block-major scales (fp16 d widened exactly for Q8_0,
//                                     fp32 d for Q8_K); M_ld = M rounded up to 128, rows
//                                     M..M_ld-1 hold 0
//   bs : int16 [M][K/16]              Q8_K bsums (sum of 16 consecutive qs)
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dcq {

constexpr int kTypeF32 = 0;
constexpr int kTypeF16 = 1;
constexpr int kTypeQ4_0 = 2;
constexpr int kTypeQ8_0 = 8;
constexpr int kTypeQ4_K = 12;
constexpr int kTypeQ5_K = 13;
constexpr int kTypeQ6_K = 14;
constexpr int kTypeQ8_K = 15;
// Library layout, not a ggml type: Q8_0 rows split into planes (dcq_repack_weights writes it from
// Q8_0 rows). A row of K elements holds the K int8 quants first (block b's 32 at byte 32b, so
// every 16-byte piece is 16-byte aligned), then the K/32 fp16 scales (block b's at byte K + 2b):
// the same 34 bytes per block as Q8_0, the same values.
constexpr int kTypeQ8_0_RS = 108;

constexpr int QK8_0 = 32;
constexpr int QK_K = 256;

struct __attribute__((packed)) BlockQ8_0 {
    uint16_t d;
    int8_t qs[QK8_0];
};
struct __attribute__((packed)) BlockQ4_0 {
    uint16_t d;
    uint8_t qs[QK8_0 / 2];
};
struct BlockQ4_K {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[QK_K / 2];
};
struct BlockQ5_K {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qh[QK_K / 8];
    uint8_t qs[QK_K / 2];
};
struct BlockQ6_K {
    uint8_t ql[QK_K / 2];
    uint8_t qh[QK_K / 4];
    int8_t scales[QK_K / 16];
    uint16_t d;
};
struct BlockQ8_K {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
};
static_assert(sizeof(BlockQ8_0) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(BlockQ4_0) == 18, "Q4_0 block is 18 bytes");
static_assert(sizeof(BlockQ4_K) == 144, "Q4_K block is 144 bytes");
static_assert(sizeof(BlockQ5_K) == 176, "Q5_K block is 176 bytes");
static_assert(sizeof(BlockQ6_K) == 210, "Q6_K block is 210 bytes");
static_assert(sizeof(BlockQ8_K) == 292, "Q8_K block is 292 bytes");

// Quantized activations in the planar layout (device pointers into the workspace).
struct ActPlanar {
    const int8_t* qs;   // [M][K]
    const float* d;     // [K/bs][m_ld]
    const int16_t* bs;  // [M][K/16] (Q8_K only)
    int64_t M;
    int64_t K;
    int64_t m_ld;
};

inline __host__ __device__ int64_t round_up(int64_t a, int64_t b) { return (a + b - 1) / b * b; }

// ---- device helpers ----

__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
    _Float16 h;
    uint16_t b = (uint16_t)h16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// fp32 -> fp16 bits, IEEE round-to-nearest-even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Four unsigned 4-bit values (one per byte, 0..15) to the signed bytes q - 8, per byte without
// borrows: (q | 0x80) - 8 = 0x78 + q stays in its byte, and the xor turns 0x80 + (q - 8) into
// the two's complement byte of q - 8.
__device__ __forceinline__ uint32_t minus8(uint32_t q) { return ((q | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }
// Q5_K levels of one sub-block: the nibbles (already shifted down to bits 0..3 of each byte) with
// bit `bit` of each qh byte as bit 4.
__device__ __forceinline__ uint32_t q5_levels(uint32_t nib, uint32_t qh, uint32_t bit) {
    return (nib & 0x0F0F0F0Fu) | (((qh >> bit) & 0x01010101u) << 4);
}

// Q4_0 block: sum over its 32 elements of (q - 8) * a; q[0..3] hold the 16 bytes of nibbles
// (elements 0..15 low, 16..31 high), lo / hi the activation's elements 0..15 / 16..31.
__device__ __forceinline__ int q4_0_block_dot(const uint32_t (&q)[4], const uint4& lo, const uint4& hi) {
    const uint32_t m = 0x0F0F0F0Fu;
    int i = 0;
    i = sdot4((int)minus8(q[0] & m), (int)lo.x, i);
    i = sdot4((int)minus8(q[1] & m), (int)lo.y, i);
    i = sdot4((int)minus8(q[2] & m), (int)lo.z, i);
    i = sdot4((int)minus8(q[3] & m), (int)lo.w, i);
    i = sdot4((int)minus8((q[0] >> 4) & m), (int)hi.x, i);
    i = sdot4((int)minus8((q[1] >> 4) & m), (int)hi.y, i);
    i = sdot4((int)minus8((q[2] >> 4) & m), (int)hi.z, i);
    i = sdot4((int)minus8((q[3] >> 4) & m), (int)hi.w, i);
    return i;
}

// (hi:lo) >> (8*shift), low 32 bits; shift in bytes (0..3).
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// A dword-aligned pair of Q4_0 blocks (36 bytes as 9 dwords: block 0's d in bytes 0..1 and its
// nibbles in 2..17, block 1's d in 18..19 and nibbles in 20..35) against 64 activation bytes:
// the two blocks' exact sums and scales.
__device__ __forceinline__ void q4_0_pair(const uint32_t (&w)[9], const uint4& a0, const uint4& a1, const uint4& a2,
                                          const uint4& a3, int& i0, int& i1, float& dW0, float& dW1) {
    const uint32_t q0[4] = {align_bytes(w[1], w[0], 2), align_bytes(w[2], w[1], 2), align_bytes(w[3], w[2], 2),
                            align_bytes(w[4], w[3], 2)};
    const uint32_t q1[4] = {w[5], w[6], w[7], w[8]};
    i0 = q4_0_block_dot(q0, a0, a1);
    i1 = q4_0_block_dot(q1, a2, a3);
    dW0 = half_bits_to_float(w[0] & 0xFFFFu);
    dW1 = half_bits_to_float(w[4] >> 16);
}

// Global loads with the alignment the data actually has. 16 B at 4-B alignment is a
// single global_load_dwordx4 (gfx9 needs dword alignment for multi-dword accesses).
struct __attribute__((aligned(4))) U32x4 {
    uint32_t x, y, z, w;
};
struct __attribute__((aligned(4))) U32x2 {
    uint32_t x, y;
};
__device__ __forceinline__ U32x4 ld4(const void* p) { return *reinterpret_cast<const U32x4*>(p); }
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint32_t ld1(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ldu16(const void* p) { return *reinterpret_cast<const uint16_t*>(p); }

// 16 bytes starting at a 2-byte aligned address p, reading only [p - (p & 3), p + 16):
// 4 dwords from the dword at or below p, then the last 2 bytes with a halfword
// load when p is not dword aligned (so a piece that ends a tensor never reads past it).
__device__ __forceinline__ void ld16_a2(const uint8_t* p, uint32_t out[4]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t sh = (uint32_t)(a & 3u);
    const U32x4 w = ld4(p - sh);
    const uint32_t w4 = ldu16(p + (sh ? 14 : 12));
    out[0] = align_bytes(w.y, w.x, sh);
    out[1] = align_bytes(w.z, w.y, sh);
    out[2] = align_bytes(w.w, w.z, sh);
    out[3] = align_bytes(w4, w.w, sh);
}

// ---- cross-lane reductions inside a 16-lane DPP row (no LDS traffic) ----
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: after the four
// steps every lane of the row holds the reduction over its 16 lanes.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
    return v;
}
// Two independent row maxima of NON-NEGATIVE floats, interleaved step by step. Their bit
// patterns order like the values as signed integers (a -0.0 sorts below everything, and is
// equal to +0.0 as a float), so the steps are integer maxima: no canonicalizing of the DPP
// operand, and each move folds into the max as its DPP source.
__device__ __forceinline__ void row16_max2_nonneg(float& a, float& b) {
    int ia = __float_as_int(a), ib = __float_as_int(b);
    ia = max(ia, __builtin_amdgcn_mov_dpp(ia, 0xB1, 0xF, 0xF, false));
    ib = max(ib, __builtin_amdgcn_mov_dpp(ib, 0xB1, 0xF, 0xF, false));
    ia = max(ia, __builtin_amdgcn_mov_dpp(ia, 0x4E, 0xF, 0xF, false));
    ib = max(ib, __builtin_amdgcn_mov_dpp(ib, 0x4E, 0xF, 0xF, false));
    ia = max(ia, __builtin_amdgcn_mov_dpp(ia, 0x141, 0xF, 0xF, false));
    ib = max(ib, __builtin_amdgcn_mov_dpp(ib, 0x141, 0xF, 0xF, false));
    ia = max(ia, __builtin_amdgcn_mov_dpp(ia, 0x140, 0xF, 0xF, false));
    ib = max(ib, __builtin_amdgcn_mov_dpp(ib, 0x140, 0xF, 0xF, false));
    a = __int_as_float(ia);
    b = __int_as_float(ib);
}
__device__ __forceinline__ int row16_or(int v) {
    v |= dpp_mov<0xB1>(v);
    v |= dpp_mov<0x4E>(v);
    v |= dpp_mov<0x141>(v);
    v |= dpp_mov<0x140>(v);
    return v;
}
__device__ __forceinline__ int row16_min(int v) {
    v = min(v, dpp_mov<0xB1>(v));
    v = min(v, dpp_mov<0x4E>(v));
    v = min(v, dpp_mov<0x141>(v));
    v = min(v, dpp_mov<0x140>(v));
    return v;
}

// Sum over aligned groups of L lanes (L a power of two <= 64); every lane of a group gets
// the group's sum. Inside a 16-lane row by DPP (quad swaps, half-row mirror, row mirror:
// each step adds a partner holding the same partial sum set), then across rows by
// ds_bpermute. Partners add the same two values, so all lanes of a group agree bitwise.
template <int L>
__device__ __forceinline__ float lanes_sum(float v) {
    if (L >= 2) v += __int_as_float(dpp_mov<0xB1>(__float_as_int(v)));
    if (L >= 4) v += __int_as_float(dpp_mov<0x4E>(__float_as_int(v)));
    if (L >= 8) v += __int_as_float(dpp_mov<0x141>(__float_as_int(v)));
    if (L >= 16) v += __int_as_float(dpp_mov<0x140>(__float_as_int(v)));
    if (L >= 32) v += __shfl_xor(v, 16, 64);
    if (L >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Maximum over aligned groups of L lanes, in the same steps as lanes_sum.
template <int L>
__device__ __forceinline__ float lanes_max(float v) {
    if (L >= 2) v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
    if (L >= 4) v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
    if (L >= 8) v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
    if (L >= 16) v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
    if (L >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if (L >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// SiLU of the SwiGLU gate, g / (1 + e^-g) (ggml_silu's definition). expf is within a few ulp,
// far inside the fp32 tolerance of the dot products it multiplies.
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Pack the low bytes of four dwords (b0 lowest) into one dword.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // b0.byte0 | b1.byte0 << 8
    const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);  // b2.byte0 << 16 | b3.byte0 << 24
    return lo | hi;
}

// One Q8_K superblock (quantize_row_q8_K_ref semantics) quantized by the 16 lanes of a
// DPP row; lane g (= lane % 16) holds elements 16g .. 16g+15 in x[16]. Returns the lane's
// 16 quantized bytes (4 dwords), the sum of its 16-element group (bsums[g]) and d.
//   max = first element of largest |x| (strict '>' scan); iscale = -127/max;
//   q = min(127, round-half-even(iscale*x)); d = 1/iscale; an all-zero block is all zero.
// Exactness notes:
//   - max |x| and the first index holding it do not depend on the reduction order. Only
//     the sign of that element matters (max = +-amax); it is decided by whether +amax /
//     -amax occur in the block, and by the exact first-index scan when both occur.
//   - |iscale*x| <= 127 (up to one rounding), so round-half-even(iscale*x) lies in
//     [-127, 127] and the min(127, .) never binds. The rounding is ggml's nearest_int:
//     u = fl(iscale*x) + 1.5*2^23 rounds to an integer (half even) and its bit pattern is
//     0x4B400000 + q, so q's two's-complement byte is u's low byte and the 16-element sum
//     is sum(bits(u)) - 16*0x4B400000.
__device__ __forceinline__ void quantize_q8k_row16(const float (&x)[16], int g, uint32_t (&packed)[4], int& bsum,
                                                   float& dval) {
#pragma clang fp contract(off)
    // max(0, x_j) and max(0, -x_j) over the lane, then over the row: amax = max |x_j|, and
    // +amax (-amax) occurs in the row iff the first (second) of the two reaches it
    float hi = 0.0f, nlo = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        hi = fmaxf(hi, x[j]);
        nlo = fmaxf(nlo, -x[j]);
    }
    row16_max2_nonneg(hi, nlo);
    const float amax = fmaxf(hi, nlo);
    const int flags = (hi == amax ? 1 : 0) | (nlo == amax ? 2 : 0);
    float maxv = (flags & 2) ? -amax : amax;
    if (flags == 3) {
        // both signs hold the maximum: the first index decides (exact scan, rare)
        int key = 0x7FFFFFFF;
#pragma unroll
        for (int j = 15; j >= 0; --j)
            key = (fabsf(x[j]) == amax) ? (((16 * g + j) << 1) | (int)(__float_as_uint(x[j]) >> 31)) : key;
        key = row16_min(key);
        maxv = (key & 1) ? -amax : amax;
    }
    bsum = 0;
    dval = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed[i] = 0u;
    if (amax != 0.0f) {
        const float iscale = -127.f / maxv;
        uint32_t u[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            // two roundings, as ggml: fl(iscale*x), then + 1.5*2^23 (contraction is off here)
            const float t = iscale * x[j];
            u[j] = __float_as_uint(t + 12582912.0f);
        }
        uint32_t sum = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) sum += u[j];
        bsum = (int)(sum - 16u * 0x4B400000u);
#pragma unroll
        for (int i = 0; i < 4; ++i) packed[i] = pack_low_bytes(u[4 * i], u[4 * i + 1], u[4 * i + 2], u[4 * i + 3]);
        dval = 1.0f / iscale;
    }
}

}  // namespace dcq
