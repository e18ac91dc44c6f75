// dcq_gemv.hip — decode GEMV / small-M mul_mat on int8 dot products (v_dot4_i32_i8).
//
// Replaces the per-row vec_dot loop of cb_gemv_custom (core/src/inference.cpp:
// 896-923) and of ggml's CPU MUL_MAT at M <= 8. The reference splits rows over
// nth CPU threads; here a wave owns 64/G rows and G lanes stream one row.
//
// Work unit: 64 weight elements of one row.
//   Q8_0: a pair of 34-byte blocks (68 B, 17 dwords, dword aligned when K % 64 == 0)
//   row-split Q8_0: a pair's 64 quants (16-byte aligned) and its two fp16 scales from the row's
//         scales plane (17 dwords, no re-slicing)
//   Q4_0: a pair of 18-byte blocks (36 B, 9 dwords, dword aligned when K % 64 == 0), or one
//         block read as 9 halfwords otherwise; nibbles become signed q - 8 bytes per dword
//   Q4_K: a quarter superblock: 32 B of nibbles (sub-blocks 2c and 2c+1) + the 16 B header
//   Q5_K: as Q4_K, plus the superblock's 32 B of fifth bits (bits 2c, 2c+1 of each byte)
//   Q6_K: (half h, column group l0): 16 B ql low, 16 B ql high, 16 B qh + scales + d; the
//         superblock is only 2-byte aligned, so pieces are re-aligned with v_alignbyte.
// Each lane issues the loads of all its units before any arithmetic (clamped
// indices keep every access inside the tensor), so a wave has up to
// UPL x (48..68) bytes in flight per lane — the decode path is HBM-bound.
// Integer sums per block are exact (sdot4 with int32 accumulation); the fp32
// scale products follow vec_dot's form: Q8_0 and Q4_0 I*(dW*dA); Q4_K and Q5_K
// dA*(d*sum sc*I - dmin*sum m*S); Q6_K (dA*d)*sum sc*I. Lanes reduce with shuffles (DPP).
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

enum GemvFmt {
    kQ8_0Pair = 0,
    kQ8_0Single = 1,
    kQ4K = 2,
    kQ6K = 3,
    kQ4_0Pair = 4,
    kQ4_0Single = 5,
    kQ5K = 6,
    kQ8_0RSPair = 7  // row-split Q8_0: two blocks' 64 quants and their two scales
};

// int32 block sums per row (the DUMP layout)
__host__ __device__ constexpr int64_t sums_per_row(int f, int64_t K) {
    return (f == kQ4K || f == kQ5K) ? 2 * (K / 256) : f == kQ6K ? K / 256 : K / 32;
}

// ---------------------------------------------------------------- raw unit loads
struct RawQ8Pair {
    uint32_t w[17];
};
struct RawQ8Single {
    uint32_t d;
    uint32_t q[8];
};
struct RawQ4K {
    uint4 hdr, q0, q1;
};
struct RawQ6K {
    uint32_t a[4], b[4], h[4], sc[4];
    uint32_t d;
};
struct RawQ4_0Pair {
    uint32_t w[9];
};
struct RawQ8RSPair {
    uint32_t q[16];
    uint32_t d;  // the two fp16 scales
};
struct RawQ4_0Single {
    uint32_t d;
    uint32_t q[4];
};
struct RawQ5K {
    uint4 hdr, h0, h1, q0, q1;
};

template <int F>
struct RawOf;
template <>
struct RawOf<kQ8_0Pair> {
    using T = RawQ8Pair;
};
template <>
struct RawOf<kQ8_0Single> {
    using T = RawQ8Single;
};
template <>
struct RawOf<kQ4K> {
    using T = RawQ4K;
};
template <>
struct RawOf<kQ6K> {
    using T = RawQ6K;
};
template <>
struct RawOf<kQ4_0Pair> {
    using T = RawQ4_0Pair;
};
template <>
struct RawOf<kQ4_0Single> {
    using T = RawQ4_0Single;
};
template <>
struct RawOf<kQ5K> {
    using T = RawQ5K;
};
template <>
struct RawOf<kQ8_0RSPair> {
    using T = RawQ8RSPair;
};

__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ8Pair& r) {
    const uint8_t* p = row + (int64_t)u * 68;
    const U32x4 a = ld4(p), b = ld4(p + 16), c = ld4(p + 32), d = ld4(p + 48);
    r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    r.w[8] = c.x; r.w[9] = c.y; r.w[10] = c.z; r.w[11] = c.w;
    r.w[12] = d.x; r.w[13] = d.y; r.w[14] = d.z; r.w[15] = d.w;
    r.w[16] = ld1(p + 64);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ8Single& r) {
    // one 34-byte block at 2-byte alignment: 17 halfword loads, never outside the block
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row + (int64_t)u * 34);
    r.d = p[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) r.q[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ4K& r) {
    const uint8_t* sb = row + (int64_t)(u >> 2) * 144;
    const int c = u & 3;
    r.hdr = ld16(sb);
    r.q0 = ld16(sb + 16 + 32 * c);
    r.q1 = ld16(sb + 32 + 32 * c);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ4_0Pair& r) {
    const uint8_t* p = row + (int64_t)u * 36;
    const U32x4 a = ld4(p), b = ld4(p + 16);
    r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    r.w[8] = ld1(p + 32);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ4_0Single& r) {
    // one 18-byte block at 2-byte alignment: 9 halfword loads, never outside the block
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row + (int64_t)u * 18);
    r.d = p[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) r.q[i] = (uint32_t)p[1 + 2 * i] | ((uint32_t)p[2 + 2 * i] << 16);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ5K& r) {
    const uint8_t* sb = row + (int64_t)(u >> 2) * 176;
    const int c = u & 3;
    r.hdr = ld16(sb);
    r.h0 = ld16(sb + 16);
    r.h1 = ld16(sb + 32);
    r.q0 = ld16(sb + 48 + 32 * c);
    r.q1 = ld16(sb + 64 + 32 * c);
}
__device__ __forceinline__ void load_unit(const uint8_t* row, int u, RawQ6K& r) {
    const uint8_t* sb = row + (int64_t)(u >> 2) * 210;
    const int q = u & 3, h = q >> 1, l0 = (q & 1) * 16;
    ld16_a2(sb + 64 * h + l0, r.a);
    ld16_a2(sb + 64 * h + 32 + l0, r.b);
    ld16_a2(sb + 128 + 32 * h + l0, r.h);
    ld16_a2(sb + 192, r.sc);
    r.d = ldu16(sb + 208);
}

// ---------------------------------------------------------------- per-unit math
// Returns the fp32 contribution of unit u for activation row m; when DUMP, adds the
// unit's integer block sums into sums_row (int32 per block of this (m, n)).
template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ8Pair& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t*, int32_t* sums_row,
                                          bool valid) {
    const uint4 a0 = ld16(xrow + 64 * u), a1 = ld16(xrow + 64 * u + 16);
    const uint4 a2 = ld16(xrow + 64 * u + 32), a3 = ld16(xrow + 64 * u + 48);
    const float dA0 = xd[(int64_t)(2 * u) * m_ld + m], dA1 = xd[(int64_t)(2 * u + 1) * m_ld + m];
    const uint32_t* w = r.w;
    int i0 = 0, i1 = 0;
    i0 = sdot4((int)align_bytes(w[1], w[0], 2), (int)a0.x, i0);
    i0 = sdot4((int)align_bytes(w[2], w[1], 2), (int)a0.y, i0);
    i0 = sdot4((int)align_bytes(w[3], w[2], 2), (int)a0.z, i0);
    i0 = sdot4((int)align_bytes(w[4], w[3], 2), (int)a0.w, i0);
    i0 = sdot4((int)align_bytes(w[5], w[4], 2), (int)a1.x, i0);
    i0 = sdot4((int)align_bytes(w[6], w[5], 2), (int)a1.y, i0);
    i0 = sdot4((int)align_bytes(w[7], w[6], 2), (int)a1.z, i0);
    i0 = sdot4((int)align_bytes(w[8], w[7], 2), (int)a1.w, i0);
    i1 = sdot4((int)w[9], (int)a2.x, i1);
    i1 = sdot4((int)w[10], (int)a2.y, i1);
    i1 = sdot4((int)w[11], (int)a2.z, i1);
    i1 = sdot4((int)w[12], (int)a2.w, i1);
    i1 = sdot4((int)w[13], (int)a3.x, i1);
    i1 = sdot4((int)w[14], (int)a3.y, i1);
    i1 = sdot4((int)w[15], (int)a3.z, i1);
    i1 = sdot4((int)w[16], (int)a3.w, i1);
    const float dW0 = half_bits_to_float(w[0] & 0xFFFFu), dW1 = half_bits_to_float(w[8] >> 16);
    if (DUMP && valid) {
        atomicAdd(sums_row + 2 * u, i0);
        atomicAdd(sums_row + 2 * u + 1, i1);
    }
    return fmaf((float)i1, dW1 * dA1, (float)i0 * (dW0 * dA0));
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ8RSPair& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t*, int32_t* sums_row,
                                          bool valid) {
    const uint4 a0 = ld16(xrow + 64 * u), a1 = ld16(xrow + 64 * u + 16);
    const uint4 a2 = ld16(xrow + 64 * u + 32), a3 = ld16(xrow + 64 * u + 48);
    const float dA0 = xd[(int64_t)(2 * u) * m_ld + m], dA1 = xd[(int64_t)(2 * u + 1) * m_ld + m];
    const uint32_t a[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                            a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
    int i0 = 0, i1 = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        i0 = sdot4((int)r.q[k], (int)a[k], i0);
        i1 = sdot4((int)r.q[8 + k], (int)a[8 + k], i1);
    }
    const float dW0 = half_bits_to_float(r.d & 0xFFFFu), dW1 = half_bits_to_float(r.d >> 16);
    if (DUMP && valid) {
        atomicAdd(sums_row + 2 * u, i0);
        atomicAdd(sums_row + 2 * u + 1, i1);
    }
    return fmaf((float)i1, dW1 * dA1, (float)i0 * (dW0 * dA0));
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ8Single& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t*, int32_t* sums_row,
                                          bool valid) {
    const uint4 a0 = ld16(xrow + 32 * u), a1 = ld16(xrow + 32 * u + 16);
    const float dA = xd[(int64_t)u * m_ld + m];
    int i0 = 0;
    i0 = sdot4((int)r.q[0], (int)a0.x, i0);
    i0 = sdot4((int)r.q[1], (int)a0.y, i0);
    i0 = sdot4((int)r.q[2], (int)a0.z, i0);
    i0 = sdot4((int)r.q[3], (int)a0.w, i0);
    i0 = sdot4((int)r.q[4], (int)a1.x, i0);
    i0 = sdot4((int)r.q[5], (int)a1.y, i0);
    i0 = sdot4((int)r.q[6], (int)a1.z, i0);
    i0 = sdot4((int)r.q[7], (int)a1.w, i0);
    if (DUMP && valid) atomicAdd(sums_row + u, i0);
    return (float)i0 * (half_bits_to_float(r.d) * dA);
}

// The scale step of a Q4_K / Q5_K quarter superblock c of superblock s (the two headers are the
// same 16 bytes): i0, i1 are the integer sums of sub-blocks 2c, 2c + 1, bsv the activation's
// four 16-element sums of those sub-blocks. Returns dA * (d * (sc0 i0 + sc1 i1) - dmin * (m0 S0 +
// m1 S1)).
template <bool DUMP>
__device__ __forceinline__ float kq_quarter_finish(const uint4& hdr, int s, int c, uint2 bsv, float dA, int i0,
                                                   int i1, int32_t* sums_row, bool valid) {
    // 6-bit scales / mins of sub-blocks j = 2c, 2c+1 (all eight unpacked SWAR-style)
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, mn_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const uint32_t scw = c < 2 ? sc_lo : sc_hi, mnw = c < 2 ? mn_lo : mn_hi;
    const uint32_t sh = (uint32_t)(c & 1) * 16u;
    const int sc0 = (int)((scw >> sh) & 0xFFu), sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    const int m0 = (int)((mnw >> sh) & 0xFFu), m1 = (int)((mnw >> (sh + 8)) & 0xFFu);
    const int S0 = (int)(int16_t)(bsv.x & 0xFFFFu) + (int)(int16_t)(bsv.x >> 16);
    const int S1 = (int)(int16_t)(bsv.y & 0xFFFFu) + (int)(int16_t)(bsv.y >> 16);
    const int iA = sc0 * i0 + sc1 * i1;
    const int iB = m0 * S0 + m1 * S1;
    if (DUMP && valid) {
        atomicAdd(sums_row + 2 * s, iA);
        atomicAdd(sums_row + 2 * s + 1, iB);
    }
    const float d = half_bits_to_float(hdr.x & 0xFFFFu), dmin = half_bits_to_float(hdr.x >> 16);
    return dA * fmaf(-dmin, (float)iB, d * (float)iA);
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ4K& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t* xbs_row, int32_t* sums_row,
                                          bool valid) {
    const int s = u >> 2, c = u & 3;
    const int8_t* ap = xrow + 256 * s + 64 * c;
    const uint4 a0 = ld16(ap), a1 = ld16(ap + 16), a2 = ld16(ap + 32), a3 = ld16(ap + 48);
    const uint2 bsv = *reinterpret_cast<const uint2*>(xbs_row + 16 * s + 4 * c);
    const float dA = xd[(int64_t)s * m_ld + m];
    const uint32_t lo = 0x0F0F0F0Fu;
    int i0 = 0, i1 = 0;
    i0 = sdot4((int)(r.q0.x & lo), (int)a0.x, i0);
    i0 = sdot4((int)(r.q0.y & lo), (int)a0.y, i0);
    i0 = sdot4((int)(r.q0.z & lo), (int)a0.z, i0);
    i0 = sdot4((int)(r.q0.w & lo), (int)a0.w, i0);
    i0 = sdot4((int)(r.q1.x & lo), (int)a1.x, i0);
    i0 = sdot4((int)(r.q1.y & lo), (int)a1.y, i0);
    i0 = sdot4((int)(r.q1.z & lo), (int)a1.z, i0);
    i0 = sdot4((int)(r.q1.w & lo), (int)a1.w, i0);
    i1 = sdot4((int)((r.q0.x >> 4) & lo), (int)a2.x, i1);
    i1 = sdot4((int)((r.q0.y >> 4) & lo), (int)a2.y, i1);
    i1 = sdot4((int)((r.q0.z >> 4) & lo), (int)a2.z, i1);
    i1 = sdot4((int)((r.q0.w >> 4) & lo), (int)a2.w, i1);
    i1 = sdot4((int)((r.q1.x >> 4) & lo), (int)a3.x, i1);
    i1 = sdot4((int)((r.q1.y >> 4) & lo), (int)a3.y, i1);
    i1 = sdot4((int)((r.q1.z >> 4) & lo), (int)a3.z, i1);
    i1 = sdot4((int)((r.q1.w >> 4) & lo), (int)a3.w, i1);
    return kq_quarter_finish<DUMP>(r.hdr, s, c, bsv, dA, i0, i1, sums_row, valid);
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ5K& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t* xbs_row, int32_t* sums_row,
                                          bool valid) {
    const int s = u >> 2, c = u & 3;
    const int8_t* ap = xrow + 256 * s + 64 * c;
    const uint4 a0 = ld16(ap), a1 = ld16(ap + 16), a2 = ld16(ap + 32), a3 = ld16(ap + 48);
    const uint2 bsv = *reinterpret_cast<const uint2*>(xbs_row + 16 * s + 4 * c);
    const float dA = xd[(int64_t)s * m_ld + m];
    // sub-block 2c: low nibbles with qh bit 2c; sub-block 2c + 1: high nibbles with bit 2c + 1
    const uint32_t b0 = 2u * (uint32_t)c, b1 = b0 + 1u;
    int i0 = 0, i1 = 0;
    i0 = sdot4((int)q5_levels(r.q0.x, r.h0.x, b0), (int)a0.x, i0);
    i0 = sdot4((int)q5_levels(r.q0.y, r.h0.y, b0), (int)a0.y, i0);
    i0 = sdot4((int)q5_levels(r.q0.z, r.h0.z, b0), (int)a0.z, i0);
    i0 = sdot4((int)q5_levels(r.q0.w, r.h0.w, b0), (int)a0.w, i0);
    i0 = sdot4((int)q5_levels(r.q1.x, r.h1.x, b0), (int)a1.x, i0);
    i0 = sdot4((int)q5_levels(r.q1.y, r.h1.y, b0), (int)a1.y, i0);
    i0 = sdot4((int)q5_levels(r.q1.z, r.h1.z, b0), (int)a1.z, i0);
    i0 = sdot4((int)q5_levels(r.q1.w, r.h1.w, b0), (int)a1.w, i0);
    i1 = sdot4((int)q5_levels(r.q0.x >> 4, r.h0.x, b1), (int)a2.x, i1);
    i1 = sdot4((int)q5_levels(r.q0.y >> 4, r.h0.y, b1), (int)a2.y, i1);
    i1 = sdot4((int)q5_levels(r.q0.z >> 4, r.h0.z, b1), (int)a2.z, i1);
    i1 = sdot4((int)q5_levels(r.q0.w >> 4, r.h0.w, b1), (int)a2.w, i1);
    i1 = sdot4((int)q5_levels(r.q1.x >> 4, r.h1.x, b1), (int)a3.x, i1);
    i1 = sdot4((int)q5_levels(r.q1.y >> 4, r.h1.y, b1), (int)a3.y, i1);
    i1 = sdot4((int)q5_levels(r.q1.z >> 4, r.h1.z, b1), (int)a3.z, i1);
    i1 = sdot4((int)q5_levels(r.q1.w >> 4, r.h1.w, b1), (int)a3.w, i1);
    return kq_quarter_finish<DUMP>(r.hdr, s, c, bsv, dA, i0, i1, sums_row, valid);
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ4_0Pair& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t*, int32_t* sums_row,
                                          bool valid) {
    const uint4 a0 = ld16(xrow + 64 * u), a1 = ld16(xrow + 64 * u + 16);
    const uint4 a2 = ld16(xrow + 64 * u + 32), a3 = ld16(xrow + 64 * u + 48);
    const float dA0 = xd[(int64_t)(2 * u) * m_ld + m], dA1 = xd[(int64_t)(2 * u + 1) * m_ld + m];
    int i0, i1;
    float dW0, dW1;
    q4_0_pair(r.w, a0, a1, a2, a3, i0, i1, dW0, dW1);
    if (DUMP && valid) {
        atomicAdd(sums_row + 2 * u, i0);
        atomicAdd(sums_row + 2 * u + 1, i1);
    }
    return fmaf((float)i1, dW1 * dA1, (float)i0 * (dW0 * dA0));
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ4_0Single& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t*, int32_t* sums_row,
                                          bool valid) {
    const uint4 a0 = ld16(xrow + 32 * u), a1 = ld16(xrow + 32 * u + 16);
    const float dA = xd[(int64_t)u * m_ld + m];
    const int i0 = q4_0_block_dot(r.q, a0, a1);
    if (DUMP && valid) atomicAdd(sums_row + u, i0);
    return (float)i0 * (half_bits_to_float(r.d) * dA);
}

template <bool DUMP>
__device__ __forceinline__ float unit_dot(const RawQ6K& r, int u, const int8_t* xrow, const float* xd,
                                          int64_t m_ld, int64_t m, const int16_t* xbs_row, int32_t* sums_row,
                                          bool valid) {
    const int s = u >> 2, q = u & 3, h = q >> 1, l0 = (q & 1) * 16;
    const int8_t* ap = xrow + 256 * s + 128 * h + l0;
    const uint4 a0 = ld16(ap), a1 = ld16(ap + 32), a2 = ld16(ap + 64), a3 = ld16(ap + 96);
    const uint4 bsv = ld16(xbs_row + 16 * s + 8 * h);  // bsums of groups 8h .. 8h+7
    const float dA = xd[(int64_t)s * m_ld + m];
    const uint32_t lo = 0x0F0F0F0Fu, hb = 0x30303030u;
    int it[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t A = r.a[i], B = r.b[i], Q = r.h[i];
        const uint32_t q0 = (A & lo) | ((Q << 4) & hb);
        const uint32_t q1 = (B & lo) | ((Q << 2) & hb);
        const uint32_t q2 = ((A >> 4) & lo) | (Q & hb);
        const uint32_t q3 = ((B >> 4) & lo) | ((Q >> 2) & hb);
        const uint32_t x0 = i == 0 ? a0.x : i == 1 ? a0.y : i == 2 ? a0.z : a0.w;
        const uint32_t x1 = i == 0 ? a1.x : i == 1 ? a1.y : i == 2 ? a1.z : a1.w;
        const uint32_t x2 = i == 0 ? a2.x : i == 1 ? a2.y : i == 2 ? a2.z : a2.w;
        const uint32_t x3 = i == 0 ? a3.x : i == 1 ? a3.y : i == 2 ? a3.z : a3.w;
        it[0] = sdot4((int)q0, (int)x0, it[0]);
        it[1] = sdot4((int)q1, (int)x1, it[1]);
        it[2] = sdot4((int)q2, (int)x2, it[2]);
        it[3] = sdot4((int)q3, (int)x3, it[3]);
    }
    // (q6 - 32) * q8 summed = q6 * q8 summed - 32 * bsum of the 16-group
    const uint32_t bsel = (uint32_t)(l0 >> 4) * 16u;
    const int b0 = (int)(int16_t)(bsv.x >> bsel), b1 = (int)(int16_t)(bsv.y >> bsel);
    const int b2 = (int)(int16_t)(bsv.z >> bsel), b3 = (int)(int16_t)(bsv.w >> bsel);
    const uint32_t sclo = h ? r.sc[2] : r.sc[0], schi = h ? r.sc[3] : r.sc[1];
    const uint32_t s8 = (uint32_t)(l0 >> 4) * 8u;
    const int sc0 = (int)(int8_t)(sclo >> s8), sc1 = (int)(int8_t)(sclo >> (16 + s8));
    const int sc2 = (int)(int8_t)(schi >> s8), sc3 = (int)(int8_t)(schi >> (16 + s8));
    const int C = sc0 * (it[0] - 32 * b0) + sc1 * (it[1] - 32 * b1) + sc2 * (it[2] - 32 * b2) +
                  sc3 * (it[3] - 32 * b3);
    if (DUMP && valid) atomicAdd(sums_row + s, C);
    return (float)C * (dA * half_bits_to_float(r.d));
}

// ---------------------------------------------------------------- the kernel
// Grid: x over groups of 4 waves; each wave owns 64/G rows (G = 1 << lg), each row G lanes.
// Units of a row: u = g + G*t (t < UPL per pass, passes until all U units are done).
template <int F, int MT, int UPL, bool DUMP>
__global__ void __launch_bounds__(256) gemv_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes, int64_t n0,
                                                   int64_t n1, int K, const int8_t* __restrict__ xqs,
                                                   const float* __restrict__ xd, const int16_t* __restrict__ xbs,
                                                   int64_t m_ld, int M, float* __restrict__ Y, int64_t y_stride,
                                                   int32_t* __restrict__ sums, int64_t sums_n_stride, int lg) {
    using Raw = typename RawOf<F>::T;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = 1 << lg;
    const int g = lane & (G - 1);
    const int64_t row = n0 + ((int64_t)blockIdx.x * 4 + wave) * (64 >> lg) + (lane >> lg);
    const bool row_ok = row < n1;
    const int64_t rowc = row_ok ? row : n1 - 1;
    const uint8_t* wrow = W + rowc * w_row_bytes;
    const int U = (F == kQ8_0Single || F == kQ4_0Single) ? K / 32 : K / 64;
    const int64_t per_row_sums = sums_per_row(F, K);

    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;

    for (int u0 = 0; u0 < U; u0 += G * UPL) {
        Raw raw[UPL];
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = u0 + g + t * G;
            const int uc = u < U ? u : U - 1;
            if constexpr (F == kQ8_0RSPair) {
                // the pair's 64 quants at row + 64u (16-byte aligned), its two scales at row + K + 4u
                const uint8_t* p = wrow + (int64_t)uc * 64;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const U32x4 v = ld4(p + 16 * i);
                    raw[t].q[4 * i] = v.x, raw[t].q[4 * i + 1] = v.y, raw[t].q[4 * i + 2] = v.z, raw[t].q[4 * i + 3] = v.w;
                }
                raw[t].d = ld1(wrow + K + (int64_t)uc * 4);
            } else {
                load_unit(wrow, uc, raw[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
            const int u = u0 + g + t * G;
            const bool valid = u < U && row_ok;
            const int uc = u < U ? u : U - 1;
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                const int64_t m = mi < M ? mi : M - 1;
                int32_t* srow = DUMP ? sums + (m * sums_n_stride + (rowc - n0)) * per_row_sums : nullptr;
                const float v = unit_dot<DUMP>(raw[t], uc, xqs + m * (int64_t)K, xd, m_ld, m,
                                               xbs ? xbs + m * (int64_t)(K / 16) : nullptr, srow,
                                               valid && mi < M);
                acc[mi] += valid ? v : 0.0f;
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        float v = acc[mi];
        for (int o = G >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        acc[mi] = v;
    }
    if (g == 0 && row_ok) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
            if (mi < M) Y[(int64_t)mi * y_stride + (row - n0)] = acc[mi];
    }
}

// ---------------------------------------------------------------- dispatch
using GemvFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, int, const int8_t*, const float*, const int16_t*,
                        int64_t, int, float*, int64_t, int32_t*, int64_t, int);

template <int F, int MT, bool DUMP>
static GemvFn pick_upl(int upl) {
    if (MT == 1) {
        if (upl >= 4) return gemv_kernel<F, MT, 4, DUMP>;
        if (upl == 3) return gemv_kernel<F, MT, 3, DUMP>;
        if (upl == 2) return gemv_kernel<F, MT, 2, DUMP>;
        return gemv_kernel<F, MT, 1, DUMP>;
    }
    if (MT == 2) {
        if (upl >= 2) return gemv_kernel<F, MT, 2, DUMP>;
        return gemv_kernel<F, MT, 1, DUMP>;
    }
    return gemv_kernel<F, MT, 1, DUMP>;
}

template <int F, bool DUMP>
static GemvFn pick_mt(int mt, int upl) {
    switch (mt) {
        case 1: return pick_upl<F, 1, DUMP>(upl);
        case 2: return pick_upl<F, 2, DUMP>(upl);
        case 4: return pick_upl<F, 4, DUMP>(upl);
        default: return pick_upl<F, 8, DUMP>(upl);
    }
}

template <bool DUMP>
static GemvFn pick_fmt(int f, int mt, int upl) {
    switch (f) {
        case kQ8_0Pair: return pick_mt<kQ8_0Pair, DUMP>(mt, upl);
        case kQ8_0Single: return pick_mt<kQ8_0Single, DUMP>(mt, upl);
        case kQ4K: return pick_mt<kQ4K, DUMP>(mt, upl);
        case kQ4_0Pair: return pick_mt<kQ4_0Pair, DUMP>(mt, upl);
        case kQ4_0Single: return pick_mt<kQ4_0Single, DUMP>(mt, upl);
        case kQ5K: return pick_mt<kQ5K, DUMP>(mt, upl);
        case kQ8_0RSPair: return pick_mt<kQ8_0RSPair, DUMP>(mt, upl);
        default: return pick_mt<kQ6K, DUMP>(mt, upl);
    }
}


hipError_t launch_gemv(int wtype, const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                       const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                       int64_t sums_n_stride, hipStream_t st, const float* R, int64_t r_stride) {
    // Q6_K: weight rows staged through LDS by coalesced direct-to-LDS loads (its 2-byte aligned
    // superblocks make lane-direct loads scatter: 4x the L1 accesses of the staged form);
    // DCQ_Q6K_DECODE=1 selects the lane-direct four-lanes-per-superblock kernel instead
    if (knob(Knob::GemvGeneric) == 0) {
        hipError_t e = hipErrorNotSupported;
        if (wtype == kTypeQ4_K || wtype == kTypeQ5_K || (wtype == kTypeQ6_K && knob(Knob::Q6KDecode)))
            e = launch_decode_kq(wtype, W, w_row_bytes, n0, n1, K, act, M, Y, y_stride, block_sums, sums_n_stride,
                                 st, R, r_stride);
        else if (wtype == kTypeQ6_K)
            e = launch_decode_q6k_lds(W, w_row_bytes, n0, n1, K, act, M, Y, y_stride, block_sums, sums_n_stride,
                                      st, R, r_stride);
        if (e != hipErrorNotSupported) return e;
    }
    if (R) return hipErrorNotSupported;  // the generic kernels have no add in their store
    int f;
    const bool pairs = K % 64 == 0 && w_row_bytes % 4 == 0;  // two 32-blocks per unit, dword aligned
    if (wtype == kTypeQ8_0_RS) {
        if (K % 64 || w_row_bytes % 16) return hipErrorNotSupported;
        f = kQ8_0RSPair;
    } else if (wtype == kTypeQ8_0)
        f = pairs ? kQ8_0Pair : kQ8_0Single;
    else if (wtype == kTypeQ4_0)
        f = pairs ? kQ4_0Pair : kQ4_0Single;
    else if (wtype == kTypeQ4_K)
        f = kQ4K;
    else if (wtype == kTypeQ5_K)
        f = kQ5K;
    else
        f = kQ6K;
    const int U = (f == kQ8_0Single || f == kQ4_0Single) ? (int)(K / 32) : (int)(K / 64);
    // lanes per row: smallest power of two covering the row's units (capped at a wave)
    int lg = 0;
    while ((1 << lg) < U && lg < 6) ++lg;
    if (knob(Knob::GemvLanes) >= 0) lg = knob(Knob::GemvLanes);
    const int G = 1 << lg;
    const int64_t rows = n1 - n0;
    const int64_t rows_per_block = 4 * (64 / G);
    const unsigned grid = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
    const int64_t per_row_sums = sums_per_row(f, K);
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const int upl_max = (U + G - 1) / G;
        const int upl = mt == 1 ? (upl_max > 4 ? 4 : upl_max) : mt == 2 ? (upl_max > 2 ? 2 : upl_max) : 1;
        GemvFn fn = block_sums ? pick_fmt<true>(f, mt, upl) : pick_fmt<false>(f, mt, upl);
        hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, st, (const uint8_t*)W, w_row_bytes, n0, n1, (int)K,
                           act.qs + m0 * K, act.d + m0, act.bs ? act.bs + m0 * (K / 16) : nullptr, act.m_ld,
                           (int)mc, Y + m0 * y_stride, y_stride,
                           block_sums ? block_sums + m0 * sums_n_stride * per_row_sums : nullptr, sums_n_stride,
                           lg);
    }
    return hipGetLastError();
}

}  // namespace dcq
