// dcq_mmq.hip — quantized mul_mat on gfx950 int8 MFMA (prefill / batched decode).
//
// Replaces ggml's CPU MUL_MAT at M > 1 (core/src/inference.cpp:1049-1063 routes
// every M > 1 projection there; executed at core/src/worker.cpp:544).
//
// Tiling. MFMA v_mfma_i32_32x32x32_i8 (Q8_0, Q4_0, Q4_K, Q5_K) / v_mfma_i32_32x32x16_i8
// (Q6_K, whose scales are per 16 elements). Operand roles: A = activations
// (MFMA rows = m), B = weights (MFMA columns = n), so every lane of the 32x32
// result owns ONE weight row n = lane % 32 and 16 activation rows
// m_v = 8*(v/4) + 4*(lane/32) + v%4; weight scales are lane-local and the
// activation scales for 4 consecutive m_v load as one float4 (the planar
// activation scales are stored block-major, [block][m]).
// A wave owns TM x TN such tiles (32*TM rows of m, 32*TN rows of n); a
// 4-wave workgroup spreads WN waves along n and WK waves along K (interleaved
// K steps, deterministic fixed-order reduction through LDS at the end).
// Operands are loaded straight from global memory into registers in MFMA
// layout (activation rows are 16-B aligned; Q8_0 / Q6_K weight bytes are
// 2-B aligned and re-aligned with v_alignbyte); the next K step is loaded
// before the current one is consumed.
//
// Per-block scales (exact integers first, fp32 last):
//   Q8_0: the MFMA accumulates on top of the constant 0x4B400000, so its int32
//     result read as fp32 is 12582912 + I exactly (|I| <= 32*127*128 < 2^22);
//     t = fma(F, dW, -dW*12582912) is then dW*I rounded once, and
//     acc = fma(t, dA, acc): two VALU ops per output per 32-block.
//   Q4_0: the same, on the nibbles turned into signed q - 8 bytes as they are loaded
//     (|I| <= 32*8*128 < 2^22 as well).
//   Q4_K: acc_i += sc_j * I_j (v_mad_i32_i24) per 32-sub-block; the mins term
//     sum_j m_j * S_j runs on the MFMA against a weight operand whose bytes all
//     equal m_j; per superblock acc += dA * (d * acc_i - dmin * acc_min).
//     The 2 x 2-tile form (large M), VALU-bound that way, moves both onto the MFMA:
//     sum_j sc_j I_j as two accumulations over the sub-blocks against the nibbles
//     times sc_hi and sc_lo (sc = 8 sc_hi + sc_lo, each <= 7: every product fits
//     int8), and sum_j m_j S_j from the activation's 16-element sums: S_j = 64 hi_j +
//     lo_j (lo_j in [0, 63], hi_j in [-64, 63]) as int8 bytes against the bytes m_j,
//     two MFMAs per tile per superblock instead of eight.
//   Q5_K: the Q4_K steps on the 5-bit levels (nibble plus the qh bit). Levels up to 31 times
//     sc_hi up to 7 do not fit int8, so Q5_K always takes the per-sub-block form.
//   Q6_K: acc_i += sc_g * I_g per 16-group (signed q - 32 operands); per
//     superblock acc += dA * d * acc_i.
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr int kMagic = 0x4B400000;  // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16i mfma32k16(long a, long b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4i as_v4i(uint4 u) {
    v4i r;
    r.x = (int)u.x;
    r.y = (int)u.y;
    r.z = (int)u.z;
    r.w = (int)u.w;
    return r;
}
// 8 bytes at a 2-byte aligned address: 3 dwords from the dword below, never past p + 10.
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint32_t* b = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t w0 = b[0], w1 = b[1], w2 = b[sh ? 2 : 1];
    return make_uint2(align_bytes(w1, w0, sh), align_bytes(w2, w1, sh));
}
// signed (q6 - 32) bytes from unsigned 6-bit bytes, per byte without borrows
__device__ __forceinline__ uint32_t minus32(uint32_t q) {
    return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

// Activation scales of the 16 rows m_v of a 32-row m-subtile for one block.
__device__ __forceinline__ void load_dA(const float* xd_blk, int64_t mbase, int hl, float out[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(xd_blk + mbase + 8 * q + 4 * hl);
        out[4 * q + 0] = v.x;
        out[4 * q + 1] = v.y;
        out[4 * q + 2] = v.z;
        out[4 * q + 3] = v.w;
    }
}

template <int TM, int TN>
struct Acc {
    float v[TM][TN][16];
};

// Fixed-order reduction of WK partial tiles through LDS; returns true on the wave that stores.
template <int TM, int TN, int WK>
__device__ __forceinline__ bool reduce_k(Acc<TM, TN>& acc, float* lds, int wn, int wk, int lane) {
    if (WK == 1) return true;
    constexpr int per_wave = TM * TN * 16 * 64;
    // waves wk > 0 publish, wave 0 adds in wk order
    if (wk > 0) {
        float* dst = lds + ((wn * (WK - 1)) + (wk - 1)) * per_wave;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) dst[((i * TN + j) * 16 + v) * 64 + lane] = acc.v[i][j][v];
    }
    __syncthreads();
    if (wk > 0) return false;
    for (int w = 1; w < WK; ++w) {
        const float* src = lds + ((wn * (WK - 1)) + (w - 1)) * per_wave;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc.v[i][j][v] += src[((i * TN + j) * 16 + v) * 64 + lane];
    }
    return true;
}

template <int TM, int TN>
__device__ __forceinline__ void store_tile(const Acc<TM, TN>& acc, float* Y, int64_t y_stride, int64_t M, int64_t N,
                                           int64_t mbase, int64_t nbase, int lane) {
    const int hl = lane >> 5, col = lane & 31;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t n = nbase + 32 * j + col;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t m = mbase + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (m < M) Y[m * y_stride + n] = acc.v[i][j][v];
            }
    }
}

// ============================================================== Q8_0
template <int TM, int TN>
struct Q8Step {
    uint4 a[TM];
    uint32_t b[TN][4];
    uint32_t dw[TN];
};

// Q40: the weight blocks are Q4_0 (18 B): lane half hl takes the low (hl = 0) or high nibbles of
// the block's 16 bytes, i.e. its elements 16 hl .. 16 hl + 15, as signed q - 8 bytes.
template <int TM, int TN, bool Q40>
__device__ __forceinline__ void q8_load(Q8Step<TM, TN>& s, const int8_t* const* arow, const uint8_t* const* wrow,
                                        int kb, int hl) {
#pragma unroll
    for (int i = 0; i < TM; ++i) s.a[i] = ld16(arow[i] + 32 * kb + 16 * hl);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        if constexpr (Q40) {
            const uint8_t* blk = wrow[j] + 18 * (int64_t)kb;
            uint32_t raw[4];
            ld16_a2(blk + 2, raw);
            const uint32_t sh = 4u * (uint32_t)hl;
#pragma unroll
            for (int e = 0; e < 4; ++e) s.b[j][e] = minus8((raw[e] >> sh) & 0x0F0F0F0Fu);
            s.dw[j] = ldu16(blk);
        } else {
            const uint8_t* blk = wrow[j] + 34 * (int64_t)kb;
            ld16_a2(blk + 2 + 16 * hl, s.b[j]);
            s.dw[j] = ldu16(blk);
        }
    }
}

template <int TM, int TN, int WN, int WK, bool DUMP, bool Q40>
__global__ void __launch_bounds__(256) mmq_q8_0_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes, int64_t N,
                                                       int64_t K, const int8_t* __restrict__ xqs,
                                                       const float* __restrict__ xd, int64_t m_ld, int64_t M,
                                                       float* __restrict__ Y, int64_t y_stride,
                                                       int32_t* __restrict__ sums, const int16_t* __restrict__ xbs) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % WN, wk = wave / WN;
    const int hl = lane >> 5, col = lane & 31;
    const int64_t mbase = (int64_t)blockIdx.y * (32 * TM);
    const int64_t nbase = (int64_t)blockIdx.x * (32 * TN * WN) + 32 * TN * wn;
    const int nb = (int)(K / 32);

    const int8_t* arow[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        int64_t m = mbase + 32 * i + col;
        m = m < M ? m : M - 1;
        arow[i] = xqs + m * K;
    }
    const uint8_t* wrow[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        int64_t n = nbase + 32 * j + col;
        n = n < N ? n : N - 1;
        wrow[j] = W + n * w_row_bytes;
    }
    v16i cmagic;
#pragma unroll
    for (int v = 0; v < 16; ++v) cmagic[v] = kMagic;

    Acc<TM, TN> acc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc.v[i][j][v] = 0.0f;

    Q8Step<TM, TN> cur, nxt;
    int kb = wk;
    if (kb < nb) q8_load<TM, TN, Q40>(cur, arow, wrow, kb, hl);
    for (; kb < nb; kb += WK) {
        const int kn = kb + WK;
        if (kn < nb) q8_load<TM, TN, Q40>(nxt, arow, wrow, kn, hl);
        const float* xdb = xd + (int64_t)kb * m_ld;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float dA[16];
            load_dA(xdb, mbase + 32 * i, hl, dA);
            const v4i av = as_v4i(cur.a[i]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                v4i bv;
                bv.x = (int)cur.b[j][0];
                bv.y = (int)cur.b[j][1];
                bv.z = (int)cur.b[j][2];
                bv.w = (int)cur.b[j][3];
                const v16i D = mfma32(av, bv, cmagic);
                const float dW = half_bits_to_float(cur.dw[j]);
                const float c = -dW * kMagicF;  // exact: 11-bit mantissa times 3 * 2^22
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float t = fmaf(__int_as_float(D[v]), dW, c);
                    acc.v[i][j][v] = fmaf(t, dA[v], acc.v[i][j][v]);
                }
                if (DUMP) {
                    const int64_t n = nbase + 32 * j + col;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int64_t m = mbase + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                        if (m < M && n < N) atomicAdd(sums + (m * N + n) * nb + kb, D[v] - kMagic);
                    }
                }
            }
        }
        cur = nxt;
    }
    if (reduce_k<TM, TN, WK>(acc, lds, wn, wk, lane)) store_tile<TM, TN>(acc, Y, y_stride, M, N, mbase, nbase, lane);
}

// ============================================================== Q4_K and Q5_K (Q5)
template <int TM, int TN, int WN, int WK, bool DUMP, bool Q5>
__global__ void __launch_bounds__(256) mmq_q4_K_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes, int64_t N,
                                                       int64_t K, const int8_t* __restrict__ xqs,
                                                       const float* __restrict__ xd, int64_t m_ld, int64_t M,
                                                       float* __restrict__ Y, int64_t y_stride,
                                                       int32_t* __restrict__ sums, const int16_t* __restrict__ xbs) {
    constexpr bool kSplit = TM == 2 && TN == 2 && !Q5;  // see the Q4_K / Q5_K notes at the top
    constexpr int kSbBytes = Q5 ? 176 : 144, kQsOff = Q5 ? 48 : 16;
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % WN, wk = wave / WN;
    const int hl = lane >> 5, col = lane & 31;
    const int64_t mbase = (int64_t)blockIdx.y * (32 * TM);
    const int64_t nbase = (int64_t)blockIdx.x * (32 * TN * WN) + 32 * TN * wn;
    const int nsb = (int)(K / 256);

    const int8_t* arow[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        int64_t m = mbase + 32 * i + col;
        m = m < M ? m : M - 1;
        arow[i] = xqs + m * K;
    }
    const uint8_t* wrow[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        int64_t n = nbase + 32 * j + col;
        n = n < N ? n : N - 1;
        wrow[j] = W + n * w_row_bytes;
    }
    Acc<TM, TN> acc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc.v[i][j][v] = 0.0f;

    for (int s = wk; s < nsb; s += WK) {
        // weight fragments of this superblock: header + 4 x 16 B of nibbles per row (Q5_K: and
        // the 16 qh bytes of this lane half's elements l = 16 hl .. 16 hl + 15)
        uint4 hdr[TN], qw[TN][4];
        [[maybe_unused]] uint4 qhw[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint8_t* sb = wrow[j] + kSbBytes * (int64_t)s;
            hdr[j] = ld16(sb);
#pragma unroll
            for (int c = 0; c < 4; ++c) qw[j][c] = ld16(sb + kQsOff + 32 * c + 16 * hl);
            if constexpr (Q5) qhw[j] = ld16(sb + 16 + 16 * hl);
        }
        uint4 qa[TM][8];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int sub = 0; sub < 8; ++sub) qa[i][sub] = ld16(arow[i] + 256 * s + 32 * sub + 16 * hl);

        // 6-bit scales / mins of the lane's weight row (n = lane % 32 of tile j)
        uint32_t scw[TN][2], mnw[TN][2];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t s0 = hdr[j].y, s1 = hdr[j].z, s2 = hdr[j].w;
            scw[j][0] = s0 & 0x3F3F3F3Fu;
            mnw[j][0] = s1 & 0x3F3F3F3Fu;
            scw[j][1] = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
            mnw[j][1] = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        }
        // 2 x 2 tiles: the mins' activation operand of each m-tile (lanes with hl = 0 carry
        // k' 0..15: lo_0..lo_7, hi_0..hi_7 of the superblock's S_j; the others zeros)
        [[maybe_unused]] v4i amop[TM];
        if constexpr (kSplit) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                int64_t m = mbase + 32 * i + col;
                m = m < M ? m : M - 1;
                const uint4* bp = reinterpret_cast<const uint4*>(xbs + m * (K / 16) + 16 * (int64_t)s);
                const uint4 b0 = bp[0], b1 = bp[1];
                const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
                uint32_t lo[2] = {0u, 0u}, hi[2] = {0u, 0u};
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int S = (int)(int16_t)(bw[jj] & 0xFFFFu) + (int)(int16_t)(bw[jj] >> 16);
                    lo[jj >> 2] |= (uint32_t)(S & 63) << (8 * (jj & 3));
                    hi[jj >> 2] |= ((uint32_t)(S >> 6) & 0xFFu) << (8 * (jj & 3));
                }
                amop[i].x = hl ? 0 : (int)lo[0];
                amop[i].y = hl ? 0 : (int)lo[1];
                amop[i].z = hl ? 0 : (int)hi[0];
                amop[i].w = hl ? 0 : (int)hi[1];
            }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            v16i ai[TM], amin[TM];
            if constexpr (kSplit) {
                v16i ahi[TM], alo[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) ahi[i][v] = alo[i][v] = 0;
#pragma unroll
                for (int sub = 0; sub < 8; ++sub) {
                    const uint4 q = qw[j][sub >> 1];
                    const uint32_t sh = (sub & 1) ? 4u : 0u;
                    const int sc = (int)((scw[j][sub >> 2] >> (8 * (sub & 3))) & 0xFFu);
                    const u16x2 s_hi = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
                    const u16x2 s_lo = {(uint16_t)(sc & 7), (uint16_t)(sc & 7)};
                    const uint32_t nib[4] = {(q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu,
                                             (q.z >> sh) & 0x0F0F0F0Fu, (q.w >> sh) & 0x0F0F0F0Fu};
                    v4i bhi, blo;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const u16x2 b = __builtin_bit_cast(u16x2, nib[e]);
                        bhi[e] = __builtin_bit_cast(int, (u16x2)(b * s_hi));
                        blo[e] = __builtin_bit_cast(int, (u16x2)(b * s_lo));
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const v4i av = as_v4i(qa[i][sub]);
                        ahi[i] = mfma32(av, bhi, ahi[i]);
                        alo[i] = mfma32(av, blo, alo[i]);
                    }
                }
                // the mins' weight operands: bytes m_0..m_7 against lo (k' 0..7), then hi (8..15)
                v4i bml, bmh;
                bml.x = hl ? 0 : (int)mnw[j][0];
                bml.y = hl ? 0 : (int)mnw[j][1];
                bml.z = bml.w = 0;
                bmh.x = bmh.y = 0;
                bmh.z = hl ? 0 : (int)mnw[j][0];
                bmh.w = hl ? 0 : (int)mnw[j][1];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    v16i zero;
#pragma unroll
                    for (int v = 0; v < 16; ++v) zero[v] = 0;
                    const v16i ml = mfma32(amop[i], bml, zero);
                    const v16i mh = mfma32(amop[i], bmh, zero);
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        ai[i][v] = (ahi[i][v] << 3) + alo[i][v];
                        amin[i][v] = ml[v] + (mh[v] << 6);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        ai[i][v] = 0;
                        amin[i][v] = 0;
                    }
#pragma unroll
                for (int sub = 0; sub < 8; ++sub) {
                    const uint4 q = qw[j][sub >> 1];
                    const uint32_t sh = (sub & 1) ? 4u : 0u;
                    v4i bv;
                    if constexpr (Q5) {
                        const uint4 h = qhw[j];
                        bv.x = (int)q5_levels(q.x >> sh, h.x, (uint32_t)sub);
                        bv.y = (int)q5_levels(q.y >> sh, h.y, (uint32_t)sub);
                        bv.z = (int)q5_levels(q.z >> sh, h.z, (uint32_t)sub);
                        bv.w = (int)q5_levels(q.w >> sh, h.w, (uint32_t)sub);
                    } else {
                        bv.x = (int)((q.x >> sh) & 0x0F0F0F0Fu);
                        bv.y = (int)((q.y >> sh) & 0x0F0F0F0Fu);
                        bv.z = (int)((q.z >> sh) & 0x0F0F0F0Fu);
                        bv.w = (int)((q.w >> sh) & 0x0F0F0F0Fu);
                    }
                    const int sc = (int)((scw[j][sub >> 2] >> (8 * (sub & 3))) & 0xFFu);
                    const uint32_t mb = ((mnw[j][sub >> 2] >> (8 * (sub & 3))) & 0xFFu) * 0x01010101u;
                    v4i bm;
                    bm.x = bm.y = bm.z = bm.w = (int)mb;
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const v4i av = as_v4i(qa[i][sub]);
                        v16i zero;
#pragma unroll
                        for (int v = 0; v < 16; ++v) zero[v] = 0;
                        const v16i I = mfma32(av, bv, zero);
                        amin[i] = mfma32(av, bm, amin[i]);
#pragma unroll
                        for (int v = 0; v < 16; ++v) ai[i][v] = __mul24(sc, I[v]) + ai[i][v];
                    }
                }
            }
            const float d = half_bits_to_float(hdr[j].x & 0xFFFFu), dmin = half_bits_to_float(hdr[j].x >> 16);
            const float* xds = xd + (int64_t)s * m_ld;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                float dA[16];
                load_dA(xds, mbase + 32 * i, hl, dA);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float y = fmaf(-dmin, (float)amin[i][v], d * (float)ai[i][v]);
                    acc.v[i][j][v] = fmaf(dA[v], y, acc.v[i][j][v]);
                }
                if (DUMP) {
                    const int64_t n = nbase + 32 * j + col;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int64_t m = mbase + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                        if (m < M && n < N) {
                            atomicAdd(sums + (m * N + n) * (2 * nsb) + 2 * s, ai[i][v]);
                            atomicAdd(sums + (m * N + n) * (2 * nsb) + 2 * s + 1, amin[i][v]);
                        }
                    }
                }
            }
        }
    }
    if (reduce_k<TM, TN, WK>(acc, lds, wn, wk, lane)) store_tile<TM, TN>(acc, Y, y_stride, M, N, mbase, nbase, lane);
}

// ============================================================== Q6_K
template <int TM, int TN, int WN, int WK, bool DUMP>
__global__ void __launch_bounds__(256) mmq_q6_K_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes, int64_t N,
                                                       int64_t K, const int8_t* __restrict__ xqs,
                                                       const float* __restrict__ xd, int64_t m_ld, int64_t M,
                                                       float* __restrict__ Y, int64_t y_stride,
                                                       int32_t* __restrict__ sums, const int16_t* __restrict__ xbs) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % WN, wk = wave / WN;
    const int hl = lane >> 5, col = lane & 31;
    const int64_t mbase = (int64_t)blockIdx.y * (32 * TM);
    const int64_t nbase = (int64_t)blockIdx.x * (32 * TN * WN) + 32 * TN * wn;
    const int nsb = (int)(K / 256);

    const int8_t* arow[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        int64_t m = mbase + 32 * i + col;
        m = m < M ? m : M - 1;
        arow[i] = xqs + m * K;
    }
    const uint8_t* wrow[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        int64_t n = nbase + 32 * j + col;
        n = n < N ? n : N - 1;
        wrow[j] = W + n * w_row_bytes;
    }
    Acc<TM, TN> acc;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc.v[i][j][v] = 0.0f;

    for (int s = wk; s < nsb; s += WK) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint8_t* sb = wrow[j] + 210 * (int64_t)s;
            uint32_t scr[4];
            ld16_a2(sb + 192, scr);
            const float d = half_bits_to_float(ldu16(sb + 208));
            v16i ai[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) ai[i][v] = 0;
            // group g = 8h + 2t + gg covers l in 16*gg + [0,16); this lane half takes l in 16*gg + 8*hl + [0,8)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int gg = 0; gg < 2; ++gg) {
                    const int l = 16 * gg + 8 * hl;
                    const uint2 qlA = ld8_a2(sb + 64 * h + l);       // t = 0 (low nibble), t = 2 (high)
                    const uint2 qlB = ld8_a2(sb + 64 * h + 32 + l);  // t = 1 (low), t = 3 (high)
                    const uint2 qh = ld8_a2(sb + 128 + 32 * h + l);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint2 src = (t & 1) ? qlB : qlA;
                        const uint32_t nsh = (t >> 1) ? 4u : 0u;
                        const uint32_t hsh = 2u * (uint32_t)t;
                        const uint32_t q0 = minus32(((src.x >> nsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4));
                        const uint32_t q1 = minus32(((src.y >> nsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4));
                        const long bq = (long)(((uint64_t)q1 << 32) | q0);
                        const int g = 8 * h + 2 * t + gg;
                        const int sc = (int)(int8_t)(scr[g >> 2] >> (8 * (g & 3)));
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
                            const uint2 av = *reinterpret_cast<const uint2*>(arow[i] + 256 * s + 128 * h + 32 * t + l);
                            const long aq = (long)(((uint64_t)av.y << 32) | av.x);
                            v16i zero;
#pragma unroll
                            for (int v = 0; v < 16; ++v) zero[v] = 0;
                            const v16i I = mfma32k16(aq, bq, zero);
#pragma unroll
                            for (int v = 0; v < 16; ++v) ai[i][v] = __mul24(sc, I[v]) + ai[i][v];
                        }
                    }
                }
            }
            const float* xds = xd + (int64_t)s * m_ld;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                float dA[16];
                load_dA(xds, mbase + 32 * i, hl, dA);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc.v[i][j][v] = fmaf(dA[v] * d, (float)ai[i][v], acc.v[i][j][v]);
                if (DUMP) {
                    const int64_t n = nbase + 32 * j + col;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int64_t m = mbase + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                        if (m < M && n < N) atomicAdd(sums + (m * N + n) * nsb + s, ai[i][v]);
                    }
                }
            }
        }
    }
    if (reduce_k<TM, TN, WK>(acc, lds, wn, wk, lane)) store_tile<TM, TN>(acc, Y, y_stride, M, N, mbase, nbase, lane);
}

// ============================================================== dispatch
using MmqFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, const int8_t*, const float*, int64_t, int64_t,
                       float*, int64_t, int32_t*, const int16_t*);

template <int TM, int TN, int WN, int WK, bool DUMP>
static MmqFn pick_fmt(int wtype) {
    if (wtype == kTypeQ8_0) return mmq_q8_0_kernel<TM, TN, WN, WK, DUMP, false>;
    if (wtype == kTypeQ4_0) return mmq_q8_0_kernel<TM, TN, WN, WK, DUMP, true>;
    if (wtype == kTypeQ4_K) return mmq_q4_K_kernel<TM, TN, WN, WK, DUMP, false>;
    if (wtype == kTypeQ5_K) return mmq_q4_K_kernel<TM, TN, WN, WK, DUMP, true>;
    return mmq_q6_K_kernel<TM, TN, WN, WK, DUMP>;
}

struct MmqShape {
    int tm, tn, wn, wk;
};

template <bool DUMP>
static MmqFn pick(int wtype, const MmqShape& s) {
    if (s.tm == 2 && s.tn == 2 && s.wn == 4) return pick_fmt<2, 2, 4, 1, DUMP>(wtype);
    if (s.tm == 2 && s.tn == 1 && s.wk == 4) return pick_fmt<2, 1, 1, 4, DUMP>(wtype);
    if (s.tm == 1 && s.tn == 1 && s.wk == 4) return pick_fmt<1, 1, 1, 4, DUMP>(wtype);
    return pick_fmt<1, 2, 4, 1, DUMP>(wtype);
}

hipError_t launch_mmq(int wtype, const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                      int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                      const SplitScratch& sc) {
    // Q8_0 / Q4_0 / Q6_K past 64 rows: the batch kernel up to 256 rows where its tiles give every CU
    // at most one workgroup and K <= 4096, else the 128 x 128-tile kernels (steps at 80 to 256 rows:
    // batch kernel faster on all 26 such shapes, 2048 x 2048 Q6_K at 128 rows 16.1 -> 9.1 us, Q8_0
    // at 256 rows 22.1 -> 13.9 us; slower past one workgroup per CU, 6144 x 4096 at 128 rows
    // 25.5 -> 33.3 us, and at K >= 8192 from 128 rows)
    const bool batch_past_64 =
        M <= 256 && K <= 4096 && ((N + 31) / 32) * ((M + 63) / 64) <= (int64_t)cu_count();
    // row-split Q8_0: the batched and the 128 x 128-tile kernels (no generic MMQ form)
    if (wtype == kTypeQ8_0_RS) {
        if (M <= 64 || batch_past_64) {
            const hipError_t e = launch_batch_q8_0(kFmtQ8_0RS, W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums,
                                                   st, sc);
            if (e != hipErrorNotSupported) return e;
        }
        return launch_prefill_q8_0(kFmtQ8_0RS, W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums, st, sc);
    }
    const bool q8 = wtype == kTypeQ8_0 || wtype == kTypeQ4_0;  // Q8_0-block kernels
    if (q8 && (M <= 64 || batch_past_64)) {
        const hipError_t e = launch_batch_q8_0(q8_fmt(wtype), W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums, st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    if (wtype == kTypeQ6_K && (M <= 64 || batch_past_64)) {
        const hipError_t e = launch_batch_q6k(W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums, st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    // Q8_0 / Q4_0 / Q6_K at 8 < M <= 32 also take the 128 x 128-tile kernels when the MMQ kernel's
    // 32 x 32 tiles would leave most CUs idle and the workspace has room to split K (Q8_0 2048 x 8192
    // at M = 16: 70 -> 25 us)
    const bool starved = (M + 31) / 32 * ((N + 31) / 32) < cu_count() / 2 && (q8 || wtype == kTypeQ6_K) &&
                         plan_split_k(((M + 127) / 128) * ((N + 127) / 128), (int)(K / 128), q8 ? 1 : 2, M, N,
                                      sc).splits > 1;
    if (q8 && (M > 32 || starved)) {
        const hipError_t e = launch_prefill_q8_0(q8_fmt(wtype), W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums,
                                                 st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    if (wtype == kTypeQ6_K && (M > 32 || starved)) {
        const hipError_t e = launch_prefill_q6_k(W, w_row_bytes, N, K, act, M, Y, y_stride, block_sums, st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    // Q4_K / Q5_K: the batch kernel (64-row m-tiles) up to 256 rows, and up to 512 while the
    // prefill kernel's 128 x 128 tiles would not give every CU one (steps: 192 x 8192 x 2048 19.9
    // against 27.8 us on the prefill kernel, 512 x 2048 x 8192 37.5 against 47.4 us, 384 x 8192 x
    // 2048 36.5 against 39.1 us; but 512 x 8192 x 2048, 256 prefill tiles, 46.3 against 40.6 us, and
    // from 768 rows the prefill kernel)
    const bool q4_batch =
        M <= 256 || (M <= 512 && ((M + 127) / 128) * ((N + 127) / 128) < (int64_t)cu_count());
    if ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && !q4_batch) {
        const hipError_t e = launch_prefill_q4_k(wtype == kTypeQ5_K, W, w_row_bytes, N, K, act, M, Y, y_stride,
                                                 block_sums, st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    if ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && q4_batch) {
        const hipError_t e = launch_batch_q4k(wtype == kTypeQ5_K, W, w_row_bytes, N, K, act, M, Y, y_stride,
                                              block_sums, st, sc);
        if (e != hipErrorNotSupported) return e;
    }
    MmqShape s;
    // Large M: 4 waves along n, 64 x 256 workgroup tiles. Small M: 4 waves split K,
    // so N/32 workgroups still fill the chip.
    const int64_t tiles_large = ((M + 63) / 64) * ((N + 255) / 256);
    if (M > 32 && tiles_large >= 512)
        s = {2, 2, 4, 1};
    else if (M > 32)
        s = {2, 1, 1, 4};
    else if ((K / (wtype == kTypeQ8_0 || wtype == kTypeQ4_0 ? 32 : 256)) >= 4)
        s = {1, 1, 1, 4};
    else
        s = {1, 2, 4, 1};
    const int64_t bm = 32 * s.tm, bn = 32 * s.tn * s.wn;
    dim3 grid((unsigned)((N + bn - 1) / bn), (unsigned)((M + bm - 1) / bm));
    const size_t lds = s.wk > 1 ? (size_t)s.tm * s.tn * 16 * 64 * 4 * (s.wk - 1) * s.wn : 0;
    MmqFn fn = block_sums ? pick<true>(wtype, s) : pick<false>(wtype, s);
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, st, (const uint8_t*)W, w_row_bytes, N, K, act.qs, act.d, act.m_ld, M,
                       Y, y_stride, block_sums, act.bs);
    return hipGetLastError();
}

}  // namespace dcq
