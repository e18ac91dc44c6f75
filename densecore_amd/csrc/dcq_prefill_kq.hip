// dcq_prefill_kq.hip — prefill / batched mul_mat for K-quant weights (Q6_K, Q4_K, Q5_K) on gfx950
// int8 MFMA.
//
// Replaces ggml's CPU MUL_MAT at M > 1 for K-quant weights (core/src/inference.cpp:1049-1063 and
// 1794-1797 route every M > 1 projection there; executed at core/src/worker.cpp:544). Q6_K has
// vec_dot_q6_K_q8_K's arithmetic per (activation row m, weight row n):
//   Y[m][n] = sum_s (d[n][s] * dA[m][s]) * iS,  iS = sum_g sc[n][s][g] * I_g  (exact int32)
//   I_g = sum over the 16 elements k of group g of qa[m][k] * (q[n][k] - 32)
//
// Tiling (as the Q8_0 prefill). A 256-thread workgroup computes a 128 (m) x 128 (n) tile of Y;
// each wave owns 64 x 64 = 2 x 2 MFMA tiles. Activation rows go global -> LDS directly
// (global_load_lds_dwordx4 from a scalar base); weight bytes pass through registers.
//
// Q6_K, group scales folded into the weights. The workgroup is 8 waves, each owning 64 x 32 (two
// MFMA tiles), so that the two accumulator planes below fit the registers; one workgroup per CU.
// K advances in stages of 128 (half a superblock, 8 groups of 16), double-buffered in LDS, the next
// stage's loads issued before the current stage's MFMAs. At commit, thread (row, part) turns the 32
// weights of its two groups into
// w = (q - 32) * sc_g (|w| <= 4096) and writes them as two int8 planes, w = 64 hi + lo with
// hi = w >> 6 in [-64, 64] and lo = w & 63 (packed 16-bit arithmetic, two weights per VALU
// instruction). The MFMA then sums whole superblocks with no VALU between groups:
//   H = sum_k qa * hi, L = sum_k qa * lo over the superblock's 256 k (v_mfma_i32_32x32x32_i8 into
//   running accumulators), iS = 64 H + L = sum_g sc_g * I_g exactly (|H| <= 256*64*128 < 2^22,
//   |iS| <= 256*4096*128 < 2^31), and per superblock acc += (d * dA) * iS.
// The per-group integer multiply-add of each output (16 VALU instructions per group per MFMA tile)
// becomes the fold at commit, once per weight element per workgroup. LDS rows are 128 bytes of
// 16-byte slots (one group each), slot XOR (row % 8).
//
// Q4_K, vec_dot_q4_K_q8_K's arithmetic, has 8 sub-blocks of 32 with 6-bit scales and mins:
//   Y[m][n] = sum_s dA[m][s] * (d[n][s] * iA - dmin[n][s] * iM)
//   iA = sum_j sc_j * I_j,  iM = sum_j m_j * S_j   (exact int32; S_j = the activation's sub-block sum)
// Stages of 128 (half a superblock: 4 sub-blocks) in 128-byte LDS rows; the nibbles are unpacked to one int8
// per element at commit. Per sub-block: v_mfma_i32_32x32x32_i8 (K = 32) into a zero accumulator,
// then iA += sc_j * I_j. iM runs on the MFMA once per superblock: S_j = 64 hi_j + lo_j (lo_j in
// [0, 63], hi_j in [-64, 63], split at commit from the 16-element bsums) as int8 bytes
// [hi_0..7, lo_0..7] against the bytes m_j in the first or the second eight k of a K = 16 MFMA.
// Q5_K (the Q5 variant) is Q4_K with 5-bit levels: the commit also takes the sub-block's qh bit of
// each element as bit 4 of its level (|I_j| <= 32*31*128 < 2^23, |iA| <= 8*63*2^17 < 2^31).
//
// Workgroup order is XCD-aware (consecutive ids go to different XCDs): each XCD takes a
// contiguous band of n tiles, so its weight rows stay in that XCD's L2.
#include "dcq_common.h"
#include "dcq_kernels.h"

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma16)

namespace dcq {

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128;  // workgroup tile
constexpr int kKS = 128;             // k per stage: half a Q6_K superblock, 8 groups of 16
constexpr int kRow = kKS;            // LDS row: 8 slots of 16 bytes (one group each), slot XOR (row % 8)
constexpr int kXcds = 8;

constexpr int kKS6 = 128;   // Q6_K: k per stage, half a superblock (8 groups of 16)
constexpr int kRow6 = kKS6;  // Q6_K LDS row: 8 slots of 16 bytes, slot XOR (row % 8)

struct __align__(16) StageQ6 {
    int8_t a[kBM * kRow6];   // activation int8, [m][k] (swizzled 16-byte slots)
    int8_t bh[kBN * kRow6];  // weight (q - 32) * sc >> 6 as int8, [n][k]
    int8_t bl[kBN * kRow6];  // weight (q - 32) * sc & 63 as int8, [n][k]
    float dw[kBN];           // weight superblock scale d
    float da[kBM];           // activation superblock scale
};
__device__ __forceinline__ int swz6(int row, int slot) { return row * kRow6 + 16 * (slot ^ (row & 7)); }

struct __align__(16) StageQ4 {
    int8_t a[kBM * kRow];  // activation int8, [m][k] (swizzled 16-byte slots)
    int8_t b[kBN * kRow];  // weight levels as int8 0..15 (Q5_K 0..31), [n][k] (swizzled 16-byte slots)
    uint32_t sc[kBN];      // the stage's 4 sub-block scales (6-bit) per weight row
    uint2 mn[kBN];         // the superblock's 8 sub-block mins (6-bit) per weight row
    float2 dw[kBN];        // weight (d, dmin)
    float da[kBM];         // activation superblock scale
    uint2 sm[kBM][2];      // per activation row: bytes hi_0..7, then lo_0..7 of S_j = 64 hi_j + lo_j
};

__device__ __forceinline__ int swz(int row, int slot) { return row * kRow + 16 * (slot ^ (row & 7)); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory (uniform base `g` + per-lane byte offset `off`) straight
// into LDS at lds_base + 16 * lane (lds_base wave-uniform, in M0): global_load_lds_dwordx4 with an
// SGPR base. Inline asm: the compiler's builtin form waits for every earlier LDS-direct load before
// the next. The compiler does not count these loads, so they are issued before the ordinary loads
// of the same stage, and the stage ends with an explicit s_waitcnt vmcnt(0) before the barrier.
// M0 has no other use in this kernel.
__device__ __forceinline__ void dma16(const void* g, uint32_t off, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(g), "s"(m0) : "memory", "m0");
}

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v16i mfma32k32(v4i a, v4i b) {
    v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ v16i mfma32k32_acc(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v16i mfma32k16(long a, long b) {
    v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, z, 0, 0, 0);
}

// Signed q - 32 bytes of four 6-bit quants: low nibbles from `ql` (bits 0-3 of each byte), the
// two high bits from `qh2` (bits 0-1 of each byte). (qh2 - 2) << 4 is the high nibble of q - 32:
// byte qh2 of the table 0x1000F0E0.
__device__ __forceinline__ uint32_t q6_minus32(uint32_t ql, uint32_t qh2) {
    const uint32_t hi = __builtin_amdgcn_perm(0u, 0x1000F0E0u, qh2);
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(0x0F0F0F0Fu), "v"(ql), "v"(hi));
    return r;
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

// Four signed bytes v times the scale sc2 (replicated in both 16-bit halves) as two int8 planes:
// for each byte b, w = b * sc (|w| <= 4096), hi byte = w >> 6, lo byte = w & 63. Each byte pair is
// widened by placing the bytes in the high halves of two 16-bit lanes and shifting right
// arithmetically, then multiplied with packed 16-bit arithmetic.
__device__ __forceinline__ void fold4(uint32_t v, s16x2 sc2, uint32_t& hi, uint32_t& lo) {
    const s16x2 a01 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v, 0x010C000Cu)) >> (s16x2){8, 8};
    const s16x2 a23 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, v, 0x030C020Cu)) >> (s16x2){8, 8};
    const s16x2 w01 = a01 * sc2, w23 = a23 * sc2;
    const uint32_t h01 = __builtin_bit_cast(uint32_t, w01 >> (s16x2){6, 6});
    const uint32_t h23 = __builtin_bit_cast(uint32_t, w23 >> (s16x2){6, 6});
    const uint32_t l01 = __builtin_bit_cast(uint32_t, w01) & 0x003F003Fu;
    const uint32_t l23 = __builtin_bit_cast(uint32_t, w23) & 0x003F003Fu;
    hi = __builtin_amdgcn_perm(h23, h01, 0x06040200u);
    lo = __builtin_amdgcn_perm(l23, l01, 0x06040200u);
}

}  // namespace

// W: Q6_K rows (w_row_bytes % 4 == 0, 16-byte aligned base); xqs: int8 [M][K]; xd: float
// [K/256][m_ld] with m_ld a multiple of 128; K % 512 == 0.
// FULL: M and N are multiples of the 128 x 128 tile (no row clamps, unguarded stores).
// Arguments: the ones the first loads need come first (the first 56 bytes of arguments are
// preloaded into scalar registers at dispatch).
template <bool DUMP, bool FULL>
__global__ void __launch_bounds__(512, 1) prefill_q6_k_kernel(int tiles_n, int tiles_m, int N, int K, int m_ld,
                                                              int w_row_bytes, const uint8_t* __restrict__ W,
                                                              const int8_t* __restrict__ xqs,
                                                              const float* __restrict__ xd, int M, int stps,
                                                              float* __restrict__ Y, int64_t y_stride,
                                                              int32_t* __restrict__ sums) {
    extern __shared__ __align__(16) uint8_t smem[];
    StageQ6* st = reinterpret_cast<StageQ6*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- split-K: workgroup id = split * tiles + tile. Split s computes stages [s * stps,
    // (s + 1) * stps) and stores its partial tile in plane s of Y (planes of M rows; with one split
    // Y is the output itself) ----
    const int tiles = tiles_n * tiles_m;
    const int split = (int)blockIdx.x / tiles;
    const int bid = (int)blockIdx.x - split * tiles;
    // ---- XCD-aware tile order: XCD x (= id % 8) takes n-tile band x, walked m-first ----
    int tile_m, tile_n;
    if (tiles_n % kXcds == 0) {
        const int band = tiles_n / kXcds;
        const int xcd = bid % kXcds, local = bid / kXcds;
        tile_n = xcd * band + local % band;
        tile_m = local / band;
    } else {
        tile_n = bid % tiles_n;
        tile_m = bid / tiles_n;
    }
    const int m0 = tile_m * kBM, n0 = tile_n * kBN;
    const int nstages = K / kKS6, nsb = K / 256;
    // stps is even: a split covers whole superblocks (two stages each)
    const int s_begin = split * stps, s_end = min(nstages, s_begin + stps);
    Y += (int64_t)split * M * y_stride;

    // ---- staging assignment (fixed for the whole K loop) ----
    // activation rows: instruction i of wave w fills tile rows 8(2w + i) .. + 8, lane l the 16-byte
    // slot (l % 8) of row 8(2w + i) + l/8, which holds logical slot (l % 8) ^ (row % 8)
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    uint32_t a_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 8 * (2 * wave_u + i) + (lane >> 3);
        const int slot = (lane & 7) ^ (r & 7);
        const int row = FULL ? m0 + r : min(m0 + r, M - 1);
        a_off[i] = (uint32_t)row * (uint32_t)K + 16u * (uint32_t)slot;
    }
    // weight rows: row rw = tid / 4 of the tile, pp = tid % 4 = 2e + p. Of the stage's half h the
    // thread holds elements 32t + 16p + [0, 16) for t = e and t = e + 2 (groups 2t + p, LDS slots pp
    // and pp + 4): the ql bytes 64h + 32e + 16p (low nibbles for t = e, high for t = e + 2) and the
    // qh bytes 128 + 32h + 16p. Every thread loads the half's 8 scales, slot 0 the fp16 d.
    // Superblock s starts 210 s bytes into the row (rows are dword aligned): its dword offset
    // sh = (210 s) & 3 is 0 or 2 for every row of the stage; loads start at the dword below.
    const int rw = tid >> 2, pp = tid & 3, e = pp >> 1, p = pp & 1;
    const uint8_t* w_row = W + (int64_t)(FULL ? n0 + rw : min(n0 + rw, N - 1)) * w_row_bytes;
    const int da_row = m0 + (tid & (kBM - 1));  // m_ld >= m0 + 128: in bounds for every tile
    uint32_t gw[10], gx[4];
    float gda;
    auto issue = [&](int stg, StageQ6& S) {
        const int8_t* ab = xqs + (int64_t)stg * kKS6;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16(ab, a_off[i], S.a + 1024 * (2 * wave_u + i));
        const int s = stg >> 1, h = stg & 1;
        const uint8_t* sb = w_row + 210 * s - ((210 * s) & 3);
#pragma unroll
        for (int piece = 0; piece < 2; ++piece) {
            const uint8_t* q = sb + (piece == 1 ? 128 + 32 * h : 64 * h + 32 * e) + 16 * p;
            const U32x4 v = ld4(q);
            gw[5 * piece] = v.x;
            gw[5 * piece + 1] = v.y;
            gw[5 * piece + 2] = v.z;
            gw[5 * piece + 3] = v.w;
            gw[5 * piece + 4] = ld1(q + 16);
        }
        gx[0] = ld1(sb + 192 + 8 * h);
        gx[1] = ld1(sb + 196 + 8 * h);
        gx[2] = ld1(sb + 200 + 8 * h);
        if (pp == 0) gx[3] = ld1(sb + 208);
        if (tid < kBM) gda = xd[(int64_t)s * m_ld + da_row];
    };
    auto commit = [&](int stg, StageQ6& S) {
        const uint32_t sh = (uint32_t)((210 * (stg >> 1)) & 3);
        const uint32_t sc_lo = align_bytes(gx[1], gx[0], sh), sc_hi = align_bytes(gx[2], gx[1], sh);
#pragma unroll
        for (int c = 0; c < 2; ++c) {  // t = e + 2c: group 2t + p, scale byte 2t + p = pp + 4c
            const int sc = __builtin_amdgcn_sbfe((int)(c ? sc_hi : sc_lo), 8 * pp, 8);
            const s16x2 sc2 = {(short)sc, (short)sc};
            const uint32_t nsh = 4u * (uint32_t)c, hsh = 2u * (uint32_t)(e + 2 * c);
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ql = align_bytes(gw[i + 1], gw[i], sh);
                const uint32_t qh = align_bytes(gw[5 + i + 1], gw[5 + i], sh);
                fold4(q6_minus32(ql >> nsh, (qh >> hsh) & 0x03030303u), sc2, hi[i], lo[i]);
            }
            *reinterpret_cast<uint4*>(S.bh + swz6(rw, pp + 4 * c)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            *reinterpret_cast<uint4*>(S.bl + swz6(rw, pp + 4 * c)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
        if (pp == 0) S.dw[rw] = half_bits_to_float((gx[3] >> (8 * sh)) & 0xFFFFu);
        if (tid < kBM) S.da[tid] = gda;
    };

    // ---- wave tile: 64 (m) x 32 (n) at (wm, wn) inside the workgroup tile: 2 MFMA tiles ----
    const int wm = (wave >> 2) * 64, wn = (wave & 3) * 32;
    const int col = lane & 31, hl = lane >> 5;
    float acc[2][16];
    v16i H[2], L[2];  // set by a superblock's first MFMAs
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;
    }

    issue(s_begin, st[0]);
    commit(s_begin, st[0]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
    __syncthreads();

    // superblocks of two stages, unrolled: stage u of a superblock reads buffer u (s_begin is even),
    // its first MFMAs start from zero, its second ends with the epilogue
    for (int sb0 = s_begin; sb0 < s_end; sb0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int stg = sb0 + u;
            const StageQ6& S = st[u];
            const bool more = stg + 1 < s_end;
            if (more) issue(stg + 1, st[u ^ 1]);  // in flight while this stage computes
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                // k 32 kb .. 32 kb + 32 of the stage: lane half hl takes the 16-byte slot 2 kb + hl;
                // fragment rows wm + 32i + col and wn + col share row % 8 = col % 8
                const int fo = col * kRow6 + 16 * ((2 * kb + hl) ^ (col & 7));
                v4i fa[2];
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) fa[ii] = *reinterpret_cast<const v4i*>(S.a + fo + (wm + 32 * ii) * kRow6);
                const v4i fh = *reinterpret_cast<const v4i*>(S.bh + fo + wn * kRow6);
                const v4i fl = *reinterpret_cast<const v4i*>(S.bl + fo + wn * kRow6);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    if (u == 0 && kb == 0) {
                        H[i] = mfma32k32(fa[i], fh);
                        L[i] = mfma32k32(fa[i], fl);
                    } else {
                        H[i] = mfma32k32_acc(fa[i], fh, H[i]);
                        L[i] = mfma32k32_acc(fa[i], fl, L[i]);
                    }
                }
            }
            if (u == 1) {
                // end of superblock s: iS = 64 H + L, acc += (d * dA) * iS, the scales from this stage
                const int s = stg >> 1;
                const float dwj = S.dw[wn + col];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v4 = *reinterpret_cast<const float4*>(&S.da[wm + 32 * i + 8 * q + 4 * hl]);
                        const float da4[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int v = 4 * q + k;
                            const int iS = (H[i][v] << 6) + L[i][v];
                            acc[i][v] = fmaf(dwj * da4[k], (float)iS, acc[i][v]);
                            if (DUMP) {
                                const int n = n0 + wn + col;
                                const int m = m0 + wm + 32 * i + 8 * q + 4 * hl + k;
                                if (m < M && n < N) sums[((int64_t)m * N + n) * nsb + s] = iS;
                            }
                        }
                    }
                }
            }
            if (more) {
                // the other buffer was last read in stage stg - 1, which every wave finished before
                // the barrier that ended it: one barrier per stage is enough
                commit(stg + 1, st[u ^ 1]);
                __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
                __syncthreads();
            }
        }
    }

    // ---- store: lane owns column n, rows m0 + wm + 32i + 8(v/4) + 4hl + v%4 ----
    if (!FULL && n0 + wn + col >= N) return;
    float* yl = Y + (int64_t)(m0 + wm + 4 * hl) * y_stride + (n0 + wn + col);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = 32 * i + 8 * (v >> 2) + (v & 3);
            if (FULL || m0 + wm + 4 * hl + r < M) yl[(int64_t)r * y_stride] = acc[i][v];
        }
}

// W: Q4_K rows (w_row_bytes % 16 == 0, 16-byte aligned base); xqs: int8 [M][K]; xd: float
// [K/256][m_ld] with m_ld a multiple of 128; xbs: int16 [M][K/16]; K % 256 == 0.
// FULL: M and N are multiples of the 128 x 128 tile (no row clamps, unguarded stores).
// Arguments: the ones the first loads need come first (the first 56 bytes of arguments are
// preloaded into scalar registers at dispatch).
template <bool DUMP, bool FULL, bool Q5>
__global__ void __launch_bounds__(256, 2) prefill_q4_k_kernel(int tiles_n, int tiles_m, int N, int K, int m_ld,
                                                              int w_row_bytes, const uint8_t* __restrict__ W,
                                                              const int8_t* __restrict__ xqs,
                                                              const float* __restrict__ xd,
                                                              const int16_t* __restrict__ xbs, int M, int stps,
                                                              float* __restrict__ Y, int64_t y_stride,
                                                              int32_t* __restrict__ sums) {
    extern __shared__ __align__(16) uint8_t smem[];
    StageQ4* st = reinterpret_cast<StageQ4*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- split-K: workgroup id = split * tiles + tile. Split s computes stages [s * stps,
    // (s + 1) * stps) and stores its partial tile in plane s of Y (planes of M rows; with one split
    // Y is the output itself) ----
    const int tiles = tiles_n * tiles_m;
    const int split = (int)blockIdx.x / tiles;
    const int bid = (int)blockIdx.x - split * tiles;
    // ---- XCD-aware tile order: XCD x (= id % 8) takes n-tile band x, walked m-first ----
    int tile_m, tile_n;
    if (tiles_n % kXcds == 0) {
        const int band = tiles_n / kXcds;
        const int xcd = bid % kXcds, local = bid / kXcds;
        tile_n = xcd * band + local % band;
        tile_m = local / band;
    } else {
        tile_n = bid % tiles_n;
        tile_m = bid / tiles_n;
    }
    const int m0 = tile_m * kBM, n0 = tile_n * kBN;
    const int nstages = K / kKS, nsb = K / 256;
    // stps is even: a split covers whole superblocks (two stages each)
    const int s_begin = split * stps, s_end = min(nstages, s_begin + stps);
    Y += (int64_t)split * M * y_stride;

    // ---- staging assignment (fixed for the whole K loop) ----
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int a_row0 = 8 * (4 * wave_u) + (lane >> 3);
    const int a_slot = (lane & 7) ^ (a_row0 & 7);
    uint32_t a_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = FULL ? m0 + a_row0 + 8 * i : min(m0 + a_row0 + 8 * i, M - 1);
        a_off[i] = (uint32_t)row * (uint32_t)K + 16u * (uint32_t)a_slot;
    }
    // weight rows: row rw = tid / 2 of the tile, part p = tid % 2: the 32 nibble bytes of chunk
    // 2h + p of the stage's half h (bytes 16 + 64h + 32p, Q5_K 48 + 64h + 32p: elements 64p + [0, 32)
    // of the stage in the low nibbles, 64p + 32 + [0, 32) in the high ones, and for Q5_K the 32 qh
    // bytes); part 0 also loads the 16-byte header (d, dmin, 12 bytes of scales and mins). Threads
    // 0..127 load activation row m0 + tid's scale and its superblock's 16 bsums.
    constexpr int kSb = Q5 ? 176 : 144, kQs = Q5 ? 48 : 16;
    const int rw = tid >> 1, p = tid & 1;
    const uint8_t* w_row = W + (int64_t)(FULL ? n0 + rw : min(n0 + rw, N - 1)) * w_row_bytes;
    const int arow = tid & (kBM - 1);
    const int da_row = m0 + arow;  // m_ld >= m0 + 128: in bounds for every tile
    const int16_t* bs_row = xbs + (int64_t)(FULL ? m0 + arow : min(m0 + arow, M - 1)) * (K / 16);
    uint4 gq[2], ghdr, gbs[2];
    [[maybe_unused]] uint4 gqh[2];
    float gda;
    auto issue = [&](int stg, StageQ4& S) {
        const int8_t* ab = xqs + (int64_t)stg * kKS;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16(ab, a_off[i], S.a + 1024 * (4 * wave_u + i));
        const int s = stg >> 1, h = stg & 1;
        const uint8_t* sb = w_row + kSb * (int64_t)s;
        gq[0] = ld16(sb + kQs + 64 * h + 32 * p);
        gq[1] = ld16(sb + kQs + 16 + 64 * h + 32 * p);
        if constexpr (Q5) {
            gqh[0] = ld16(sb + 16);
            gqh[1] = ld16(sb + 32);
        }
        if (p == 0) ghdr = ld16(sb);
        gda = xd[(int64_t)s * m_ld + da_row];
        gbs[0] = ld16(bs_row + 16 * s);
        gbs[1] = ld16(bs_row + 16 * s + 8);
    };
    auto commit = [&](int stg, StageQ4& S) {
        const int h = stg & 1;
        const uint32_t lo = 0x0F0F0F0Fu;
        const uint32_t q[8] = {gq[0].x, gq[0].y, gq[0].z, gq[0].w, gq[1].x, gq[1].y, gq[1].z, gq[1].w};
        if constexpr (Q5) {
            // sub-blocks j = 4h + 2p (low nibbles) and j + 1 (high): bit j / j + 1 of qh[l] is bit 4
            const uint32_t qh[8] = {gqh[0].x, gqh[0].y, gqh[0].z, gqh[0].w, gqh[1].x, gqh[1].y, gqh[1].z, gqh[1].w};
            const uint32_t j0 = 4u * (uint32_t)h + 2u * (uint32_t)p, j1 = j0 + 1u;
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p)) =
                make_uint4(q5_levels(q[0], qh[0], j0), q5_levels(q[1], qh[1], j0), q5_levels(q[2], qh[2], j0),
                           q5_levels(q[3], qh[3], j0));
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 1)) =
                make_uint4(q5_levels(q[4], qh[4], j0), q5_levels(q[5], qh[5], j0), q5_levels(q[6], qh[6], j0),
                           q5_levels(q[7], qh[7], j0));
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 2)) =
                make_uint4(q5_levels(q[0] >> 4, qh[0], j1), q5_levels(q[1] >> 4, qh[1], j1),
                           q5_levels(q[2] >> 4, qh[2], j1), q5_levels(q[3] >> 4, qh[3], j1));
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 3)) =
                make_uint4(q5_levels(q[4] >> 4, qh[4], j1), q5_levels(q[5] >> 4, qh[5], j1),
                           q5_levels(q[6] >> 4, qh[6], j1), q5_levels(q[7] >> 4, qh[7], j1));
        } else {
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p)) = make_uint4(q[0] & lo, q[1] & lo, q[2] & lo, q[3] & lo);
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 1)) = make_uint4(q[4] & lo, q[5] & lo, q[6] & lo, q[7] & lo);
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 2)) =
                make_uint4((q[0] >> 4) & lo, (q[1] >> 4) & lo, (q[2] >> 4) & lo, (q[3] >> 4) & lo);
            *reinterpret_cast<uint4*>(S.b + swz(rw, 4 * p + 3)) =
                make_uint4((q[4] >> 4) & lo, (q[5] >> 4) & lo, (q[6] >> 4) & lo, (q[7] >> 4) & lo);
        }
        if (p == 0) {
            // 6-bit scales and mins of the 8 sub-blocks (get_scale_min_k4): j < 4 from bytes j, j + 4;
            // j >= 4 from the low / high nibble of byte j + 4 and the top two bits of bytes j - 4, j
            const uint32_t s0 = ghdr.y, s1 = ghdr.z, s2 = ghdr.w;
            const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
            const uint32_t mn_lo = s1 & 0x3F3F3F3Fu, mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
            S.sc[rw] = h ? sc_hi : sc_lo;
            S.mn[rw] = make_uint2(mn_lo, mn_hi);
            S.dw[rw] = make_float2(half_bits_to_float(ghdr.x & 0xFFFFu), half_bits_to_float(ghdr.x >> 16));
        }
        if (tid < kBM) {
            S.da[tid] = gda;
            // S_j = bsums 2j + 2j + 1, then its bytes: hi_j = S_j >> 6, lo_j = S_j & 63
            const uint32_t b[8] = {gbs[0].x, gbs[0].y, gbs[0].z, gbs[0].w, gbs[1].x, gbs[1].y, gbs[1].z, gbs[1].w};
            uint32_t hw[2] = {0u, 0u}, lw[2] = {0u, 0u};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int sj = (int)(int16_t)(b[j] & 0xFFFFu) + ((int)b[j] >> 16);
                hw[j >> 2] |= ((uint32_t)(sj >> 6) & 0xFFu) << (8 * (j & 3));
                lw[j >> 2] |= ((uint32_t)sj & 63u) << (8 * (j & 3));
            }
            S.sm[tid][0] = make_uint2(hw[0], hw[1]);
            S.sm[tid][1] = make_uint2(lw[0], lw[1]);
        }
    };

    // ---- wave tile: 64 x 64 at (wm, wn) inside the workgroup tile ----
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int col = lane & 31, hl = lane >> 5;
    float acc[2][2][16];
    int ai[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f, ai[i][j][v] = 0;

    issue(s_begin, st[s_begin & 1]);
    commit(s_begin, st[s_begin & 1]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
    __syncthreads();

    for (int stg = s_begin; stg < s_end; ++stg) {
        const StageQ4& S = st[stg & 1];
        const bool more = stg + 1 < s_end;
        if (more) issue(stg + 1, st[(stg + 1) & 1]);  // in flight while this stage computes
        uint32_t scw[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) scw[j] = S.sc[wn + 32 * j + col];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            // sub-block kb: lane half hl takes the 16-byte slot 2 kb + hl
            const int fo = col * kRow + 16 * ((2 * kb + hl) ^ (col & 7));
            v4i fa[2], fb[2];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) fa[ii] = *reinterpret_cast<const v4i*>(S.a + fo + (wm + 32 * ii) * kRow);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) fb[jj] = *reinterpret_cast<const v4i*>(S.b + fo + (wn + 32 * jj) * kRow);
            int sc[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) sc[j] = (int)((scw[j] >> (8 * kb)) & 0xFFu);
            v16i D[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) D[i][j] = mfma32k32(fa[i], fb[j]);
            // |I_j| <= 32*31*128 < 2^23; |iA| <= 8*63*32*31*128 < 2^31
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) ai[i][j][v] = __mul24(sc[j], D[i][j][v]) + ai[i][j][v];
        }
        if (stg & 1) {
            // end of superblock s: iM on the MFMA, then acc += dA * (d * iA - dmin * iM)
            const int s = stg >> 1;
            long am[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint2 v = S.sm[wm + 32 * i + col][hl];
                am[i] = (long)(((uint64_t)v.y << 32) | v.x);
            }
            long bh[2], bl[2];
            float2 dmj[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint2 v = S.mn[wn + 32 * j + col];
                const long mb = (long)(((uint64_t)v.y << 32) | v.x);
                bh[j] = hl ? 0 : mb;  // k 0..7 (the hi bytes) against the mins
                bl[j] = hl ? mb : 0;  // k 8..15 (the lo bytes)
                dmj[j] = S.dw[wn + 32 * j + col];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float da[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v4 = *reinterpret_cast<const float4*>(&S.da[wm + 32 * i + 8 * q + 4 * hl]);
                    da[4 * q] = v4.x, da[4 * q + 1] = v4.y, da[4 * q + 2] = v4.z, da[4 * q + 3] = v4.w;
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v16i Mh = mfma32k16(am[i], bh[j]);
                    const v16i Ml = mfma32k16(am[i], bl[j]);
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int iM = (Mh[v] << 6) + Ml[v];  // |iM| <= 8*63*4064 < 2^31
                        const float t = fmaf(-dmj[j].y, (float)iM, dmj[j].x * (float)ai[i][j][v]);
                        acc[i][j][v] = fmaf(da[v], t, acc[i][j][v]);
                        if (DUMP) {
                            const int n = n0 + wn + 32 * j + col;
                            const int m = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                            if (m < M && n < N) {
                                int32_t* o = sums + (((int64_t)m * N + n) * nsb + s) * 2;
                                o[0] = ai[i][j][v];
                                o[1] = iM;
                            }
                        }
                        ai[i][j][v] = 0;
                    }
                }
            }
        }
        if (more) {
            commit(stg + 1, st[(stg + 1) & 1]);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
            __syncthreads();
        }
    }

    // ---- store: lane owns column n, rows m0 + wm + 32i + 8(v/4) + 4hl + v%4 ----
    float* yl = Y + (int64_t)(m0 + wm + 4 * hl) * y_stride + (n0 + wn + col);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (!FULL && n0 + wn + 32 * j + col >= N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 32 * i + 8 * (v >> 2) + (v & 3);
                if (FULL || m0 + wm + 4 * hl + r < M) yl[(int64_t)r * y_stride + 32 * j] = acc[i][j][v];
            }
    }
}

hipError_t launch_prefill_q4_k(bool q5, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                               const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const SplitScratch& sc) {
    if (K % 256 || w_row_bytes % 16 || w_row_bytes > INT32_MAX || act.m_ld % kBM || act.m_ld > INT32_MAX ||
        !act.bs || N > (1 << 30) || M > (1 << 30) || K > (1 << 30))
        return hipErrorNotSupported;
    if ((uint64_t)M * (uint64_t)K >= (1ull << 32)) return hipErrorNotSupported;  // 32-bit DMA offsets
    const int tiles_n = (int)((N + kBN - 1) / kBN), tiles_m = (int)((M + kBM - 1) / kBM);
    const size_t lds = 2 * sizeof(StageQ4);
    const bool full = M % kBM == 0 && N % kBN == 0;
    auto fn = q5 ? (block_sums ? (full ? prefill_q4_k_kernel<true, true, true> : prefill_q4_k_kernel<true, false, true>)
                               : (full ? prefill_q4_k_kernel<false, true, true> : prefill_q4_k_kernel<false, false, true>))
                 : (block_sums ? (full ? prefill_q4_k_kernel<true, true, false> : prefill_q4_k_kernel<true, false, false>)
                               : (full ? prefill_q4_k_kernel<false, true, false> : prefill_q4_k_kernel<false, false, false>));
    // split-K when the tiles cannot fill the chip (ranges of whole superblocks: two stages each)
    const SplitPlan sp = plan_split_k((int64_t)tiles_n * tiles_m, (int)(K / kKS), 2, M, N, sc);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    hipLaunchKernelGGL(fn, dim3((unsigned)(tiles_n * tiles_m * sp.splits)), dim3(256), lds, st, tiles_n, tiles_m,
                       (int)N, (int)K, (int)act.m_ld, (int)w_row_bytes, (const uint8_t*)W, act.qs, act.d,
                       (const int16_t*)act.bs, (int)M, sp.stps, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

hipError_t launch_prefill_q6_k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                               int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                               const SplitScratch& sc) {
    // K % 512: an even number of superblocks, so the 2-byte overreach of the scale and d loads of
    // an even superblock (dword offset 0) stays inside the next one
    if (K % 512 || w_row_bytes % 4 || w_row_bytes > INT32_MAX || act.m_ld % kBM || act.m_ld > INT32_MAX ||
        N > (1 << 30) || M > (1 << 30) || K > (1 << 30))
        return hipErrorNotSupported;
    // the DMA offsets are 32-bit: every activation row must lie within 4 GiB of the base
    if ((uint64_t)M * (uint64_t)K >= (1ull << 32)) return hipErrorNotSupported;
    const int tiles_n = (int)((N + kBN - 1) / kBN), tiles_m = (int)((M + kBM - 1) / kBM);
    const size_t lds = 2 * sizeof(StageQ6);
    const bool full = M % kBM == 0 && N % kBN == 0;
    auto fn = block_sums ? (full ? prefill_q6_k_kernel<true, true> : prefill_q6_k_kernel<true, false>)
                         : (full ? prefill_q6_k_kernel<false, true> : prefill_q6_k_kernel<false, false>);
    // stages of half a superblock (splits cover whole superblocks)
    const SplitPlan sp = plan_split_k((int64_t)tiles_n * tiles_m, (int)(K / kKS6), 2, M, N, sc);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    hipLaunchKernelGGL(fn, dim3((unsigned)(tiles_n * tiles_m * sp.splits)), dim3(512), lds, st, tiles_n, tiles_m,
                       (int)N, (int)K, (int)act.m_ld, (int)w_row_bytes, (const uint8_t*)W, act.qs, act.d, (int)M,
                       sp.stps, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

}  // namespace dcq
