// dcq_prefill.hip — prefill / batched mul_mat for Q8_0 (and Q4_0) weights on gfx950 int8 MFMA.
//
// Replaces ggml's CPU MUL_MAT at M > 1 for Q8_0 weights (core/src/inference.cpp:1049-1063
// routes every M > 1 projection there; executed at core/src/worker.cpp:544):
//   Y[m][n] = sum_b dA[m][b] * dW[n][b] * I_b[m][n],  I_b = sum_{k in block b} qa*qw  (exact)
//
// Tiling. A 256-thread workgroup computes a 128 (m) x 128 (n) tile of Y; its four waves
// each own 64 x 64 = 2 x 2 MFMA tiles of v_mfma_i32_32x32x32_i8 (K = 32 = one Q8_0 block,
// so every MFMA result is one block's exact integer sums I_b for 32 x 32 outputs).
// K advances in stages of 4 blocks (128 k): the next stage's global loads (activation
// int8 rows, Q8_0 weight block pairs re-sliced into int8 rows and fp32 scales, activation
// scales) are issued before the current stage's MFMAs and land in the other half of a
// double-buffered LDS tile. Activation rows and scales go global -> LDS directly
// (global_load_lds_dwordx4 from a scalar base, no registers in flight); weight block pairs
// pass through registers to be re-sliced, and the commit also stores each block's epilogue
// constants (dW, -dW * 1.5*2^23) beside the quants. LDS rows are 128 bytes whose 16-byte slots
// are XOR-swizzled by a key of the row (swz_key), so the rows a ds_read_b128 touches spread over
// the banks.
//
// Epilogue per MFMA (16 values per lane; lane = one weight row n, 16 activation rows m):
// the accumulator is seeded with the bit pattern of 1.5 * 2^23, so the int32 result read
// as fp32 is exactly 1.5*2^23 + I (|I| <= 32*127*128 < 2^22); then
//   t = fma(F, dW, -dW * 1.5*2^23)   (= dW * I, rounded once)
//   acc = fma(t, dA, acc)
// two VALU ops per value per block — the bound of this kernel (VALU at 4 cycles per
// wave64 op against 32 cycles per MFMA: 25 % of the int8 MFMA peak without packed fp32).
// The seed is held in 16 VGPRs for the whole loop; everything else per block is the LDS
// reads, four MFMAs and ~4 address instructions (about 37 VALU per MFMA over the kernel).
//
// Q4_0 weights (FMT kFmtQ4_0) take the same path: a thread's block pair is 36 bytes (two
// 18-byte blocks) and the commit unpacks the nibbles into signed q - 8 bytes, so the LDS tile,
// MFMAs and epilogue are the Q8_0 ones (|I_b| <= 32*8*128 < 2^22 as well).
// Row-split Q8_0 weights (FMT kFmtQ8_0RS: each row's quants, then its fp16 scales) skip the
// register pass: the quants go global -> LDS directly like the activation rows, and each lane
// widens the two scales its own dword load brought into the (dW, -dW * 1.5*2^23) pairs after its
// wait, before the stage's barrier.
//
// The MFMAs of block kb + 1 are issued tile by tile, each right after block kb's epilogue of that
// tile, so the matrix unit runs one block ahead of the VALU within a wave.
//
// Workgroup order is XCD-aware: consecutive workgroup ids go to different XCDs, so the
// id is remapped to give each XCD a contiguous band of n tiles (its weight rows stay in
// that XCD's L2) walked in m order.
#include "dcq_common.h"
#include "dcq_kernels.h"

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma16)

namespace dcq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128;  // workgroup tile
constexpr int kKB = 4;               // Q8_0 blocks per stage
constexpr int kKS = kKB * 32;        // k per stage = bytes per LDS row
constexpr int kRow = kKS;            // LDS row: 8 slots of 16 bytes, slot index XOR swz_key(row)
constexpr int kMagic = 0x4B400000;   // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;
constexpr int kXcds = 8;

struct __align__(16) Stage {
    int8_t a[kBM * kRow];    // activation int8, [m][k] (swizzled 16-byte slots)
    int8_t b[kBN * kRow];    // weight int8, [n][k] (swizzled 16-byte slots)
    float2 dwc[kKB][kBN];    // per weight row and block: (dW, -dW * 1.5*2^23), the epilogue's constants
    float da[kKB][kBM];      // activation block scales
    uint2 dw16[kBN];         // row-split weights: the stage's four fp16 block scales per row, as loaded
};

// LDS byte offset of logical 16-byte slot `slot` (= 2*block + half) of tile row `row`.
// The XOR key is row % 8 with bit 3 of the row folded in, so the 16 rows one ds_read_b128 pass
// serves (8 of each parity: 64 banks) hit 16 distinct 4-bank groups; with row % 8 alone, rows r and
// r + 8 collided.
__device__ __forceinline__ int swz_key(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int slot) { return row * kRow + 16 * (slot ^ swz_key(row)); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 4 bytes per lane from global memory (uniform base `g` + per-lane byte offset `off`) into LDS at
// lds_base + 4 * lane, as dma16 below.
__device__ __forceinline__ void dma4(const void* g, uint32_t off, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(g), "s"(m0) : "memory", "m0");
}

// 16 bytes per lane from global memory (uniform base `g` + per-lane byte offset `off`) straight
// into LDS at lds_base + 16 * lane (lds_base wave-uniform, in M0): global_load_lds_dwordx4 with an
// SGPR base, so advancing a stage costs scalar adds only and no registers are held while the load
// is in flight. Written as inline asm because the compiler's builtin form waits for every earlier
// LDS-direct load before the next one (it cannot tell the destinations apart). The compiler does
// not count these loads, so every call precedes the ordinary loads of the same stage (loads retire
// in order, so its own vmcnt waits stay conservative), and the stage ends with an explicit
// s_waitcnt vmcnt(0) before the barrier. M0 has no other use in this kernel.
__device__ __forceinline__ void dma16(const void* g, uint32_t off, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(g), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

}  // namespace

// W: Q8_0 rows, or Q4_0 rows when Q40 (w_row_bytes % 4 == 0); xqs: int8 [M][K]; xd: float
// [K/32][m_ld]; K % 128 == 0.
// FULL: M and N are multiples of the 128 x 128 tile (no row clamps, unguarded stores).
// Arguments: the ones the first loads need come first (the first 56 bytes of arguments are
// preloaded into scalar registers at dispatch).
template <bool DUMP, bool FULL, int FMT>
__global__ void __launch_bounds__(256, 2) prefill_q8_0_kernel(int tiles_n, int tiles_m, int N, int K, int m_ld,
                                                              int w_row_bytes, const uint8_t* __restrict__ W,
                                                              const int8_t* __restrict__ xqs,
                                                              const float* __restrict__ xd, int M, int stps,
                                                              float* __restrict__ Y, int64_t y_stride,
                                                              int32_t* __restrict__ sums) {
    constexpr bool Q40 = FMT == kFmtQ4_0, RS = FMT == kFmtQ8_0RS;
    extern __shared__ __align__(16) uint8_t smem[];
    Stage* st = reinterpret_cast<Stage*>(smem);
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
        const int band = tiles_n / kXcds;  // n tiles per XCD
        const int xcd = bid % kXcds, local = bid / kXcds;
        tile_n = xcd * band + local % band;
        tile_m = local / band;
    } else {  // shapes the band map does not cover exactly: plain order
        tile_n = bid % tiles_n;
        tile_m = bid / tiles_n;
    }
    const int m0 = tile_m * kBM, n0 = tile_n * kBN;
    const int nstages = K / kKS;
    const int s_begin = split * stps, s_end = min(nstages, s_begin + stps);
    Y += (int64_t)split * M * y_stride;

    // ---- staging assignment (per-lane byte offsets, fixed for the whole K loop) ----
    // activation rows: straight to LDS, 4 x 1 KB per wave per stage; instruction i of wave w
    // fills tile rows 8*(4w+i) .. +8, lane l the 16-byte slot (l % 8) of row 8*(4w+i) + l/8,
    // which holds logical slot (l % 8) ^ swz_key(row); rows past M clamp to M - 1
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int a_row0 = 8 * (4 * wave_u) + (lane >> 3);
    uint32_t a_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int a_slot = (lane & 7) ^ swz_key(a_row0 + 8 * i);
        const int row = FULL ? m0 + a_row0 + 8 * i : min(m0 + a_row0 + 8 * i, M - 1);
        a_off[i] = (uint32_t)row * (uint32_t)K + 16u * (uint32_t)a_slot;
    }
    // activation scales: waves 0 and 1, one 1 KB instruction each: lane l of wave w holds
    // block (64w + l) / 32, rows 4 * ((64w + l) % 32) .. +4
    const int dc = 64 * (wave_u & 1) + lane;
    const uint32_t da_off = (uint32_t)(((int64_t)(dc >> 5) * m_ld + m0 + 4 * (dc & 31)) * 4);
    // weight rows: row rw = tid / 2, block pair hw of the stage (68 bytes: d0, q0, d1, q1; Q4_0: 36
    // bytes, the same order), through registers: q0 sits 2 bytes off a dword and is re-sliced; d1
    // and q1 start on dwords
    constexpr int kBlk = Q40 ? 18 : 34;  // weight block bytes
    const int rw = tid >> 1, hw = tid & 1;
    const uint8_t* w_src = W + (int64_t)(FULL ? n0 + rw : min(n0 + rw, N - 1)) * w_row_bytes + hw * 2 * kBlk;
    uint32_t gw[17];  // Q4_0 uses gw[0..8]
    // row-split weights (RS): the quants go straight to LDS like the activation rows (instruction i
    // of wave w fills tile rows 8*(4w+i) .. +8), and each wave's 32 rows' four fp16 scales per stage
    // by one dword instruction (lane l: row 32w + l/2, scales 2(l%2), 2(l%2)+1); the rows' byte
    // offsets fit 32 bits (the launcher checks N * w_row_bytes < 4 GiB)
    uint32_t b_off[4], bd_off;
    if constexpr (RS) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b_slot = (lane & 7) ^ swz_key(a_row0 + 8 * i);
            const int row = FULL ? n0 + a_row0 + 8 * i : min(n0 + a_row0 + 8 * i, N - 1);
            b_off[i] = (uint32_t)row * (uint32_t)w_row_bytes + 16u * (uint32_t)b_slot;
        }
        const int row = FULL ? n0 + 32 * wave_u + (lane >> 1) : min(n0 + 32 * wave_u + (lane >> 1), N - 1);
        bd_off = (uint32_t)row * (uint32_t)w_row_bytes + 4u * (uint32_t)(lane & 1);
    }
#define DCQ_ISSUE(s_, S_)                                                                      \
    do {                                                                                       \
        const int8_t* ab_ = xqs + (int64_t)(s_) * kKS;                                         \
        _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                                       \
            dma16(ab_, a_off[i_], (S_).a + 1024 * (4 * wave_u + i_));                          \
        if (wave_u < 2) dma16(xd + (int64_t)(s_) * kKB * m_ld, da_off, &(S_).da[0][0] + 256 * wave_u); \
        if constexpr (RS) {                                                                    \
            _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                                   \
                dma16(W + (int64_t)(s_) * kKS, b_off[i_], (S_).b + 1024 * (4 * wave_u + i_));  \
            dma4(W + K + (int64_t)(s_) * (2 * kKB), bd_off, &(S_).dw16[32 * wave_u]);          \
            break;                                                                             \
        }                                                                                      \
        const uint8_t* wp_ = w_src + (int64_t)(s_) * (kKB * kBlk);                             \
        _Pragma("unroll") for (int i_ = 0; i_ < 2; ++i_) {                                     \
            const U32x4 v_ = ld4(wp_ + 16 * i_);                                               \
            gw[4 * i_] = v_.x;                                                                 \
            gw[4 * i_ + 1] = v_.y;                                                             \
            gw[4 * i_ + 2] = v_.z;                                                             \
            gw[4 * i_ + 3] = v_.w;                                                             \
        }                                                                                      \
        gw[8] = ld1(wp_ + 32);                                                                 \
        if constexpr (!Q40) {                                                                  \
            _Pragma("unroll") for (int i_ = 0; i_ < 2; ++i_) {                                 \
                const U32x4 v_ = ld4(wp_ + 36 + 16 * i_);                                      \
                gw[9 + 4 * i_] = v_.x;                                                         \
                gw[10 + 4 * i_] = v_.y;                                                        \
                gw[11 + 4 * i_] = v_.z;                                                        \
                gw[12 + 4 * i_] = v_.w;                                                        \
            }                                                                                  \
        }                                                                                      \
    } while (0)
    // weight block pair bytes: [0,2) d0, [2,34) q0, [34,36) d1, [36,68) q1 (Q4_0: [0,2) d0,
    // [2,18) q0, [18,20) d1, [20,36) q1, each block's 16 nibble bytes holding its elements 0..15 in
    // the low nibbles and 16..31 in the high ones); logical slots 4hw .. 4hw+3 of row rw
#define DCQ_COMMIT(S_)                                                                         \
    do {                                                                                       \
        if constexpr (RS) break; /* staged by DMA; the scales are widened by DCQ_WIDEN */      \
        float d0_, d1_;                                                                        \
        if constexpr (Q40) {                                                                   \
            const uint32_t m_ = 0x0F0F0F0Fu;                                                   \
            const uint32_t q0_[4] = {align_bytes(gw[1], gw[0], 2), align_bytes(gw[2], gw[1], 2), \
                                     align_bytes(gw[3], gw[2], 2), align_bytes(gw[4], gw[3], 2)}; \
            const uint32_t q1_[4] = {gw[5], gw[6], gw[7], gw[8]};                              \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw)) =                              \
                make_uint4(minus8(q0_[0] & m_), minus8(q0_[1] & m_), minus8(q0_[2] & m_), minus8(q0_[3] & m_)); \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 1)) =                          \
                make_uint4(minus8((q0_[0] >> 4) & m_), minus8((q0_[1] >> 4) & m_),             \
                           minus8((q0_[2] >> 4) & m_), minus8((q0_[3] >> 4) & m_));            \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 2)) =                          \
                make_uint4(minus8(q1_[0] & m_), minus8(q1_[1] & m_), minus8(q1_[2] & m_), minus8(q1_[3] & m_)); \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 3)) =                          \
                make_uint4(minus8((q1_[0] >> 4) & m_), minus8((q1_[1] >> 4) & m_),             \
                           minus8((q1_[2] >> 4) & m_), minus8((q1_[3] >> 4) & m_));            \
            d0_ = half_bits_to_float(gw[0] & 0xFFFFu);                                         \
            d1_ = half_bits_to_float(gw[4] >> 16);                                             \
        } else {                                                                               \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw)) =                              \
                make_uint4(align_bytes(gw[1], gw[0], 2), align_bytes(gw[2], gw[1], 2),          \
                           align_bytes(gw[3], gw[2], 2), align_bytes(gw[4], gw[3], 2));        \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 1)) =                          \
                make_uint4(align_bytes(gw[5], gw[4], 2), align_bytes(gw[6], gw[5], 2),          \
                           align_bytes(gw[7], gw[6], 2), align_bytes(gw[8], gw[7], 2));        \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 2)) =                          \
                make_uint4(gw[9], gw[10], gw[11], gw[12]);                                     \
            *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 3)) =                          \
                make_uint4(gw[13], gw[14], gw[15], gw[16]);                                    \
            d0_ = half_bits_to_float(gw[0] & 0xFFFFu);                                         \
            d1_ = half_bits_to_float(gw[8] >> 16);                                             \
        }                                                                                      \
        /* -dW * 1.5 * 2^23 is exact: an 11-bit significand times 3 * 2^22 */                  \
        (S_).dwc[2 * hw][rw] = make_float2(d0_, -d0_ * kMagicF);                               \
        (S_).dwc[2 * hw + 1][rw] = make_float2(d1_, -d1_ * kMagicF);                           \
    } while (0)
    // row-split weights, after the wait for this wave's loads: each lane widens the two fp16 scales
    // its own dword load brought (row 32w + l/2, blocks 2(l%2) and 2(l%2)+1) into the epilogue's
    // constants; the barrier that follows publishes them
#define DCQ_WIDEN(S_)                                                                          \
    do {                                                                                       \
        if constexpr (RS) {                                                                    \
            const int r_ = 32 * wave_u + (lane >> 1), k_ = 2 * (lane & 1);                     \
            const uint32_t h_ = reinterpret_cast<const uint32_t*>(&(S_).dw16[r_])[lane & 1];   \
            const float e0_ = half_bits_to_float(h_ & 0xFFFFu), e1_ = half_bits_to_float(h_ >> 16); \
            (S_).dwc[k_][r_] = make_float2(e0_, -e0_ * kMagicF);                               \
            (S_).dwc[k_ + 1][r_] = make_float2(e1_, -e1_ * kMagicF);                           \
        }                                                                                      \
    } while (0)

    // ---- wave tile: 64 x 64 at (wm, wn) inside the workgroup tile ----
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int col = lane & 31, hl = lane >> 5;
    v16i cmagic;
#pragma unroll
    for (int v = 0; v < 16; ++v) cmagic[v] = kMagic;
    // opaque to the compiler: it keeps the seed in 16 VGPRs for the whole loop instead of
    // rematerialising it from scalar registers before every block (8 moves per block)
    asm volatile("" : "+v"(cmagic));
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    DCQ_ISSUE(s_begin, st[s_begin & 1]);
    DCQ_COMMIT(st[s_begin & 1]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
    DCQ_WIDEN(st[s_begin & 1]);
    __syncthreads();

    // Fragments of block kb: this lane's fragment rows wm + 32i + col and wn + 32j + col share
    // swz_key(col) (wm, wn and 32i are multiples of 16), so the swizzled slot of block kb depends on
    // (kb, hl, col) only; the rows are immediates.
    v4i fa[2], fb[2];
    auto read_frags = [&](const Stage& S, int kb) {
        const int fo = col * kRow + 16 * ((2 * kb + hl) ^ swz_key(col));
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) fa[ii] = *reinterpret_cast<const v4i*>(S.a + fo + (wm + 32 * ii) * kRow);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) fb[jj] = *reinterpret_cast<const v4i*>(S.b + fo + (wn + 32 * jj) * kRow);
    };
    // Epilogue of tile (i, j) of block kb: acc += dA * (dW * I), I read from the seeded result.
    auto epilogue = [&](const v16i& d, float2 wc, const float4 (&da_v)[4], float (&a)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float da4[4] = {da_v[q].x, da_v[q].y, da_v[q].z, da_v[q].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 4 * q + e;
                const float t = fmaf(__int_as_float(d[v]), wc.x, wc.y);
                a[v] = fmaf(t, da4[e], a[v]);
            }
        }
    };
    // activation scales of the 16 rows this lane holds in m-tile i: rows wm + 32i + 8q + 4hl + e
    auto read_da = [&](const Stage& S, int kb, int i, float4 (&da_v)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) da_v[q] = *reinterpret_cast<const float4*>(&S.da[kb][wm + 32 * i + 8 * q + 4 * hl]);
    };

    if constexpr (!DUMP) {
        // Software pipeline inside a stage: the MFMAs of block kb + 1 are issued one tile at a time,
        // each right after the epilogue of block kb has consumed that tile's registers, so the matrix
        // unit works on the next block while the VALU runs this block's epilogue (only the four
        // result tiles of one block are live). Config 5: 95.2 / 94.6 -> 93.2 / 93.8 us.
        for (int s = s_begin; s < s_end; ++s) {
            const Stage& S = st[s & 1];
            const bool more = s + 1 < s_end;
            if (more) DCQ_ISSUE(s + 1, st[(s + 1) & 1]);  // in flight while this stage computes
            v16i D[2][2];
            read_frags(S, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) D[i][j] = mfma32(fa[i], fb[j], cmagic);
#pragma unroll
            for (int kb = 0; kb < kKB; ++kb) {
                float2 wc[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) wc[j] = S.dwc[kb][wn + 32 * j + col];
                if (kb + 1 < kKB) read_frags(S, kb + 1);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    float4 da_v[4];
                    read_da(S, kb, i, da_v);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        epilogue(D[i][j], wc[j], da_v, acc[i][j]);
                        if (kb + 1 < kKB) {
                            // the empty asm ties the next MFMA behind this tile's epilogue:
                            // instruction selection orders side-effect-free operations freely, and
                            // would otherwise issue every MFMA of the stage up front
                            float* a_ = acc[i][j];
                            asm volatile(""
                                         : "+v"(a_[0]), "+v"(a_[1]), "+v"(a_[2]), "+v"(a_[3]), "+v"(a_[4]),
                                           "+v"(a_[5]), "+v"(a_[6]), "+v"(a_[7]), "+v"(a_[8]), "+v"(a_[9]),
                                           "+v"(a_[10]), "+v"(a_[11]), "+v"(a_[12]), "+v"(a_[13]), "+v"(a_[14]),
                                           "+v"(a_[15]), "+v"(fa[i]), "+v"(fb[j]));
                            D[i][j] = mfma32(fa[i], fb[j], cmagic);
                        }
                    }
                }
            }
            if (more) {
                // the other buffer was last read in stage s - 1, which every wave finished before
                // the barrier that ended stage s - 1: one barrier per stage is enough
                DCQ_COMMIT(st[(s + 1) & 1]);
                __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
                DCQ_WIDEN(st[(s + 1) & 1]);
                __syncthreads();
            }
        }
    } else {
        // Block sums (a test variant): each block's MFMAs, its dumps, then its epilogue.
        for (int s = s_begin; s < s_end; ++s) {
            const Stage& S = st[s & 1];
            const bool more = s + 1 < s_end;
            if (more) DCQ_ISSUE(s + 1, st[(s + 1) & 1]);
            read_frags(S, 0);
#pragma unroll 1
            for (int kb = 0; kb < kKB; ++kb) {
                float2 wc[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) wc[j] = S.dwc[kb][wn + 32 * j + col];
                v16i D[2][2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) D[i][j] = mfma32(fa[i], fb[j], cmagic);
                if (kb + 1 < kKB) read_frags(S, kb + 1);
                const int kblk = s * kKB + kb, nkb = K / 32;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    float4 da_v[4];
                    read_da(S, kb, i, da_v);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int n = n0 + wn + 32 * j + col;
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int m = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                            if (m < M && n < N) sums[((int64_t)m * N + n) * nkb + kblk] = D[i][j][v] - kMagic;
                        }
                        epilogue(D[i][j], wc[j], da_v, acc[i][j]);
                    }
                }
            }
            if (more) {
                DCQ_COMMIT(st[(s + 1) & 1]);
                __builtin_amdgcn_s_waitcnt(0);
                DCQ_WIDEN(st[(s + 1) & 1]);
                __syncthreads();
            }
        }
    }
#undef DCQ_ISSUE
#undef DCQ_COMMIT
#undef DCQ_WIDEN

    // ---- store: lane owns column n, rows m_v = m0 + wm + 32i + 8(v/4) + 4hl + v%4; the row
    // offsets beyond the lane's first row are uniform multiples of y_stride (scalar arithmetic) ----
    float* yl = Y + (int64_t)(m0 + wm + 4 * hl) * y_stride + (n0 + wn + col);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (!FULL && n0 + wn + 32 * j + col >= N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 32 * i + 8 * (v >> 2) + (v & 3);  // row within the wave tile, minus 4hl
                if (FULL || m0 + wm + 4 * hl + r < M) yl[(int64_t)r * y_stride + 32 * j] = acc[i][j][v];
            }
    }
}

size_t prefill_q8_0_lds_bytes() { return 2 * sizeof(Stage); }

template <int FMT>
using PrefillQ8Fn = decltype(&prefill_q8_0_kernel<false, true, FMT>);
template <int FMT>
PrefillQ8Fn<FMT> prefill_q8_pick(bool dump, bool full) {
    return dump ? (full ? prefill_q8_0_kernel<true, true, FMT> : prefill_q8_0_kernel<true, false, FMT>)
                : (full ? prefill_q8_0_kernel<false, true, FMT> : prefill_q8_0_kernel<false, false, FMT>);
}

hipError_t launch_prefill_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                               const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const SplitScratch& sc) {
    if (K % kKS || w_row_bytes % 4 || w_row_bytes > INT32_MAX || act.m_ld > INT32_MAX || N > (1 << 30) ||
        M > (1 << 30) || K > (1 << 30))
        return hipErrorNotSupported;
    // row-split weights: 16-byte pieces straight to LDS (rows 16-byte aligned), 32-bit row offsets
    if (fmt == kFmtQ8_0RS && (w_row_bytes % 16 || (uint64_t)N * (uint64_t)w_row_bytes >= (1ull << 32)))
        return hipErrorNotSupported;
    // the DMA offsets are 32-bit: every activation row, weight row and scale row must lie within 4 GiB
    if ((uint64_t)M * (uint64_t)K >= (1ull << 32) || (uint64_t)(K / 32) * (uint64_t)act.m_ld * 4 >= (1ull << 32))
        return hipErrorNotSupported;
    const int tiles_n = (int)((N + kBN - 1) / kBN), tiles_m = (int)((M + kBM - 1) / kBM);
    const size_t lds = prefill_q8_0_lds_bytes();
    const bool full = M % kBM == 0 && N % kBN == 0;
    const bool dump = block_sums != nullptr;
    auto fn = fmt == kFmtQ4_0     ? prefill_q8_pick<kFmtQ4_0>(dump, full)
              : fmt == kFmtQ8_0RS ? prefill_q8_pick<kFmtQ8_0RS>(dump, full)
                                  : prefill_q8_pick<kFmtQ8_0>(dump, full);
    // split-K when the tiles cannot fill the chip: partial planes in the scratch, then their sum
    const SplitPlan sp = plan_split_k((int64_t)tiles_n * tiles_m, (int)(K / kKS), 1, M, N, sc);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    hipLaunchKernelGGL(fn, dim3((unsigned)(tiles_n * tiles_m * sp.splits)), dim3(256), lds, st, tiles_n, tiles_m,
                       (int)N, (int)K, (int)act.m_ld, (int)w_row_bytes, (const uint8_t*)W, act.qs, act.d, (int)M,
                       sp.stps, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

}  // namespace dcq
