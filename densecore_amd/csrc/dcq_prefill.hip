// dcq_prefill.hip — prefill / batched mul_mat for Q8_0 weights on gfx950 int8 MFMA.
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
// (global_load_lds_dwordx4, no registers in flight); weight block pairs pass through
// registers to be re-sliced. LDS rows are 128 bytes whose 16-byte slots are XOR-swizzled
// by row % 8, so the 32 rows a ds_read_b128 touches spread over the banks.
//
// Epilogue per MFMA (16 values per lane; lane = one weight row n, 16 activation rows m):
// the accumulator is seeded with the bit pattern of 1.5 * 2^23, so the int32 result read
// as fp32 is exactly 1.5*2^23 + I (|I| <= 32*127*128 < 2^22); then
//   t = fma(F, dW, -dW * 1.5*2^23)   (= dW * I, rounded once)
//   acc = fma(t, dA, acc)
// two VALU ops per value per block — the bound of this kernel (VALU at 4 cycles per
// wave64 op against 32 cycles per MFMA: 25 % of the int8 MFMA peak without packed fp32).
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
constexpr int kRow = kKS;            // LDS row: 8 slots of 16 bytes, slot index XOR (row % 8)
constexpr int kMagic = 0x4B400000;   // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;
constexpr int kXcds = 8;

struct __align__(16) Stage {
    int8_t a[kBM * kRow];  // activation int8, [m][k] (swizzled 16-byte slots)
    int8_t b[kBN * kRow];  // weight int8, [n][k] (swizzled 16-byte slots)
    float dw[kKB][kBN];    // weight block scales (fp16 widened)
    float da[kKB][kBM];    // activation block scales
};

// LDS byte offset of logical 16-byte slot `slot` (= 2*block + half) of tile row `row`.
__device__ __forceinline__ int swz(int row, int slot) { return row * kRow + 16 * (slot ^ (row & 7)); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS at base + 16 * lane (base
// wave-uniform, in M0): global_load_lds_dwordx4, no registers held while in flight.
// Written as inline asm because the compiler's builtin form waits for every earlier
// LDS-direct load before the next one (it cannot tell the destinations apart). The
// compiler does not count these loads, so every call must precede the ordinary loads
// of the same stage (loads retire in order, so its own vmcnt waits stay conservative),
// and the stage ends with an explicit s_waitcnt vmcnt(0) before the barrier. M0 has no
// other use in this kernel.
__device__ __forceinline__ void dma16(const void* g, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

}  // namespace

// fragments of one block for a wave's 2 x 2 MFMA tiles: A (2 m-tiles), B (2 n-tiles) and
// the weight scales of the B rows
struct Frag {
    v4i a[2], b[2];
    float dw[2];
};

__device__ __forceinline__ void load_frag(const Stage& S, int kb, int wm, int wn, int col, int hl, Frag& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
        f.a[i] = *reinterpret_cast<const v4i*>(S.a + swz(wm + 32 * i + col, 2 * kb + hl));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        f.b[j] = *reinterpret_cast<const v4i*>(S.b + swz(wn + 32 * j + col, 2 * kb + hl));
        f.dw[j] = S.dw[kb][wn + 32 * j + col];
    }
}

// One block's MFMAs and epilogue for the wave's 2 x 2 tiles.
template <bool DUMP>
__device__ __forceinline__ void block_step(const Stage& S, int kb, const Frag& f, const v16i& cmagic, int wm, int col,
                                           int hl, float (&acc)[2][2][16], int32_t* sums, int m_base, int n_base,
                                           int M, int N, int nkb, int kblk) {
    float cw[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) cw[j] = -f.dw[j] * kMagicF;  // exact: 11-bit significand times 3*2^22
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const v16i D0 = mfma32(f.a[i], f.b[0], cmagic);
        const v16i D1 = mfma32(f.a[i], f.b[1], cmagic);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v4 = *reinterpret_cast<const float4*>(&S.da[kb][wm + 32 * i + 8 * q + 4 * hl]);
            const float da4[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 4 * q + e;
                const float t0 = fmaf(__int_as_float(D0[v]), f.dw[0], cw[0]);
                acc[i][0][v] = fmaf(t0, da4[e], acc[i][0][v]);
                const float t1 = fmaf(__int_as_float(D1[v]), f.dw[1], cw[1]);
                acc[i][1][v] = fmaf(t1, da4[e], acc[i][1][v]);
            }
        }
        if (DUMP) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n_base + 32 * j + col;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = m_base + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                    const int I = (j == 0 ? D0[v] : D1[v]) - kMagic;
                    if (m < M && n < N) sums[((int64_t)m * N + n) * nkb + kblk] = I;
                }
            }
        }
    }
}

// W: Q8_0 rows (w_row_bytes % 4 == 0); xqs: int8 [M][K]; xd: float [K/32][m_ld]; K % 128 == 0.
template <bool DUMP>
__global__ void __launch_bounds__(256, 2) prefill_q8_0_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                              int N, int K, const int8_t* __restrict__ xqs,
                                                              const float* __restrict__ xd, int64_t m_ld, int M,
                                                              float* __restrict__ Y, int64_t y_stride,
                                                              int32_t* __restrict__ sums, int tiles_n, int tiles_m) {
    extern __shared__ __align__(16) uint8_t smem[];
    Stage* st = reinterpret_cast<Stage*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- XCD-aware tile order: XCD x (= id % 8) takes n-tile band x, walked m-first ----
    const int bid = blockIdx.x;
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
    const int nkb = K / 32;
    const int nstages = K / kKS;

    // ---- staging assignment ----
    // activation rows: straight to LDS, 4 x 1 KB per wave per stage; instruction i of wave w
    // fills tile rows 8*(4w+i) .. +8, lane l the 16-byte slot (l % 8) of row 8*(4w+i) + l/8,
    // which holds logical slot (l % 8) ^ (row % 8)
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // instruction i: rows 8*(4w + i) + lane/8 share the slot pattern; one base row pointer,
    // the other rows at +8*K per instruction (rows past M clamp to M - 1)
    const int a_row0 = 8 * (4 * wave_u) + (lane >> 3);
    const int a_slot = (lane & 7) ^ (a_row0 & 7);
    // activation scales: waves 0 and 1, one 1 KB instruction each: lane l of wave w holds
    // block (64w + l) / 32, rows 4 * ((64w + l) % 32) .. +4
    const int dc = 64 * (wave_u & 1) + lane;
    const float* da_src = xd + (int64_t)(dc >> 5) * m_ld + m0 + 4 * (dc & 31);
    // weight rows: row rw = tid / 2, block pair (tid & 1) * 2 of the stage (68 bytes), through
    // registers (the 34-byte blocks are re-sliced into int8 rows and fp32 scales)
    const int rw = tid >> 1, hw = tid & 1;
    const uint8_t* w_src = W + (int64_t)min(n0 + rw, N - 1) * w_row_bytes + hw * 68;
    uint32_t gw[17];
#define DCQ_ISSUE(s_, S_)                                                                      \
    do {                                                                                       \
        _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                                       \
            dma16(xqs + (int64_t)min(m0 + a_row0 + 8 * i_, M - 1) * K + 16 * a_slot + (s_) * kKS, \
                  (S_).a + 1024 * (4 * wave_u + i_));                                          \
        if (wave_u < 2) dma16(da_src + (int64_t)(s_) * kKB * m_ld, &(S_).da[0][0] + 256 * wave_u); \
        const uint8_t* wp_ = w_src + (int64_t)(s_) * (kKB * 34);                               \
        _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_) {                                     \
            const U32x4 v_ = ld4(wp_ + 16 * i_);                                               \
            gw[4 * i_] = v_.x;                                                                 \
            gw[4 * i_ + 1] = v_.y;                                                             \
            gw[4 * i_ + 2] = v_.z;                                                             \
            gw[4 * i_ + 3] = v_.w;                                                             \
        }                                                                                      \
        gw[16] = ld1(wp_ + 64);                                                                \
    } while (0)
    // weight block pair bytes: [0,2) d0, [2,34) q0, [34,36) d1, [36,68) q1 (dword aligned);
    // logical slots 4hw .. 4hw+3 of row rw
#define DCQ_COMMIT(S_)                                                                         \
    do {                                                                                       \
        *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw)) =                                  \
            make_uint4(align_bytes(gw[1], gw[0], 2), align_bytes(gw[2], gw[1], 2),              \
                       align_bytes(gw[3], gw[2], 2), align_bytes(gw[4], gw[3], 2));            \
        *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 1)) =                              \
            make_uint4(align_bytes(gw[5], gw[4], 2), align_bytes(gw[6], gw[5], 2),              \
                       align_bytes(gw[7], gw[6], 2), align_bytes(gw[8], gw[7], 2));            \
        *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 2)) = make_uint4(gw[9], gw[10], gw[11], gw[12]); \
        *reinterpret_cast<uint4*>((S_).b + swz(rw, 4 * hw + 3)) = make_uint4(gw[13], gw[14], gw[15], gw[16]); \
        (S_).dw[2 * hw][rw] = half_bits_to_float(gw[0] & 0xFFFFu);                            \
        (S_).dw[2 * hw + 1][rw] = half_bits_to_float(gw[8] >> 16);                            \
    } while (0)

    // ---- wave tile: 64 x 64 at (wm, wn) inside the workgroup tile ----
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int col = lane & 31, hl = lane >> 5;
    v16i cmagic;
#pragma unroll
    for (int v = 0; v < 16; ++v) cmagic[v] = kMagic;
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    DCQ_ISSUE(0, st[0]);
    DCQ_COMMIT(st[0]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
    __syncthreads();

    for (int s = 0; s < nstages; ++s) {
        const Stage& S = st[s & 1];
        const bool more = s + 1 < nstages;
        if (more) DCQ_ISSUE(s + 1, st[(s + 1) & 1]);  // in flight while this stage computes
        // software pipeline over the stage's blocks: the next block's fragments are read
        // from LDS while this block's MFMAs and epilogue run (two named fragment sets)
        Frag f0, f1;
        load_frag(S, 0, wm, wn, col, hl, f0);
#pragma unroll 1
        for (int kb = 0; kb < kKB; kb += 2) {
            load_frag(S, kb + 1, wm, wn, col, hl, f1);
            block_step<DUMP>(S, kb, f0, cmagic, wm, col, hl, acc, sums, m0 + wm, n0 + wn, M, N, nkb, s * kKB + kb);
            if (kb + 2 < kKB) load_frag(S, kb + 2, wm, wn, col, hl, f0);
            block_step<DUMP>(S, kb + 1, f1, cmagic, wm, col, hl, acc, sums, m0 + wm, n0 + wn, M, N, nkb,
                             s * kKB + kb + 1);
        }
        if (more) {
            // the other buffer was last read in stage s - 1, which every wave finished before
            // the barrier that ended stage s - 1: one barrier per stage is enough
            DCQ_COMMIT(st[(s + 1) & 1]);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
            __syncthreads();
        }
    }
#undef DCQ_ISSUE
#undef DCQ_COMMIT

    // ---- store: lane owns column n, rows m_v ----
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + 32 * j + col;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (m < M) Y[(int64_t)m * y_stride + n] = acc[i][j][v];
            }
    }
}

size_t prefill_q8_0_lds_bytes() { return 2 * sizeof(Stage); }

hipError_t launch_prefill_q8_0(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                               int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st) {
    if (K % kKS || w_row_bytes % 4 || N > (1 << 30) || M > (1 << 30) || K > (1 << 30)) return hipErrorNotSupported;
    const int tiles_n = (int)((N + kBN - 1) / kBN), tiles_m = (int)((M + kBM - 1) / kBM);
    const size_t lds = prefill_q8_0_lds_bytes();
    auto fn = block_sums ? prefill_q8_0_kernel<true> : prefill_q8_0_kernel<false>;
    hipLaunchKernelGGL(fn, dim3((unsigned)(tiles_n * tiles_m)), dim3(256), lds, st, (const uint8_t*)W, w_row_bytes,
                       (int)N, (int)K, act.qs, act.d, act.m_ld, (int)M, Y, y_stride, block_sums, tiles_n, tiles_m);
    return hipGetLastError();
}

}  // namespace dcq
