// dcq_batch.hip — batched-decode mul_mat (8 < M <= 64 per m-tile) for Q4_K and Q5_K weights on int8
// MFMA.
//
// Replaces ggml's CPU MUL_MAT at small M > 1 (continuous-batching decode; every M > 1
// projection goes there: core/src/inference.cpp:1049-1063, executed at
// core/src/worker.cpp:544). HBM-bound at M = 64: each weight byte feeds 64 activation
// rows, so the kernel must stream W once at full bandwidth and keep the MFMA work
// off the critical path.
//
// Launch shape. A workgroup of 8 waves owns 32 weight rows (one MFMA n-tile) and 64
// activation rows (two MFMA m-tiles; 32 rows, one m-tile, at M <= 32); its waves split K by
// superblock (wave w takes
// superblocks w, w + 8, ...). Per superblock a wave
//   - loads the 64 x 256 activation bytes and 64 scales straight into its own LDS
//     region (global_load_lds_dwordx4: coalesced, no registers in flight, no barrier:
//     only this wave reads the region), 16-byte slots XOR-swizzled by row % 16;
//   - loads its weight fragments (row = lane % 32, 16 nibble bytes per 32-element
//     sub-block half, plus the 16-byte header) into registers;
//   - runs v_mfma_i32_32x32x32_i8 per 32-element sub-block j, accumulating over the
//     superblock's eight: sum_j sc_j I_j as two MFMAs on the nibbles pre-multiplied by the
//     two halves of the 6-bit scale (sc = 8 sc_hi + sc_lo, each product <= 105 fits int8),
//     and the mins term (a weight operand whose bytes all equal m_j, so the MFMA yields
//     m_j * S_j);
//   - per superblock: acc += dA * (d * sum_j sc_j I_j - dmin * sum_j m_j S_j)
//     (vec_dot_q4_K_q8_K's per-superblock form).
// Q5_K (the Q5 variant): the level is q = nib + 16 h with h the element's qh bit, so
// sum_j sc_j I_j(q) = sum_j sc_j I_j(nib) + 16 sum_j I_j(h sc_j): one more MFMA per sub-block on
// the bytes h * sc_j (0 or sc_j <= 63), the nibble part as for Q4_K.
// The 8 partial tiles are summed in wave order through LDS at the end (deterministic), each
// wave summing an eighth of the tile. With few weight rows the superblocks are also split over
// workgroups (grid z): each stores its partial tile in a plane of the split-K scratch and
// launch_sum_splits adds them in order.
#include "dcq_common.h"
#include "dcq_kernels.h"

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma16)

namespace dcq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kWaves = 8;
// MTI m-tiles of 32 activation rows per workgroup: 2 (64 rows) in general, 1 at M <= 32
template <int MTI>
struct BGeo {
    static constexpr int kMT = 32 * MTI;                // activation rows per workgroup
    static constexpr int kRegion = kMT * 256 + 1024;    // per-wave LDS: activation + 1 KB scales
};
constexpr int kNT = 32;         // weight rows per workgroup

// 16 bytes per lane from global memory straight into LDS at base + 16 * lane (base
// wave-uniform, in M0). Inline asm: the builtin form makes the compiler wait for every
// earlier LDS-direct load before the next. The compiler does not count these loads, so
// they are issued before the ordinary loads they must precede, and the wave waits with
// an explicit s_waitcnt vmcnt(0) before reading the region. M0 has no other use here.
__device__ __forceinline__ void dma16(const void* g, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// LDS byte offset of logical 16-byte slot `slot` (0..15) of activation row `row` (256 B rows)
__device__ __forceinline__ int aswz(int row, int slot) { return row * 256 + 16 * (slot ^ (row & 15)); }

}  // namespace

template <int MTI, bool DUMP, bool Q5>
__global__ void __launch_bounds__(64 * kWaves, 1) batch_q4k_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                                   int N, int nsb, const int8_t* __restrict__ xqs,
                                                                   const float* __restrict__ xd, int64_t m_ld, int M,
                                                                   int cpz, float* __restrict__ Y, int64_t y_stride,
                                                                   int32_t* __restrict__ sums) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = nsb * 256;
    constexpr int kMT = BGeo<MTI>::kMT, kRegion = BGeo<MTI>::kRegion, kDA = kMT / 4;
    const int n0 = blockIdx.x * kNT, m0 = blockIdx.y * kMT;
    // workgroup z takes superblocks [z * cpz, (z + 1) * cpz) and stores plane z of Y (planes of M
    // rows; with one plane Y is the output itself)
    const int s_begin = blockIdx.z * cpz, s_end = min(nsb, s_begin + cpz);
    Y += (int64_t)blockIdx.z * M * y_stride;
    const int col = lane & 31, hl = lane >> 5;
    uint8_t* region = smem + wave * kRegion;
    int8_t* a_lds = reinterpret_cast<int8_t*>(region);
    float* d_lds = reinterpret_cast<float*>(region + kMT * 256);

    // activation DMA: instruction i (0..kDA-1) fills rows 4i .. 4i+3; lane l the physical slot
    // l % 16 of row 4i + l / 16, which holds logical slot (l % 16) ^ (row % 16)
    const int8_t* a_src[kDA];
#pragma unroll
    for (int i = 0; i < kDA; ++i) {
        const int row = 4 * i + (lane >> 4);
        const int slot = (lane & 15) ^ (row & 15);
        a_src[i] = xqs + (int64_t)min(m0 + row, M - 1) * K + 16 * slot;
    }
    // activation scales: lanes 0..15 carry rows 4l .. 4l+3 (the other lanes repeat lane 15)
    const float* d_src = xd + m0 + 4 * min(lane, kMT / 4 - 1);
    // weight row of this lane (MFMA B operand: column n = lane % 32)
    const uint8_t* wrow = W + (int64_t)min(n0 + col, N - 1) * w_row_bytes;

    float acc[MTI][16];
#pragma unroll
    for (int i = 0; i < MTI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    for (int s = s_begin + wave; s < s_end; s += kWaves) {
        // ---- loads: activation + scales into this wave's LDS region, weights into registers ----
#pragma unroll
        for (int i = 0; i < kDA; ++i) dma16(a_src[i] + 256 * s, a_lds + 1024 * i);
        dma16(d_src + (int64_t)s * m_ld, d_lds);
        constexpr int kSb = Q5 ? 176 : 144, kQs = Q5 ? 48 : 16;
        const uint8_t* sb = wrow + (int64_t)s * kSb;
        const uint4 hdr = ld16(sb);
        uint4 qw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) qw[c] = ld16(sb + kQs + 32 * c + 16 * hl);
        // Q5_K: qh[16hl .. 16hl + 15], the fifth bits of this lane half's elements
        [[maybe_unused]] uint4 qhw;
        if constexpr (Q5) qhw = ld16(sb + 16 + 16 * hl);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads have landed
        __builtin_amdgcn_wave_barrier();

        // 6-bit scales / mins of the 8 sub-blocks (get_scale_min_k4)
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
        const uint32_t scw[2] = {s0 & 0x3F3F3F3Fu, (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u)};
        const uint32_t mnw[2] = {s1 & 0x3F3F3F3Fu, ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u)};
        const float d = half_bits_to_float(hdr.x & 0xFFFFu), dmin = half_bits_to_float(hdr.x >> 16);
        // weight operands of the 8 sub-blocks, shared by both m-tiles. The 6-bit scale is split
        // as sc = 8 sc_hi + sc_lo (both <= 7), so sc_hi * q and sc_lo * q (<= 105) are int8
        // operands and sum_j sc_j I_j = 8 sum_j I_j(sc_hi q) + sum_j I_j(sc_lo q) accumulates
        // inside the MFMA over all eight sub-blocks. The products are formed per byte by a
        // packed 16-bit multiply (no byte carries into the next: 15 * 7 < 256). The mins operand
        // (every byte m_j) is rebuilt per use: it would hold 32 registers.
        v4i bhi[8], blo[8];
        [[maybe_unused]] v4i bhb[8];
        int mn[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 q = qw[j >> 1];
            const uint32_t sh = (j & 1) ? 4u : 0u;
            const int sc = (int)((scw[j >> 2] >> (8 * (j & 3))) & 0xFFu);
            const u16x2 s_hi = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
            const u16x2 s_lo = {(uint16_t)(sc & 7), (uint16_t)(sc & 7)};
            const uint32_t nib[4] = {(q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu, (q.z >> sh) & 0x0F0F0F0Fu,
                                     (q.w >> sh) & 0x0F0F0F0Fu};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const u16x2 b = __builtin_bit_cast(u16x2, nib[e]);
                bhi[j][e] = __builtin_bit_cast(int, (u16x2)(b * s_hi));
                blo[j][e] = __builtin_bit_cast(int, (u16x2)(b * s_lo));
            }
            if constexpr (Q5) {
                // bytes h * sc_j: bit j of each qh byte, times sc (no carries: 0 or sc <= 63)
                const uint32_t h[4] = {qhw.x, qhw.y, qhw.z, qhw.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) bhb[j][e] = (int)(((h[e] >> j) & 0x01010101u) * (uint32_t)sc);
            }
            mn[j] = (int)(((mnw[j >> 2] >> (8 * (j & 3))) & 0xFFu) * 0x01010101u);
        }
#pragma unroll
        for (int i = 0; i < MTI; ++i) {
            v16i ahi, alo, amin;
            [[maybe_unused]] v16i ahb;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                ahi[v] = 0;
                alo[v] = 0;
                amin[v] = 0;
                if constexpr (Q5) ahb[v] = 0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // activation fragment: rows 32i + col, k = 32j + 16hl .. +16 (logical slot 2j + hl)
                const v4i av = *reinterpret_cast<const v4i*>(a_lds + aswz(32 * i + col, 2 * j + hl));
                v4i bm;
                bm.x = bm.y = bm.z = bm.w = mn[j];
                ahi = mfma32(av, bhi[j], ahi);
                alo = mfma32(av, blo[j], alo);
                amin = mfma32(av, bm, amin);
                if constexpr (Q5) ahb = mfma32(av, bhb[j], ahb);
            }
            v16i ai;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                ai[v] = (ahi[v] << 3) + alo[v];
                if constexpr (Q5) ai[v] += ahb[v] << 4;
            }
            // lane owns weight row n = n0 + col and activation rows m_v = 32i + 8(v/4) + 4hl + v%4
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 dav = *reinterpret_cast<const float4*>(d_lds + 32 * i + 8 * q + 4 * hl);
                const float da4[4] = {dav.x, dav.y, dav.z, dav.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = 4 * q + e;
                    const float y = fmaf(-dmin, (float)amin[v], d * (float)ai[v]);
                    acc[i][v] = fmaf(da4[e], y, acc[i][v]);
                }
            }
            if (DUMP) {
                const int n = n0 + col;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                    if (m < M && n < N) {
                        int32_t* sp = sums + ((int64_t)m * N + n) * (2 * nsb) + 2 * s;
                        sp[0] = ai[v];
                        sp[1] = amin[v];
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the region is rewritten by the next superblock's loads
    }

    // ---- fixed-order reduction of the 8 partial tiles through LDS: each wave's partial tile
    // ([i][v][64], 8 KB) goes into its own region, which only it has read, so one barrier ----
    auto part = [&](int w) { return reinterpret_cast<float*>(smem + w * kRegion); };
#pragma unroll
    for (int i = 0; i < MTI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) part(wave)[(i * 16 + v) * 64 + lane] = acc[i][v];
    __syncthreads();
    // every wave sums 2 * MTI of the 16 * MTI (m-tile, value) pairs over the 8 partial tiles, in
    // wave order
    {
        const int n = n0 + col;
#pragma unroll
        for (int k = 0; k < 2 * MTI; ++k) {
            const int pv = wave * 2 * MTI + k, i = pv >> 4, v = pv & 15;
            float p8[kWaves];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) p8[w] = part(w)[(i * 16 + v) * 64 + lane];
            float y = p8[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) y += p8[w];
            const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
            if (m < M && n < N) Y[(int64_t)m * y_stride + n] = y;
        }
    }
}

hipError_t launch_batch_q4k(bool q5, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                            const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                            hipStream_t st, const SplitScratch& sc) {
    if (w_row_bytes % 16 || N > (1 << 30) || M > (1 << 30) || K > (1 << 30)) return hipErrorNotSupported;
    // the per-superblock scale DMA reads 64 scales at [s][m0 .. m0 + 63]: m_ld must cover the
    // last m-tile (it is M rounded up to 128)
    // 64-row m-tiles (two MFMA m-tiles per workgroup) above 32 rows, except where 64-row tiles would
    // leave CUs idle and 32-row ones give every CU at most one workgroup (4096 x 4096 at M = 64: 128
    // workgroups with split K 13.2 us, 256 of 32 rows 10.7 us; but 6144 x 4096: 192 workgroups
    // 13.5 us against 384 of 32 rows 15.7 us)
    const int forced = knob(Knob::BatchTile);
    const int64_t n_tiles = (N + kNT - 1) / kNT;
    const bool fill32 = n_tiles * ((M + 63) / 64) < cu_count() && n_tiles * ((M + 31) / 32) <= cu_count();
    const int mti = forced == 1 || forced == 2 ? forced : M <= 32 || fill32 ? 1 : 2, kMT = 32 * mti;
    if (act.m_ld < ((M + kMT - 1) / kMT) * kMT) return hipErrorNotSupported;
    const int nsb = (int)(K / 256);
    const int64_t tiles = ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT);
    // with few weight rows the superblocks are also split over workgroups (at least one per wave;
    // about 0.6 us per superblock of a workgroup: 4096 x 4096 at M = 64, 128 workgroups, 10.1 us)
    const SplitPlan sp = plan_split_k(tiles, nsb, kWaves, M, N, sc, 0.6);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    dim3 grid((unsigned)((N + kNT - 1) / kNT), (unsigned)((M + kMT - 1) / kMT), (unsigned)sp.splits);
    const size_t lds = (size_t)kWaves * (mti == 1 ? BGeo<1>::kRegion : BGeo<2>::kRegion);
    auto fn = q5 ? (mti == 1 ? (block_sums ? batch_q4k_kernel<1, true, true> : batch_q4k_kernel<1, false, true>)
                             : (block_sums ? batch_q4k_kernel<2, true, true> : batch_q4k_kernel<2, false, true>))
                 : (mti == 1 ? (block_sums ? batch_q4k_kernel<1, true, false> : batch_q4k_kernel<1, false, false>)
                             : (block_sums ? batch_q4k_kernel<2, true, false> : batch_q4k_kernel<2, false, false>));
    hipLaunchKernelGGL(fn, grid, dim3(64 * kWaves), lds, st, (const uint8_t*)W, w_row_bytes, (int)N, nsb, act.qs,
                       act.d, act.m_ld, (int)M, sp.stps, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

}  // namespace dcq
