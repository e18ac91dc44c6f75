// dcq_batch_q6.hip — batched-decode mul_mat (4 < M <= 64) for Q6_K weights on int8 MFMA.
//
// Replaces ggml's CPU MUL_MAT at small M > 1 for Q6_K weights (continuous-batching decode of a
// Q4_K_M model's ffn_down and attn_v; core/src/inference.cpp:1049-1063, executed at
// core/src/worker.cpp:544).
//
// Launch shape (the Q4_K and Q8_0 batch kernels'): a workgroup of 8 waves owns 32 weight rows
// and 32 * MTI activation rows; its waves split K by superblock (wave w takes superblocks
// w, w + 8, ... of the workgroup's range; with few weight rows the range is also split over
// workgroups, grid z, through the split-K room). Per superblock a wave
//   - loads the 32 * MTI x 256 activation bytes and scales straight into its own LDS region;
//   - loads its weight row's bits into registers. A 16-element scale group g = (half h, quarter
//     t, part p) holds elements 128h + 32t + 16p + [0, 16): low nibbles (t = 0, 1) or high
//     nibbles (t = 2, 3) of ql bytes 64h + 32(t & 1) + 16p + [0, 16), two bits 2t of qh bytes
//     128 + 32h + 16p + [0, 16). Lane half hl takes bytes [8hl, 8hl + 8) of each span, so the 24
//     bytes it loads per (h, p) serve the four quarters. Superblocks start 2 bytes into a dword
//     on odd indices: every span is read as dwords from the one at or below it and re-aligned;
//   - converts them to signed q - 32 (a v_perm table for the two high bits, v_bfi for the
//     nibble) and runs one v_mfma_i32_32x32x16_i8 per group and m-tile, the activation fragment
//     being the same 8 elements of the group (k order within a group is free: the sum is over
//     it), then iS += sc_g * I_g (v_mad_i32_i24, exact: |sc_g * I_g| < 2^23);
//   - per superblock: acc += (d * dA) * iS          (vec_dot_q6_K_q8_K's per-superblock form).
// The 8 partial tiles are summed in wave order through LDS at the end (deterministic).
#include "dcq_common.h"
#include "dcq_kernels.h"

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma16)

namespace dcq {

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kWaves = 8;
constexpr int kNT = 32;  // weight rows per workgroup

template <int MTI>
struct Geo {
    static constexpr int kMT = 32 * MTI;        // activation rows per workgroup
    static constexpr int kAct = kMT * 256;      // activation bytes per superblock
    static constexpr int kRegion = kAct + 1024; // + the superblock's activation scales (1 KB DMA)
};

// 16 bytes per lane from global memory straight into LDS at base + 16 * lane (base wave-uniform,
// in M0). Inline asm: the builtin form makes the compiler wait for every earlier LDS-direct load
// before the next. The compiler does not count these loads: the wave waits with an explicit
// s_waitcnt before reading the region. M0 has no other use here.
__device__ __forceinline__ void dma16(const void* g, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ v16i mfma32k16(long a, long b) {
    v16i z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, z, 0, 0, 0);
}

// Signed q - 32 bytes of four 6-bit quants: low nibbles from `ql` (bits 0-3 of each byte), the two
// high bits from `qh2` (bits 0-1 of each byte). (qh2 - 2) << 4 is the high nibble of q - 32: byte
// qh2 of the table 0x1000F0E0. Plain code, not an inline-asm v_bfi_b32: the result is an MFMA
// operand, and the compiler inserts the wait states between a VALU write and an MFMA read of it
// only for instructions it can see (with the asm form, an MFMA read its B operand three
// instructions after the v_bfi wrote it and summed stale bytes).
__device__ __forceinline__ uint32_t q6_minus32(uint32_t ql, uint32_t qh2) {
    const uint32_t hi = __builtin_amdgcn_perm(0u, 0x1000F0E0u, qh2);
    return (ql & 0x0F0F0F0Fu) | (hi & 0xF0F0F0F0u);
}

// LDS byte offset of logical 16-byte slot `slot` (0..15) of activation row `row` (256 B rows)
__device__ __forceinline__ int aswz(int row, int slot) { return row * 256 + 16 * (slot ^ (row & 15)); }

}  // namespace

// W: Q6_K rows (w_row_bytes % 4 == 0, 16-byte aligned base, nsb even); xqs: int8 [M][K]; xd:
// float [nsb][m_ld], m_ld >= M rounded up to the m-tile. Workgroup z computes superblocks
// [z * cpz, (z + 1) * cpz) and stores plane z of Y (planes of M rows; one plane: Y itself).
template <int MTI, bool DUMP>
__global__ void __launch_bounds__(64 * kWaves) batch_q6k_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                                int N, int nsb, int cpz,
                                                                const int8_t* __restrict__ xqs,
                                                                const float* __restrict__ xd, int64_t m_ld, int M,
                                                                float* __restrict__ Y, int64_t y_stride,
                                                                int32_t* __restrict__ sums) {
    using G = Geo<MTI>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = nsb * 256;
    const int n0 = blockIdx.x * kNT, m0 = blockIdx.y * G::kMT;
    const int s_begin = blockIdx.z * cpz, s_end = min(nsb, s_begin + cpz);
    Y += (int64_t)blockIdx.z * M * y_stride;
    const int col = lane & 31, hl = lane >> 5;
    uint8_t* region = smem + wave * G::kRegion;
    int8_t* a_lds = reinterpret_cast<int8_t*>(region);
    float* d_lds = reinterpret_cast<float*>(region + G::kAct);

    // activation DMA: instruction i fills rows 4i .. 4i+3; lane l the physical slot l % 16 of row
    // 4i + l / 16, which holds logical slot (l % 16) ^ (row % 16); rows past M repeat row M - 1
    constexpr int kDA = G::kMT / 4;
    const int8_t* a_src[kDA];
#pragma unroll
    for (int i = 0; i < kDA; ++i) {
        const int row = 4 * i + (lane >> 4);
        const int slot = (lane & 15) ^ (row & 15);
        a_src[i] = xqs + (int64_t)min(m0 + row, M - 1) * K + 16 * slot;
    }
    // activation scales: lane l carries rows 4l .. 4l+3 (lanes past the tile repeat the last four)
    const float* d_src = xd + m0 + 4 * min(lane, G::kMT / 4 - 1);
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
        // superblock s starts sh = (210 s) & 3 (0 or 2) bytes into a dword: every piece is read as
        // dwords from the one at or below it (nsb is even, so the reads past byte 209 of an even
        // superblock stay inside the next one)
        const uint32_t sh = (uint32_t)((210 * s) & 3);
        const uint8_t* sb = wrow + (int64_t)210 * s - sh;
        // pieces of (h, p): [0] ql quarter-0/2 bytes, [1] ql quarter-1/3 bytes, [2] qh bytes; 8 each
        uint32_t raw[2][2][3][3];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const int off = (k == 2 ? 128 + 32 * h : 64 * h + 32 * k) + 16 * p + 8 * hl;
                    const uint32_t* q = reinterpret_cast<const uint32_t*>(sb + off);
                    raw[h][p][k][0] = q[0];
                    raw[h][p][k][1] = q[1];
                    raw[h][p][k][2] = q[2];
                }
        const uint4 sc4 = ld16(sb + 192);
        const uint32_t sc5 = ld1(sb + 208);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads (and the rest) have landed
        __builtin_amdgcn_wave_barrier();

        // the 16 int8 group scales and d
        const uint32_t scw[4] = {align_bytes(sc4.y, sc4.x, sh), align_bytes(sc4.z, sc4.y, sh),
                                 align_bytes(sc4.w, sc4.z, sh), align_bytes(sc5, sc4.w, sh)};
        const float dw = half_bits_to_float((sc5 >> (8 * sh)) & 0xFFFFu);
        int iS[MTI][16];
#pragma unroll
        for (int i = 0; i < MTI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) iS[i][v] = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                uint32_t w[3][2];
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    w[k][0] = align_bytes(raw[h][p][k][1], raw[h][p][k][0], sh);
                    w[k][1] = align_bytes(raw[h][p][k][2], raw[h][p][k][1], sh);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int g = 8 * h + 2 * t + p;  // scale group
                    const uint32_t b0 = q6_minus32(w[t & 1][0] >> (4 * (t >> 1)), (w[2][0] >> (2 * t)) & 0x03030303u);
                    const uint32_t b1 = q6_minus32(w[t & 1][1] >> (4 * (t >> 1)), (w[2][1] >> (2 * t)) & 0x03030303u);
                    const long b = (long)(((uint64_t)b1 << 32) | b0);
                    const int sc = __builtin_amdgcn_sbfe((int)scw[g >> 2], 8 * (g & 3), 8);
#pragma unroll
                    for (int i = 0; i < MTI; ++i) {
                        // activation fragment: rows 32i + col, the same 8 elements of group g
                        const long a = *reinterpret_cast<const long*>(a_lds + aswz(32 * i + col, g) + 8 * hl);
                        const v16i I = mfma32k16(a, b);
#pragma unroll
                        for (int v = 0; v < 16; ++v) iS[i][v] = __mul24(sc, I[v]) + iS[i][v];
                    }
                }
            }
        // lane owns weight row n0 + col and activation rows 32i + 8(v/4) + 4hl + v%4
#pragma unroll
        for (int i = 0; i < MTI; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 dav = *reinterpret_cast<const float4*>(d_lds + 32 * i + 8 * q + 4 * hl);
                const float da4[4] = {dav.x, dav.y, dav.z, dav.w};
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) {
                    const int v = 4 * q + ee;
                    acc[i][v] = fmaf(dw * da4[ee], (float)iS[i][v], acc[i][v]);
                }
            }
            if (DUMP) {
                const int n = n0 + col;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                    if (m < M && n < N) sums[((int64_t)m * N + n) * nsb + s] = iS[i][v];
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the region is rewritten by the next superblock's loads
    }

    // ---- fixed-order reduction of the 8 partial tiles through LDS: each wave's partial tile
    // ([i][v][64]) goes into its own region, which only it has read, so one barrier ----
    auto part = [&](int w) { return reinterpret_cast<float*>(smem + w * G::kRegion); };
#pragma unroll
    for (int i = 0; i < MTI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) part(wave)[(i * 16 + v) * 64 + lane] = acc[i][v];
    __syncthreads();
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

hipError_t launch_batch_q6k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const PlanarBuffers& act,
                            int64_t M, float* Y, int64_t y_stride, int32_t* block_sums, hipStream_t st,
                            const SplitScratch& sc) {
    // K % 512: an even superblock count, so the dword reads past an even superblock's byte 209 stay
    // inside the next one
    if (K % 512 || w_row_bytes % 4 || w_row_bytes < K / 256 * 210 || (uintptr_t)W % 16 || M < 1 ||
        N > (1 << 30) || K > (1 << 30))
        return hipErrorNotSupported;
    // 64-row m-tiles above 32 rows, except where 32-row tiles give every CU at most one workgroup,
    // 64-row ones would leave CUs idle, and the 32-row tiles would not need split K themselves (each
    // m-tile reads the weights again, which a split does not make up for at these weights' 0.8-1.1
    // bytes per element: 2048 x 8192 Q8_0 at M = 64 17.4 -> 18.5 us). 4096 x 4096 at M = 64: Q6_K
    // 17.3 -> 13.3 us, Q8_0 16.8 -> 16.2 us; 3072 x 3072 Q8_0 15.6 -> 12.3 us; M = 48 2048 x 2048
    // Q6_K 12.9 -> 9.0 us.
    const int64_t n_tiles = (N + kNT - 1) / kNT;
    const int64_t t32 = n_tiles * ((M + 31) / 32);
    const bool fill32 = n_tiles * ((M + 63) / 64) < cu_count() && t32 <= cu_count() &&
                        (2 * t32 > cu_count() || K / 256 < 2 * kWaves);
    const int mti = M <= 32 || fill32 ? 1 : 2, mt = 32 * mti;
    const int m_tiles = (int)((M + mt - 1) / mt);
    if (act.m_ld < ((M + mt - 1) / mt) * mt) return hipErrorNotSupported;
    const int nsb = (int)(K / 256);
    const int64_t tiles_n = (N + kNT - 1) / kNT;
    // about 1 us per superblock of a workgroup (4096 x 4096 at M = 64, 128 workgroups: 16.8 us)
    const SplitPlan sp = plan_split_k(tiles_n * m_tiles, nsb, kWaves, M, N, sc, 1.0);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    dim3 grid((unsigned)tiles_n, (unsigned)m_tiles, (unsigned)sp.splits);
    const size_t lds = (size_t)kWaves * (mti == 1 ? Geo<1>::kRegion : Geo<2>::kRegion);
    auto fn = mti == 1 ? (block_sums ? batch_q6k_kernel<1, true> : batch_q6k_kernel<1, false>)
                       : (block_sums ? batch_q6k_kernel<2, true> : batch_q6k_kernel<2, false>);
    hipLaunchKernelGGL(fn, grid, dim3(64 * kWaves), lds, st, (const uint8_t*)W, w_row_bytes, (int)N, nsb, sp.stps,
                       act.qs, act.d, act.m_ld, (int)M, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

}  // namespace dcq
