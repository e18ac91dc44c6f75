// dcq_batch_q8.hip — batched-decode mul_mat (4 < M <= 64) for Q8_0 and Q4_0 weights on int8 MFMA.
//
// Replaces ggml's CPU MUL_MAT at small M > 1 for Q8_0 weights (continuous-batching decode: every
// M > 1 projection goes there, core/src/inference.cpp:1049-1063, executed at
// core/src/worker.cpp:544). HBM-bound: each weight byte feeds every activation row of the tile.
// The lane-per-block decode kernels spend VALU per activation row and, past four rows, fall
// behind; the generic MMQ kernel re-reads its operands through small tiles.
//
// Launch shape (the Q4_K batch kernel's): a workgroup of 8 waves owns 32 weight rows (one MFMA
// n-tile) and 32 * MTI activation rows (MTI MFMA m-tiles); its waves split K by chunks of 256
// elements (8 Q8_0 blocks): wave w takes chunks w, w + 8, ... of the workgroup's range. Per chunk a
// wave
//   - loads the 32 * MTI x 256 activation bytes and the 8 blocks' activation scales straight into
//     its own LDS region (global_load_lds_dwordx4; only this wave reads the region);
//   - loads its weight row's chunk (4 block pairs of 68 bytes) into registers: lane half hl takes
//     bytes 16hl .. 16hl + 16 of each block's 32 quants; an even block's quants start 2 bytes into
//     a dword (one v_alignbyte per dword), an odd block's on a dword;
//   - runs one v_mfma_i32_32x32x32_i8 per block and m-tile with the accumulator seeded with the
//     bit pattern of 1.5 * 2^23, so the int32 block sums I_b read as fp32 are 1.5*2^23 + I_b
//     (|I_b| < 2^22), and accumulates
//       acc += dA * fma(F, dW, -dW * 1.5*2^23)          (= dA * dW * I_b, vec_dot_q8_0_q8_0's form).
// Q4_0 weights (Q40): a chunk is 4 pairs of 18-byte blocks (36 bytes, 9 dwords, both lane halves
// load the pair); lane half hl takes the low (hl = 0) or high nibbles of a block's 16 bytes, its
// elements 16hl .. 16hl + 15, as signed q - 8 bytes. The rest is the Q8_0 path (|I_b| <= 32*8*128).
// Row-split Q8_0 (RS): lane half hl loads bytes 16hl .. 16hl + 16 of each block's 32 quants from the
// row's quants plane (16-byte aligned, no re-slicing) and the chunk's eight fp16 scales as one
// 16-byte load from its scales plane.
// The 8 partial tiles are summed in wave order through LDS at the end (deterministic). With few
// weight rows the chunks are also split over workgroups (grid z): each stores its partial tile in
// a plane of the split-K scratch and launch_sum_splits adds them in order.
#include "dcq_common.h"
#include "dcq_kernels.h"

#include <type_traits>

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma16)

namespace dcq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kWaves = 8;
constexpr int kNT = 32;              // weight rows per workgroup
constexpr int kMagic = 0x4B400000;   // bit pattern of 12582912.0f = 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;

template <int MTI>
struct Geo {
    static constexpr int kMT = 32 * MTI;                  // activation rows per workgroup
    static constexpr int kAct = kMT * 256;                // activation bytes per chunk
    static constexpr int kRegion = kAct + 8 * kMT * 4;    // + scales [8 blocks][kMT rows]
};

// 16 bytes per lane from global memory straight into LDS at base + 16 * lane (base wave-uniform,
// in M0). Inline asm: the builtin form makes the compiler wait for every earlier LDS-direct load
// before the next. The compiler does not count these loads: the wave waits with an explicit
// s_waitcnt before reading the region. M0 has no other use here.
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

// W: Q8_0, Q4_0 or row-split Q8_0 rows (FMT; w_row_bytes % 4 == 0, row-split % 16; 16-byte aligned
// base); xqs: int8
// [M][K]; xd: float [K/32][m_ld], m_ld >= M rounded up to the m-tile; K = 256 * nch. Workgroup z
// computes chunks [z * cpz, (z + 1) * cpz) and stores plane z of Y (planes of M rows; one plane: Y
// itself).
template <int MTI, bool DUMP, int FMT>
__global__ void __launch_bounds__(64 * kWaves) batch_q8_0_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                                 int N, int nch, int cpz,
                                                                 const int8_t* __restrict__ xqs,
                                                                 const float* __restrict__ xd, int64_t m_ld, int M,
                                                                 float* __restrict__ Y, int64_t y_stride,
                                                                 int32_t* __restrict__ sums) {
    using G = Geo<MTI>;
    constexpr bool Q40 = FMT == kFmtQ4_0, RS = FMT == kFmtQ8_0RS;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = nch * 256;
    const int n0 = blockIdx.x * kNT, m0 = blockIdx.y * G::kMT;
    const int c_begin = blockIdx.z * cpz, c_end = min(nch, c_begin + cpz);
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
    // activation scales, [8 blocks][kMT rows] floats: instruction k, lane l carries the 4 floats
    // at 256k + 4l, i.e. block (256k + 4l) / kMT, rows (256k + 4l) % kMT .. +3 (m_ld covers them)
    constexpr int kDD = 8 * G::kMT / 256;
    const float* d_src[kDD];
#pragma unroll
    for (int k = 0; k < kDD; ++k) {
        const int f = 256 * k + 4 * lane;
        d_src[k] = xd + (int64_t)(f / G::kMT) * m_ld + m0 + f % G::kMT;
    }
    // 4-row activation groups that hold rows < M: only those are loaded. The tile's other LDS rows
    // keep stale bytes, which only reach outputs of rows >= M (never stored); at M = 8 this loads 2
    // of the tile's groups instead of 8.
    const int a_groups = (min(M - m0, G::kMT) + 3) / 4;
    // weight row of this lane (MFMA B operand: column n = lane % 32)
    const uint8_t* wrow = W + (int64_t)min(n0 + col, N - 1) * w_row_bytes;

    v16i cmagic;
#pragma unroll
    for (int v = 0; v < 16; ++v) cmagic[v] = kMagic;
    asm volatile("" : "+v"(cmagic));  // kept in registers, not rematerialised per block
    float acc[MTI][16];
#pragma unroll
    for (int i = 0; i < MTI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    for (int c = c_begin + wave; c < c_end; c += kWaves) {
        // ---- loads: activation + scales into this wave's LDS region, weights into registers ----
#pragma unroll
        for (int i = 0; i < kDA; ++i)
            if (i < a_groups) dma16(a_src[i] + 256 * c, a_lds + 1024 * i);
#pragma unroll
        for (int k = 0; k < kDD; ++k) dma16(d_src[k] + (int64_t)8 * c * m_ld, d_lds + 256 * k);
        // block pair p: dwords D0..D16 at chunk byte 68p (d_even = low half of D0, the even block's
        // quants at bytes 2..33, d_odd = high half of D8, the odd block's quants at bytes 36..67).
        // Lane half hl: A = D[4hl..4hl+3], e = D[4hl+4], B = D[9+4hl..12+4hl], s = D[8 - 8hl]
        // (Q4_0: D0..D8 at chunk byte 36p, A = D0..D3, e = D4, B = D5..D8 for both halves)
        uint4 A[4], B[4];
        uint32_t e[4], sx[4];
        [[maybe_unused]] uint4 scl;
        if constexpr (RS) {
            // block 2p's half hl in A[p], block 2p + 1's in B[p]; the chunk's 8 scales in scl
            const uint8_t* cb = wrow + (int64_t)c * 256 + 16 * hl;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                A[p] = ld16(cb + 64 * p);
                B[p] = ld16(cb + 64 * p + 32);
            }
            scl = ld16(wrow + K + (int64_t)c * 16);
        } else if constexpr (Q40) {
            const uint8_t* cb = wrow + (int64_t)c * 144;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint8_t* pb = cb + 36 * p;  // dword aligned only
                const U32x4 lo = ld4(pb), hi = ld4(pb + 16);
                A[p] = make_uint4(lo.x, lo.y, lo.z, lo.w);  // D0..D3
                B[p] = make_uint4(hi.x, hi.y, hi.z, hi.w);  // D4..D7
                e[p] = ld1(pb + 32);                        // D8
            }
        } else {
            const uint8_t* cb = wrow + (int64_t)c * 272;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint8_t* pb = cb + 68 * p;
                A[p] = ld16(pb + 16 * hl);
                e[p] = ld1(pb + 16 + 16 * hl);
                B[p] = ld16(pb + 36 + 16 * hl);
                sx[p] = ld1(pb + 32 - 32 * hl);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-direct loads (and the rest) have landed
        __builtin_amdgcn_wave_barrier();

#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int p = j >> 1;
            v4i b;
            uint32_t dbits;
            if constexpr (RS) {
                const uint4 q = (j & 1) ? B[p] : A[p];
                b.x = (int)q.x, b.y = (int)q.y, b.z = (int)q.z, b.w = (int)q.w;
                const uint32_t sw = p == 0 ? scl.x : p == 1 ? scl.y : p == 2 ? scl.z : scl.w;
                dbits = (sw >> (16 * (j & 1))) & 0xFFFFu;
            } else if constexpr (Q40) {
                // A[p] = D0..D3, B[p] = D4..D7, e[p] = D8; lane half hl takes nibble half hl
                const uint32_t sh = 4u * (uint32_t)hl, m = 0x0F0F0F0Fu;
                uint32_t q[4];
                if ((j & 1) == 0) {
                    q[0] = align_bytes(A[p].y, A[p].x, 2);
                    q[1] = align_bytes(A[p].z, A[p].y, 2);
                    q[2] = align_bytes(A[p].w, A[p].z, 2);
                    q[3] = align_bytes(B[p].x, A[p].w, 2);
                    dbits = A[p].x & 0xFFFFu;
                } else {
                    q[0] = B[p].y, q[1] = B[p].z, q[2] = B[p].w, q[3] = e[p];
                    dbits = B[p].x >> 16;
                }
                b.x = (int)minus8((q[0] >> sh) & m);
                b.y = (int)minus8((q[1] >> sh) & m);
                b.z = (int)minus8((q[2] >> sh) & m);
                b.w = (int)minus8((q[3] >> sh) & m);
            } else if ((j & 1) == 0) {
                b.x = (int)align_bytes(A[p].y, A[p].x, 2);
                b.y = (int)align_bytes(A[p].z, A[p].y, 2);
                b.z = (int)align_bytes(A[p].w, A[p].z, 2);
                b.w = (int)align_bytes(e[p], A[p].w, 2);
                dbits = (hl ? sx[p] : A[p].x) & 0xFFFFu;
            } else {
                b.x = (int)B[p].x, b.y = (int)B[p].y, b.z = (int)B[p].z, b.w = (int)B[p].w;
                dbits = (hl ? e[p] : sx[p]) >> 16;
            }
            const float dw = half_bits_to_float(dbits);
            const float dwc = -dw * kMagicF;  // exact: an 11-bit significand times 3 * 2^22
#pragma unroll
            for (int i = 0; i < MTI; ++i) {
                // activation fragment: rows 32i + col, k = 32j + 16hl .. +16 (logical slot 2j + hl)
                const v4i av = *reinterpret_cast<const v4i*>(a_lds + aswz(32 * i + col, 2 * j + hl));
                const v16i D = mfma32(av, b, cmagic);
                // lane owns weight row n0 + col and activation rows 32i + 8(v/4) + 4hl + v%4
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 dav = *reinterpret_cast<const float4*>(d_lds + j * G::kMT + 32 * i + 8 * q + 4 * hl);
                    const float da4[4] = {dav.x, dav.y, dav.z, dav.w};
#pragma unroll
                    for (int ee = 0; ee < 4; ++ee) {
                        const int v = 4 * q + ee;
                        const float t = fmaf(__int_as_float(D[v]), dw, dwc);
                        acc[i][v] = fmaf(t, da4[ee], acc[i][v]);
                    }
                }
                if (DUMP) {
                    const int n = n0 + col, nkb = K / 32;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
                        if (m < M && n < N) sums[((int64_t)m * N + n) * nkb + 8 * c + j] = D[v] - kMagic;
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the region is rewritten by the next chunk's loads
    }

    // ---- fixed-order reduction of the 8 partial tiles through LDS: each wave's partial tile
    // ([i][v][64]) goes into its own region, which only it has read, so one barrier ----
    auto part = [&](int w) { return reinterpret_cast<float*>(smem + w * G::kRegion); };
#pragma unroll
    for (int i = 0; i < MTI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) part(wave)[(i * 16 + v) * 64 + lane] = acc[i][v];
    __syncthreads();
    // every wave sums 2 * MTI of the 16 * MTI (m-tile, value) pairs over the 8 partial tiles
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

hipError_t launch_batch_q8_0(int fmt, const void* W, int64_t w_row_bytes, int64_t N, int64_t K,
                             const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                             hipStream_t st, const SplitScratch& sc) {
    const bool q40 = fmt == kFmtQ4_0;
    if (K % 256 || w_row_bytes % 4 || w_row_bytes < K / 32 * (q40 ? 18 : 34) || (uintptr_t)W % 16 || M < 1 ||
        N > (1 << 30) || K > (1 << 30) || (fmt == kFmtQ8_0RS && w_row_bytes % 16))
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
    // the scale DMA reads rows m0 .. m0 + mt - 1 of every block: m_ld must cover the m-tile
    if (act.m_ld < ((M + mt - 1) / mt) * mt) return hipErrorNotSupported;
    const int nch = (int)(K / 256);
    const int64_t tiles_n = (N + kNT - 1) / kNT;
    // a chunk range per workgroup of at least one chunk per wave; about 1 us per chunk of a
    // workgroup (4096 x 4096 at M = 64, 128 workgroups of 16 chunks: 17.0 us; with 0.25 us the rule
    // left that shape and 2048 x 5632 unsplit, 2.4 - 2.9 us slower per step than two ranges)
    const SplitPlan sp = plan_split_k(tiles_n * m_tiles, nch, kWaves, M, N, sc, 1.0);
    float* out = sp.splits > 1 ? sc.p : Y;
    const int64_t out_stride = sp.splits > 1 ? N : y_stride;
    dim3 grid((unsigned)tiles_n, (unsigned)m_tiles, (unsigned)sp.splits);
    const size_t lds = (size_t)kWaves * (mti == 1 ? Geo<1>::kRegion : Geo<2>::kRegion);
    auto pick = [&](auto f) {
        constexpr int F = decltype(f)::value;
        return mti == 1 ? (block_sums ? batch_q8_0_kernel<1, true, F> : batch_q8_0_kernel<1, false, F>)
                        : (block_sums ? batch_q8_0_kernel<2, true, F> : batch_q8_0_kernel<2, false, F>);
    };
    auto fn = fmt == kFmtQ4_0     ? pick(std::integral_constant<int, kFmtQ4_0>{})
              : fmt == kFmtQ8_0RS ? pick(std::integral_constant<int, kFmtQ8_0RS>{})
                                  : pick(std::integral_constant<int, kFmtQ8_0>{});
    hipLaunchKernelGGL(fn, grid, dim3(64 * kWaves), lds, st, (const uint8_t*)W, w_row_bytes, (int)N, nch, sp.stps,
                       act.qs, act.d, act.m_ld, (int)M, out, out_stride, block_sums);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && sp.splits > 1) e = launch_sum_splits(sc.p, sp.splits, M, N, Y, y_stride, st);
    return e;
}

}  // namespace dcq
