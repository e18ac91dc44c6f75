// dcq_decode.hip — decode GEMV (M <= 8 per launch) for Q4_K weights.
//
// Replaces the per-row vec_dot loop of cb_gemv_custom (core/src/inference.cpp:896-923)
// and ggml's CPU MUL_MAT at small M (core/src/inference.cpp:1794-1797, executed at
// core/src/worker.cpp:544). HBM-bound: every weight byte is read exactly once per call.
//
// Launch shape. A 256-thread workgroup owns 4 * 64/L weight rows; each row is streamed
// by L = 4*P lanes: 4 lanes per superblock, lane c (0..3) holding the 32 nibble bytes of
// sub-blocks 2c and 2c+1 (64 weights), P superblocks of a row per step. Loads are
// coalesced (the 4 lanes of a superblock cover its 128 nibble bytes) and every weight
// load of a lane is issued up front, right after the few loads that stage the
// activation rows, so a wave makes a single round trip to HBM.
//
// Activation staging (LDS, per workgroup): either the planar Q8_K workspace written by
// the quantize kernel, or, fused, the fp32 rows themselves, quantized in the workgroup
// with the same wave quantizer (bit-identical bytes) — the fused form saves the
// separate quantize launch of a decode step.
//
// Arithmetic per lane and superblock: 16 v_dot4 over the unpacked nibbles, the two 6-bit
// sub-block scales applied to exact sums, the mins term from the 16-element bsums:
//   iA = sc_2c*I_2c + sc_2c+1*I_2c+1,  iB = m_2c*S_2c + m_2c+1*S_2c+1   (exact int32)
//   acc += dA * (d * iA - dmin * iB)      (vec_dot_q4_K_q8_K's per-superblock form)
// The 4*P lanes of a row are reduced once at the end.
#include "dcq_common.h"
#include "dcq_kernels.h"

#include <stdlib.h>

namespace dcq {

namespace {

constexpr int kWG = 256;

struct ActLds {
    int8_t* qs;   // [MT][K]
    int16_t* bs;  // [MT][K/16]
    float* d;     // [nsb][MT]
};

__device__ __forceinline__ ActLds act_lds_carve(uint8_t* smem, int MT, int K) {
    ActLds a;
    a.qs = reinterpret_cast<int8_t*>(smem);
    a.bs = reinterpret_cast<int16_t*>(smem + (size_t)MT * K);
    a.d = reinterpret_cast<float*>(smem + (size_t)MT * K + (size_t)MT * (K / 8));
    return a;
}

size_t act_lds_bytes_q8k(int MT, int64_t K) {
    return (size_t)MT * K + (size_t)MT * (K / 8) + (size_t)MT * (K / 256) * 4;
}

int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return (s && *s) ? atoi(s) : dflt;
}

}  // namespace

// Staging passes for the largest K a (P, NS) shape covers (nsb <= P*NS):
// FUSE: (superblock, m) pairs, 16 per workgroup pass (one per 16-lane DPP row);
// else: 16-byte chunks of the planar activation per thread.
__host__ __device__ constexpr int stage_chunks(int P, int NS, int MT, bool fuse) {
    return fuse ? (MT * P * NS + 15) / 16 : (MT * P * NS * 256 / 16 + kWG - 1) / kWG;
}

// FUSE: X is fp32 [M][x_stride], quantized in the workgroup; else planar Q8_K
// (xqs, xd, xbs, m_ld). M <= MT activation rows; LDS holds MT rows, rows >= M unused.
template <int P, int MT, int NS, bool FUSE, bool DUMP, int QC = stage_chunks(P, NS, MT, FUSE)>
__global__ void __launch_bounds__(kWG) decode_q4k_kernel(const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                         int64_t n0, int64_t n1, int nsb,
                                                         const float* __restrict__ X, int64_t x_stride,
                                                         const int8_t* __restrict__ xqs, const float* __restrict__ xd,
                                                         const int16_t* __restrict__ xbs, int64_t m_ld, int M,
                                                         float* __restrict__ Y, int64_t y_stride,
                                                         int32_t* __restrict__ sums, int64_t sums_n_stride) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int L = 4 * P;     // lanes per row
    constexpr int RPW = 64 / L;  // rows per wave
    const int K = nsb * 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const ActLds act = act_lds_carve(smem, MT, K);
    const int last_pair = nsb * MT - 1;

    // ---- 1. activation loads, issued first ----
    float4 xv[FUSE ? QC : 1][4];
    uint4 sq[FUSE ? 1 : QC], sb16[FUSE ? 1 : QC];
    float sd[FUSE ? 1 : QC];
    if (FUSE) {
        const int g = tid & 15;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            int pr = (tid >> 4) + 16 * i;
            pr = pr < last_pair ? pr : last_pair;
            const int s = pr / MT, m = pr % MT;  // MT is a power of two
            const float4* xp = reinterpret_cast<const float4*>(X + (int64_t)(m < M ? m : M - 1) * x_stride + 256 * s + 16 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[i][j] = xp[j];
        }
    } else {
        // rows 0..M-1 of the planar qs / bsums are contiguous; d is [nsb][m_ld]
        const int q_last = M * K / 16 - 1, b_last = M * K / 128 - 1;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int cc = tid + i * kWG;
            sq[i] = ld16(xqs + 16 * (int64_t)(cc < q_last ? cc : q_last));
            sb16[i] = ld16(xbs + 8 * (int64_t)(cc < b_last ? cc : b_last));
            const int cd = cc < last_pair ? cc : last_pair;
            const int s = cd / MT, m = cd % MT;
            sd[i] = xd[(int64_t)s * m_ld + (m < M ? m : M - 1)];
        }
    }
    // loads retire in order: keeping the activation loads ahead of the weight loads lets the
    // staging below wait for the activation only
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. every weight load of this lane ----
    const int64_t row = n0 + ((int64_t)blockIdx.x * 4 + wave) * RPW + lane / L;
    const bool row_ok = row < n1;
    const uint8_t* wrow = W + (row_ok ? row : n1 - 1) * w_row_bytes;
    const int q = lane % L, p = q >> 2, c = q & 3;
    uint4 hdr[NS], nb0[NS], nb1[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        int s = t * P + p;
        s = s < nsb ? s : nsb - 1;
        const uint8_t* sb = wrow + s * 144;
        hdr[t] = ld16(sb);
        nb0[t] = ld16(sb + 16 + 32 * c);
        nb1[t] = ld16(sb + 32 + 32 * c);
    }

    // ---- 3. activation into LDS ----
    if (FUSE) {
        const int g = tid & 15;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            int pr = (tid >> 4) + 16 * i;
            pr = pr < last_pair ? pr : last_pair;
            const int s = pr / MT, m = pr % MT;
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[4 * j] = xv[i][j].x;
                x[4 * j + 1] = xv[i][j].y;
                x[4 * j + 2] = xv[i][j].z;
                x[4 * j + 3] = xv[i][j].w;
            }
            uint32_t packed[4];
            int bsum;
            float dval;
            quantize_q8k_row16(x, g, packed, bsum, dval);
            *reinterpret_cast<uint4*>(act.qs + (size_t)m * K + 256 * s + 16 * g) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
            act.bs[m * (K / 16) + 16 * s + g] = (int16_t)bsum;
            if (g == 0) act.d[s * MT + m] = dval;
        }
    } else {
        // unconditional stores (a load used only under a branch gets sunk below the weight
        // loads); lanes past the end rewrite the last chunk with the bytes it already holds
        const int q_last = M * K / 16 - 1, b_last = M * K / 128 - 1;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const int cc = tid + i * kWG;
            *reinterpret_cast<uint4*>(act.qs + 16 * (cc < q_last ? cc : q_last)) = sq[i];
            *reinterpret_cast<uint4*>(act.bs + 8 * (cc < b_last ? cc : b_last)) = sb16[i];
            act.d[cc < last_pair ? cc : last_pair] = sd[i];
        }
    }
    __syncthreads();

    // ---- 4. per step: exact integer sums, one fp32 update per superblock ----
    const bool lo_sc = c < 2;  // sub-blocks 0..3 keep their 6 bits in one byte
    const uint32_t sh = (uint32_t)(c & 1) * 16u;
    float acc[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        const int s_raw = t * P + p;
        const bool valid = s_raw < nsb;
        const int s = valid ? s_raw : nsb - 1;
        const uint4 hd = hdr[t], w0 = nb0[t], w1 = nb1[t];
        const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;
        const uint32_t scw = lo_sc ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnw = lo_sc ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
        const int sc0 = (int)((scw >> sh) & 0xFFu), sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
        const int mn0 = (int)((mnw >> sh) & 0xFFu), mn1 = (int)((mnw >> (sh + 8)) & 0xFFu);
        const float d = half_bits_to_float(hd.x & 0xFFFFu), dmin = half_bits_to_float(hd.x >> 16);
        const uint32_t lo = 0x0F0F0F0Fu;
        const int l0 = (int)(w0.x & lo), l1 = (int)(w0.y & lo), l2 = (int)(w0.z & lo), l3 = (int)(w0.w & lo);
        const int l4 = (int)(w1.x & lo), l5 = (int)(w1.y & lo), l6 = (int)(w1.z & lo), l7 = (int)(w1.w & lo);
        const int h0 = (int)((w0.x >> 4) & lo), h1 = (int)((w0.y >> 4) & lo), h2 = (int)((w0.z >> 4) & lo),
                  h3 = (int)((w0.w >> 4) & lo);
        const int h4 = (int)((w1.x >> 4) & lo), h5 = (int)((w1.y >> 4) & lo), h6 = (int)((w1.z >> 4) & lo),
                  h7 = (int)((w1.w >> 4) & lo);
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            if (mi >= M) break;  // wave-uniform
            const int8_t* aq = act.qs + mi * K + 256 * s + 64 * c;
            const uint4 a0 = *reinterpret_cast<const uint4*>(aq);
            const uint4 a1 = *reinterpret_cast<const uint4*>(aq + 16);
            const uint4 a2 = *reinterpret_cast<const uint4*>(aq + 32);
            const uint4 a3 = *reinterpret_cast<const uint4*>(aq + 48);
            const uint2 bq = *reinterpret_cast<const uint2*>(act.bs + mi * (K / 16) + 16 * s + 4 * c);
            const float dA = act.d[s * MT + mi];
            int il = sdot4(l0, (int)a0.x, 0);
            il = sdot4(l1, (int)a0.y, il);
            il = sdot4(l2, (int)a0.z, il);
            il = sdot4(l3, (int)a0.w, il);
            il = sdot4(l4, (int)a1.x, il);
            il = sdot4(l5, (int)a1.y, il);
            il = sdot4(l6, (int)a1.z, il);
            il = sdot4(l7, (int)a1.w, il);
            int ih = sdot4(h0, (int)a2.x, 0);
            ih = sdot4(h1, (int)a2.y, ih);
            ih = sdot4(h2, (int)a2.z, ih);
            ih = sdot4(h3, (int)a2.w, ih);
            ih = sdot4(h4, (int)a3.x, ih);
            ih = sdot4(h5, (int)a3.y, ih);
            ih = sdot4(h6, (int)a3.z, ih);
            ih = sdot4(h7, (int)a3.w, ih);
            // S_2c = bsums[4c] + bsums[4c+1], S_2c+1 = bsums[4c+2] + bsums[4c+3]
            const int S0 = (int)(int16_t)(bq.x & 0xFFFFu) + (int)(int16_t)(bq.x >> 16);
            const int S1 = (int)(int16_t)(bq.y & 0xFFFFu) + (int)(int16_t)(bq.y >> 16);
            const int iA = sc0 * il + sc1 * ih;
            const int iB = mn0 * S0 + mn1 * S1;
            if (DUMP && valid && row_ok) {
                int32_t* srow = sums + ((int64_t)mi * sums_n_stride + (row - n0)) * (2 * nsb);
                atomicAdd(srow + 2 * s, iA);
                atomicAdd(srow + 2 * s + 1, iB);
            }
            const float y = fmaf(-dmin, (float)iB, d * (float)iA);
            acc[mi] = valid ? fmaf(dA, y, acc[mi]) : acc[mi];
        }
    }
    // ---- 5. reduce the L lanes of each row ----
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        float v = acc[mi];
#pragma unroll
        for (int o = L >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        acc[mi] = v;
    }
    if (q == 0 && row_ok) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
            if (mi < M) Y[(int64_t)mi * y_stride + (row - n0)] = acc[mi];
    }
}

// ------------------------------------------------------------------ dispatch
namespace {

using DecodeFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, int, const float*, int64_t, const int8_t*,
                          const float*, const int16_t*, int64_t, int, float*, int64_t, int32_t*, int64_t);

// Launch shapes (P superblocks of a row per step, NS steps): a row of nsb <= P*NS
// superblocks. Other K fall back to the generic kernel.
struct Shape {
    int P, NS;
};
constexpr Shape kShapes[] = {{8, 1}, {4, 3}, {2, 5}, {16, 1}, {4, 5}, {8, 3}, {16, 2}, {8, 5}, {8, 6}, {16, 4}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

template <int I, int MT, bool FUSE, bool DUMP>
DecodeFn fn_of() {
    return decode_q4k_kernel<kShapes[I].P, MT, kShapes[I].NS, FUSE, DUMP>;
}

template <int I, bool FUSE, bool DUMP>
DecodeFn pick_mt(int mt) {
    switch (mt) {
        case 1: return fn_of<I, 1, FUSE, DUMP>();
        case 2: return fn_of<I, 2, FUSE, DUMP>();
        case 4: return fn_of<I, 4, FUSE, DUMP>();
        default: return fn_of<I, 8, FUSE, DUMP>();
    }
}

template <bool FUSE, bool DUMP>
DecodeFn pick_shape(int idx, int mt) {
    switch (idx) {
        case 0: return pick_mt<0, FUSE, DUMP>(mt);
        case 1: return pick_mt<1, FUSE, DUMP>(mt);
        case 2: return pick_mt<2, FUSE, DUMP>(mt);
        case 3: return pick_mt<3, FUSE, DUMP>(mt);
        case 4: return pick_mt<4, FUSE, DUMP>(mt);
        case 5: return pick_mt<5, FUSE, DUMP>(mt);
        case 6: return pick_mt<6, FUSE, DUMP>(mt);
        case 7: return pick_mt<7, FUSE, DUMP>(mt);
        case 8: return pick_mt<8, FUSE, DUMP>(mt);
        default: return pick_mt<9, FUSE, DUMP>(mt);
    }
}
static_assert(kNumShapes == 10, "pick_shape covers every shape");

// The shape for nsb superblocks per row: the fewest steps (shortest waves, most of them)
// whose idle superblock slots stay within a quarter of the slots; DCQ_Q4K_SHAPE=<index>
// forces one (tuning).
int choose_shape(int nsb) {
    const int forced = env_int("DCQ_Q4K_SHAPE", -1);
    if (forced >= 0 && forced < kNumShapes && kShapes[forced].P * kShapes[forced].NS >= nsb) return forced;
    int best = -1;
    for (int pass = 0; pass < 2 && best < 0; ++pass) {
        int best_ns = 1 << 30, best_waste = 1 << 30;
        for (int i = 0; i < kNumShapes; ++i) {
            const int cap = kShapes[i].P * kShapes[i].NS;
            if (cap < nsb) continue;
            const int waste = cap - nsb;
            if (pass == 0 && 4 * waste > cap) continue;  // second pass: any shape that fits
            if (kShapes[i].NS < best_ns || (kShapes[i].NS == best_ns && waste < best_waste)) {
                best = i;
                best_ns = kShapes[i].NS;
                best_waste = waste;
            }
        }
    }
    return best;
}

hipError_t launch_q4k(bool fuse, const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                      const float* X, int64_t x_stride, const PlanarBuffers* act, int64_t M, float* Y,
                      int64_t y_stride, int32_t* block_sums, int64_t sums_n_stride, hipStream_t st) {
    const int nsb = (int)(K / 256);
    if (w_row_bytes % 16) return hipErrorNotSupported;
    const int idx = choose_shape(nsb);
    if (idx < 0) return hipErrorNotSupported;
    const int P = kShapes[idx].P;
    const int rows_per_block = 4 * (64 / (4 * P));
    const unsigned grid = (unsigned)((n1 - n0 + rows_per_block - 1) / rows_per_block);
    const int64_t per_row_sums = 2 * (K / 256);
    // validate every M tile before launching anything
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        if (act_lds_bytes_q8k(mt, K) > 64 * 1024) return hipErrorNotSupported;
        if (stage_chunks(P, kShapes[idx].NS, mt, fuse) > 16) return hipErrorNotSupported;
    }
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const size_t lds = act_lds_bytes_q8k(mt, K);
        DecodeFn fn = fuse ? (block_sums ? pick_shape<true, true>(idx, mt) : pick_shape<true, false>(idx, mt))
                           : (block_sums ? pick_shape<false, true>(idx, mt) : pick_shape<false, false>(idx, mt));
        // rows beyond mc in an MT tile stage the last real activation row and are never stored
        hipLaunchKernelGGL(fn, dim3(grid), dim3(kWG), lds, st, (const uint8_t*)W, w_row_bytes, n0, n1, nsb,
                           fuse ? X + m0 * x_stride : nullptr, x_stride, fuse ? nullptr : act->qs + m0 * K,
                           fuse ? nullptr : act->d + m0, fuse ? nullptr : act->bs + m0 * (K / 16),
                           fuse ? 0 : act->m_ld, (int)mc, Y + m0 * y_stride, y_stride,
                           block_sums ? block_sums + m0 * sums_n_stride * per_row_sums : nullptr, sums_n_stride);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_q4k(const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                             const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                             int64_t sums_n_stride, hipStream_t st) {
    return launch_q4k(false, W, w_row_bytes, n0, n1, K, nullptr, 0, &act, M, Y, y_stride, block_sums, sums_n_stride,
                      st);
}

hipError_t launch_decode_fused(int wtype, const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const float* X,
                               int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st) {
    if (wtype != kTypeQ4_K || env_int("DCQ_NO_FUSE", 0)) return hipErrorNotSupported;
    return launch_q4k(true, W, w_row_bytes, 0, N, K, X, x_stride, nullptr, M, Y, y_stride, block_sums, N, st);
}

}  // namespace dcq
