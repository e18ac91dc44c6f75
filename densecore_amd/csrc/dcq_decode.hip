// dcq_decode.hip — decode GEMV (M <= 8 per launch) for the K-quant weights (Q4_K, Q5_K, Q6_K).
//
// Replaces the per-row vec_dot loop of cb_gemv_custom (core/src/inference.cpp:896-923)
// and ggml's CPU MUL_MAT at small M (core/src/inference.cpp:1794-1797, executed at
// core/src/worker.cpp:544). HBM-bound: every weight byte is read exactly once per call.
//
// Launch shape. A 256-thread workgroup owns 4 * 64/L weight rows; each row is streamed
// by L = 4*P lanes: 4 lanes per superblock, lane c (0..3) holding the 32 nibble bytes of
// sub-blocks 2c and 2c+1 (64 weights), P superblocks of a row per step. Loads are
// coalesced (the 4 lanes of a superblock cover its 128 nibble bytes). A lane issues the
// few loads that stage the activation rows, then its weight loads for the first steps;
// the rest follow as soon as the activation is staged, before the workgroup barrier, so
// every weight load is in flight before the first step computes.
//
// Activation staging (LDS, per workgroup): either the planar Q8_K workspace written by
// the quantize kernel, or, fused, the fp32 rows themselves, quantized in the workgroup
// with the same wave quantizer (bit-identical bytes) — the fused form saves the
// separate quantize launch of a decode step.
//
// The per-format work of a lane (one quarter of a superblock, 64 weights) is a policy:
// Q4_K (144 B): lane c holds the 32 nibble bytes of sub-blocks 2c and 2c+1; 16 v_dot4,
//   the two 6-bit scales applied to exact sums, the mins term from the 16-element bsums:
//     iA = sc_2c*I_2c + sc_2c+1*I_2c+1,  iB = m_2c*S_2c + m_2c+1*S_2c+1   (exact int32)
//     acc += dA * (d * iA - dmin * iB)      (vec_dot_q4_K_q8_K's per-superblock form)
// Q5_K (176 B): as Q4_K, the levels 5-bit: lane c also holds the superblock's 32 qh bytes and
//   takes bits 2c, 2c+1 of them as bit 4 of its two sub-blocks' levels (vec_dot_q5_K_q8_K)
// Q6_K (210 B, 2-byte aligned): lane (h, lh) holds elements l in [16lh, 16lh+16) of half h
//   for all four quarters t: 16 bytes of ql low/high nibbles twice, 16 bytes of qh, the 16
//   int8 scales and d; q = (nibble | 2 qh bits << 4) - 32 with the -32 taken through the
//   bsums, 16 v_dot4:
//     iS = sum_t sc_t * (sum q6*q8 - 32 * bsum_t)                        (exact int32)
//     acc += (d * dA) * iS                   (vec_dot_q6_K_q8_K's per-superblock form)
// The 4*P lanes of a row are reduced once at the end.
#include "dcq_common.h"
#include "dcq_kernels.h"

#include <stdlib.h>

#include <atomic>
#include <type_traits>

namespace dcq {

namespace {


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


}  // namespace


// ---------------------------------------------------------------- per-format policies
// Q4_K (Q5 false) and Q5_K (Q5 true): the same header, scales and scale step
template <bool Q5>
struct FmtKq {
    static constexpr int kBytes = Q5 ? 176 : 144;  // superblock bytes
    static constexpr int kQs = Q5 ? 48 : 16;       // offset of the nibbles
    static constexpr int kSumsPerSb = 2;           // dumped int32 per superblock: sum sc*I, sum m*S
    struct Raw {
        uint4 hdr, n0, n1;
        uint4 h0, h1;  // Q5_K: qh[0..15], qh[16..31] (unused for Q4_K)
    };
    __device__ __forceinline__ static void load(const uint8_t* sb, int c, Raw& r) {
        r.hdr = ld16(sb);
        r.n0 = ld16(sb + kQs + 32 * c);
        r.n1 = ld16(sb + kQs + 16 + 32 * c);
        if constexpr (Q5) {
            r.h0 = ld16(sb + 16);
            r.h1 = ld16(sb + 32);
        }
    }
    // the levels of four elements: nibbles (shift 0: sub-block 2c, 4: sub-block 2c + 1), with the
    // qh bit of that sub-block for Q5_K
    __device__ __forceinline__ static uint32_t lv(uint32_t n, uint32_t h, uint32_t nsh, int c) {
        if constexpr (Q5)
            return q5_levels(n >> nsh, h, 2u * (uint32_t)c + (nsh >> 2));
        else
            return (n >> nsh) & 0x0F0F0F0Fu;
    }
    // exact integer sums of this lane's quarter against activation row mi; returns the fp32 term
    __device__ __forceinline__ static float dot(const Raw& r, const ActLds& act, int mi, int s, int c, int K, int MT,
                                                int nsb, int (&ints)[2]) {
        const bool lo_sc = c < 2;  // sub-blocks 0..3 keep their 6 bits in one byte
        const uint32_t sh = (uint32_t)(c & 1) * 16u;
        const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
        const uint32_t scw = lo_sc ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
        const uint32_t mnw = lo_sc ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
        const int sc0 = (int)((scw >> sh) & 0xFFu), sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
        const int mn0 = (int)((mnw >> sh) & 0xFFu), mn1 = (int)((mnw >> (sh + 8)) & 0xFFu);
        const int8_t* aq = act.qs + mi * K + 256 * s + 64 * c;
        const uint4 a0 = *reinterpret_cast<const uint4*>(aq);
        const uint4 a1 = *reinterpret_cast<const uint4*>(aq + 16);
        const uint4 a2 = *reinterpret_cast<const uint4*>(aq + 32);
        const uint4 a3 = *reinterpret_cast<const uint4*>(aq + 48);
        const uint2 bq = *reinterpret_cast<const uint2*>(act.bs + mi * (K / 16) + 16 * s + 4 * c);
        int il = sdot4((int)lv(r.n0.x, r.h0.x, 0, c), (int)a0.x, 0);
        il = sdot4((int)lv(r.n0.y, r.h0.y, 0, c), (int)a0.y, il);
        il = sdot4((int)lv(r.n0.z, r.h0.z, 0, c), (int)a0.z, il);
        il = sdot4((int)lv(r.n0.w, r.h0.w, 0, c), (int)a0.w, il);
        il = sdot4((int)lv(r.n1.x, r.h1.x, 0, c), (int)a1.x, il);
        il = sdot4((int)lv(r.n1.y, r.h1.y, 0, c), (int)a1.y, il);
        il = sdot4((int)lv(r.n1.z, r.h1.z, 0, c), (int)a1.z, il);
        il = sdot4((int)lv(r.n1.w, r.h1.w, 0, c), (int)a1.w, il);
        int ih = sdot4((int)lv(r.n0.x, r.h0.x, 4, c), (int)a2.x, 0);
        ih = sdot4((int)lv(r.n0.y, r.h0.y, 4, c), (int)a2.y, ih);
        ih = sdot4((int)lv(r.n0.z, r.h0.z, 4, c), (int)a2.z, ih);
        ih = sdot4((int)lv(r.n0.w, r.h0.w, 4, c), (int)a2.w, ih);
        ih = sdot4((int)lv(r.n1.x, r.h1.x, 4, c), (int)a3.x, ih);
        ih = sdot4((int)lv(r.n1.y, r.h1.y, 4, c), (int)a3.y, ih);
        ih = sdot4((int)lv(r.n1.z, r.h1.z, 4, c), (int)a3.z, ih);
        ih = sdot4((int)lv(r.n1.w, r.h1.w, 4, c), (int)a3.w, ih);
        // S_2c = bsums[4c] + bsums[4c+1], S_2c+1 = bsums[4c+2] + bsums[4c+3]
        const int S0 = (int)(int16_t)(bq.x & 0xFFFFu) + (int)(int16_t)(bq.x >> 16);
        const int S1 = (int)(int16_t)(bq.y & 0xFFFFu) + (int)(int16_t)(bq.y >> 16);
        const int iA = sc0 * il + sc1 * ih;
        const int iB = mn0 * S0 + mn1 * S1;
        ints[0] = iA;
        ints[1] = iB;
        const float d = half_bits_to_float(r.hdr.x & 0xFFFFu), dmin = half_bits_to_float(r.hdr.x >> 16);
        const float dA = act.d[s * MT + mi];
        return dA * fmaf(-dmin, (float)iB, d * (float)iA);
    }
};
using FmtQ4K = FmtKq<false>;
using FmtQ5K = FmtKq<true>;

struct FmtQ6K {
    static constexpr int kBytes = 210;
    static constexpr int kSumsPerSb = 1;  // sum_g sc_g * I_g
    struct Raw {
        uint32_t a[4], b[4], h[4], sc[4];
        uint32_t d;
    };
    // lane c = (h, lh): ql[64h + 16lh ..] (quarters 0/2), ql[64h + 32 + 16lh ..] (1/3),
    // qh[32h + 16lh ..], scales[16], d — every piece 2-byte aligned
    __device__ __forceinline__ static void load(const uint8_t* sb, int c, Raw& r) {
        const int h = c >> 1, lh = c & 1;
        ld16_a2(sb + 64 * h + 16 * lh, r.a);
        ld16_a2(sb + 64 * h + 32 + 16 * lh, r.b);
        ld16_a2(sb + 128 + 32 * h + 16 * lh, r.h);
        ld16_a2(sb + 192, r.sc);
        r.d = ldu16(sb + 208);
    }
    __device__ __forceinline__ static float dot(const Raw& r, const ActLds& act, int mi, int s, int c, int K, int MT,
                                                int nsb, int (&ints)[2]) {
        const int h = c >> 1, lh = c & 1;
        const int8_t* aq = act.qs + mi * K + 256 * s + 128 * h + 16 * lh;
        // bsums of groups 8h + 2t + lh, t = 0..3: int16 [16s + 8h .. +8), every other one
        const uint4 bq = *reinterpret_cast<const uint4*>(act.bs + mi * (K / 16) + 16 * s + 8 * h);
        const uint32_t bsh = (uint32_t)lh * 16u;
        const int bs[4] = {(int)(int16_t)(bq.x >> bsh), (int)(int16_t)(bq.y >> bsh), (int)(int16_t)(bq.z >> bsh),
                           (int)(int16_t)(bq.w >> bsh)};
        // scales of the same groups: bytes 8h + lh + 2t of the 16 scales
        const uint32_t scw0 = r.sc[2 * h], scw1 = r.sc[2 * h + 1];
        const uint32_t ssh = (uint32_t)lh * 8u;
        const int sc[4] = {(int)(int8_t)(scw0 >> ssh), (int)(int8_t)(scw0 >> (16 + ssh)), (int)(int8_t)(scw1 >> ssh),
                           (int)(int8_t)(scw1 >> (16 + ssh))};
        int iS = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 av = *reinterpret_cast<const uint4*>(aq + 32 * t);
            const uint32_t* src = (t & 1) ? r.b : r.a;
            const uint32_t nsh = (t >> 1) ? 4u : 0u;
            int I = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo4 = (src[i] >> nsh) & 0x0F0F0F0Fu;
                const uint32_t hi2 = ((r.h[i] >> (2 * t)) & 0x03030303u) << 4;
                const uint32_t a = i == 0 ? av.x : i == 1 ? av.y : i == 2 ? av.z : av.w;
                I = sdot4((int)(lo4 | hi2), (int)a, I);
            }
            iS += sc[t] * (I - 32 * bs[t]);
        }
        ints[0] = iS;
        ints[1] = 0;
        const float dA = act.d[s * MT + mi];
        return (half_bits_to_float(r.d) * dA) * (float)iS;
    }
};

// Waves that stage the fused activation: at most four, one per SIMD. In wider workgroups the
// last-dispatched waves would otherwise hold the barrier: their activation loads queue behind
// the earlier waves' weight loads.
__host__ __device__ constexpr int stage_waves(int NW) { return NW > 4 ? 4 : NW; }

// Staging passes for the largest K a (P, NS) shape covers (nsb <= P*NS):
// FUSE: (superblock, m) pairs, 4 per staging wave per pass (one per 16-lane DPP row);
// else: 16-byte chunks of the planar activation per thread.
__host__ __device__ constexpr int stage_chunks(int P, int NS, int MT, bool fuse, int NW) {
    return fuse ? (MT * P * NS + 4 * stage_waves(NW) - 1) / (4 * stage_waves(NW))
                : (MT * P * NS * 256 / 16 + 64 * NW - 1) / (64 * NW);
}

// FUSE: X is fp32 [M][x_stride], quantized in the workgroup; else planar Q8_K
// (xqs, xd, xbs, m_ld). M <= MT activation rows; LDS holds MT rows, rows >= M unused.
// GLU: a second weight matrix W2 of the same shape shares the activation; the output is
// silu(W x) * (W2 x) (the SwiGLU gate and up projections).
// The arguments the first loads need come first: the first 56 bytes of arguments are preloaded
// into scalar registers at dispatch (-amdgpu-kernarg-preload-count), the rest take a dependent
// scalar load.
template <class Fmt, int P, int MT, int NS, bool FUSE, bool DUMP, bool GLU = false, int NW = 4,
          int QC = stage_chunks(P, NS, MT, FUSE, NW)>
__global__ void __launch_bounds__(64 * NW) decode_kq_kernel(const float* __restrict__ X, int64_t x_stride, int M,
                                                         int nsb, const uint8_t* __restrict__ W, int64_t w_row_bytes,
                                                         int64_t n0, int64_t n1, const uint8_t* __restrict__ W2,
                                                         const int8_t* __restrict__ xqs, const float* __restrict__ xd,
                                                         const int16_t* __restrict__ xbs, int64_t m_ld,
                                                         float* Y, int64_t y_stride,  // R may alias Y
                                                         int32_t* __restrict__ sums, int64_t sums_n_stride,
                                                         const float* R, int64_t r_stride) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int L = 4 * P;     // lanes per row
    constexpr int RPW = 64 / L;  // rows per wave
    const int K = nsb * 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const ActLds act = act_lds_carve(smem, MT, K);
    const int last_pair = nsb * MT - 1;

    // ---- 1. activation loads, issued first ----
    constexpr int SW = stage_waves(NW);  // waves >= SW load (clamped pairs) but never quantize
    float4 xv[FUSE ? QC : 1][4];
    uint4 sq[FUSE ? 1 : QC], sb16[FUSE ? 1 : QC];
    float sd[FUSE ? 1 : QC];
    if (FUSE) {
        const int g = tid & 15;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            int pr = (tid >> 4) + 4 * SW * i;
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
            const int cc = tid + i * 64 * NW;
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

    // ---- 2. the weight loads of the first NA steps ----
    // The rest are issued once the activation is staged: behind every weight load of the
    // chip the activation's own load waited about 2.2 us; behind the first 40 % of them it
    // lands after about 1.45 us, and the later steps' loads still arrive before their turn
    // (config 2: 5.81 -> 5.18 us per launch).
    constexpr int NA = (2 * NS) / 5 > 0 ? (2 * NS) / 5 : 1;
    const int64_t row = n0 + ((int64_t)blockIdx.x * NW + wave) * RPW + lane / L;
    const bool row_ok = row < n1;
    const uint8_t* wrow = W + (row_ok ? row : n1 - 1) * w_row_bytes;
    const uint8_t* wrow2 = GLU ? W2 + (row_ok ? row : n1 - 1) * w_row_bytes : nullptr;
    const int q = lane % L, p = q >> 2, c = q & 3;  // superblock p of the step, quarter c
    typename Fmt::Raw raw[NS], raw2[GLU ? NS : 1];
    auto load_steps = [&](auto t0, auto t1) {
#pragma clang loop unroll(full)
        for (int t = decltype(t0)::value; t < decltype(t1)::value; ++t) {
            int s = t * P + p;
            s = s < nsb ? s : nsb - 1;
            Fmt::load(wrow + s * Fmt::kBytes, c, raw[t]);
            if constexpr (GLU) Fmt::load(wrow2 + s * Fmt::kBytes, c, raw2[t]);
        }
    };
    load_steps(std::integral_constant<int, 0>{}, std::integral_constant<int, NA>{});
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. activation into LDS ----
    if (FUSE) {
        const int g = tid & 15;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            // a wave whose four pairs all lie past the last one would only rewrite the last
            // pair's bytes: it skips the quantizer (wave-uniform), which frees its SIMD for the
            // wave that shares it (K = 2560, 5 waves: 10 pairs in 20 slots; 5.13 -> 4.96 us)
            if (wave >= SW || 4 * wave + 4 * SW * i > last_pair) continue;
            int pr = (tid >> 4) + 4 * SW * i;
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
            const int cc = tid + i * 64 * NW;
            *reinterpret_cast<uint4*>(act.qs + 16 * (cc < q_last ? cc : q_last)) = sq[i];
            *reinterpret_cast<uint4*>(act.bs + 8 * (cc < b_last ? cc : b_last)) = sb16[i];
            act.d[cc < last_pair ? cc : last_pair] = sd[i];
        }
    }
    // ---- 2b. the remaining weight loads, before the barrier ----
    __builtin_amdgcn_sched_barrier(0);
    load_steps(std::integral_constant<int, NA>{}, std::integral_constant<int, NS>{});
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if constexpr (FUSE) {
        // An empty use of each activation load after the barrier (where it has long landed):
        // with their only uses inside the skip branch above, the compiler would otherwise sink
        // the loads into it, behind the weight loads, and the activation would wait for those.
#pragma unroll
        for (int i = 0; i < QC; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) asm volatile("" ::"v"(xv[i][j].x), "v"(xv[i][j].y), "v"(xv[i][j].z), "v"(xv[i][j].w));
    }

    // ---- 4. per step: exact integer sums, one fp32 update per superblock ----
    float acc[MT], acc2[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = acc2[mi] = 0.0f;
    // fully unrolled: raw[t] must stay in registers (a rolled loop indexes it dynamically)
#pragma clang loop unroll(full)
    for (int t = 0; t < NS; ++t) {
        const int s_raw = t * P + p;
        const bool valid = s_raw < nsb;
        const int s = valid ? s_raw : nsb - 1;
        // all MT rows, also those >= M (their LDS rows hold stale bytes and their sums are
        // never stored): a guard here lets the compiler merge the unrolled steps into one
        // block fed by selects
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            int ints[2];
            const float v = Fmt::dot(raw[t], act, mi, s, c, K, MT, nsb, ints);
            if (DUMP && valid && row_ok && mi < M) {
                int32_t* srow = sums + ((int64_t)mi * sums_n_stride + (row - n0)) * (Fmt::kSumsPerSb * nsb);
#pragma unroll
                for (int k = 0; k < Fmt::kSumsPerSb; ++k) atomicAdd(srow + Fmt::kSumsPerSb * s + k, ints[k]);
            }
            acc[mi] = valid ? acc[mi] + v : acc[mi];
            if constexpr (GLU) {
                const float v2 = Fmt::dot(raw2[t], act, mi, s, c, K, MT, nsb, ints);
                acc2[mi] = valid ? acc2[mi] + v2 : acc2[mi];
            }
        }
    }
    // ---- 5. reduce the L lanes of each row ----
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        acc[mi] = lanes_sum<L>(acc[mi]);
        if constexpr (GLU) acc[mi] = silu(acc[mi]) * lanes_sum<L>(acc2[mi]);
    }
    if (q == 0 && row_ok) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
            if (mi < M)  // R (optional, may alias Y): Y = W x + R, the residual or bias add
                Y[(int64_t)mi * y_stride + (row - n0)] = R ? acc[mi] + R[(int64_t)mi * r_stride + (row - n0)] : acc[mi];
    }
}

// ------------------------------------------------------------------ dispatch
// compute units of the current device, cached per device (threads that race on the first
// call store the same value; atomics keep that well defined)
int cu_count() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        hipDeviceProp_t p;
        n = hipGetDeviceProperties(&p, dev) == hipSuccess && p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

namespace {

using DecodeFn = void (*)(const float*, int64_t, int, int, const uint8_t*, int64_t, int64_t, int64_t, const uint8_t*,
                          const int8_t*, const float*, const int16_t*, int64_t, float*, int64_t, int32_t*, int64_t,
                          const float*, int64_t);

// Launch shapes (P superblocks of a row per step, NS steps): a row of nsb <= P*NS
// superblocks. Other K fall back to the generic kernel.
struct Shape {
    int P, NS;
};
constexpr Shape kShapes[] = {{8, 1}, {4, 3}, {2, 5}, {16, 1}, {4, 5}, {8, 3}, {16, 2}, {8, 5}, {8, 6}, {16, 4}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

// waves per workgroup (measured on config 2, fused: 2 waves 6.8 us, 4 waves 6.1 us, 8 waves
// 7.05 us — 8-wave workgroups quantize the activation once per 32 weight rows instead of
// 16 but are fewer and longer-lived)
template <bool FUSE, int MT>
constexpr int waves_of() {
    return 4;
}

template <class Fmt, int I, int MT, bool FUSE, bool DUMP, bool GLU, int NW = waves_of<FUSE, MT>()>
DecodeFn fn_of() {
    return decode_kq_kernel<Fmt, kShapes[I].P, MT, kShapes[I].NS, FUSE, DUMP, GLU, NW>;
}

// the fused single-row decode (the common decode step, and the gate/up pair) also comes in
// 5-wave workgroups: rows per workgroup then spread the matrix over the CUs more evenly for some
// N (see choose_launch)
template <class Fmt, int I, bool FUSE, bool DUMP, bool GLU>
DecodeFn pick_mt(int mt, int nw) {
    if constexpr (FUSE && !DUMP) {
        if (mt == 1 && nw == 5) return fn_of<Fmt, I, 1, FUSE, DUMP, GLU, 5>();
    }
    switch (mt) {
        case 1: return fn_of<Fmt, I, 1, FUSE, DUMP, GLU>();
        case 2: return fn_of<Fmt, I, 2, FUSE, DUMP, GLU>();
        case 4: return fn_of<Fmt, I, 4, FUSE, DUMP, GLU>();
        default: return fn_of<Fmt, I, 8, FUSE, DUMP, GLU>();
    }
}

template <class Fmt, bool FUSE, bool DUMP, bool GLU = false>
DecodeFn pick_shape(int idx, int mt, int nw) {
    switch (idx) {
        case 0: return pick_mt<Fmt, 0, FUSE, DUMP, GLU>(mt, nw);
        case 1: return pick_mt<Fmt, 1, FUSE, DUMP, GLU>(mt, nw);
        case 2: return pick_mt<Fmt, 2, FUSE, DUMP, GLU>(mt, nw);
        case 3: return pick_mt<Fmt, 3, FUSE, DUMP, GLU>(mt, nw);
        case 4: return pick_mt<Fmt, 4, FUSE, DUMP, GLU>(mt, nw);
        case 5: return pick_mt<Fmt, 5, FUSE, DUMP, GLU>(mt, nw);
        case 6: return pick_mt<Fmt, 6, FUSE, DUMP, GLU>(mt, nw);
        case 7: return pick_mt<Fmt, 7, FUSE, DUMP, GLU>(mt, nw);
        case 8: return pick_mt<Fmt, 8, FUSE, DUMP, GLU>(mt, nw);
        default: return pick_mt<Fmt, 9, FUSE, DUMP, GLU>(mt, nw);
    }
}

// the gate/up pair (GLU) is built for Q4_K and Q5_K with the fused activation only
template <class Fmt>
DecodeFn pick_fn(bool fuse, bool dump, bool glu, int idx, int mt, int nw) {
    if constexpr (!std::is_same<Fmt, FmtQ6K>::value) {
        if (glu) return pick_shape<Fmt, true, false, true>(idx, mt, nw);
    }
    return fuse ? (dump ? pick_shape<Fmt, true, true>(idx, mt, nw) : pick_shape<Fmt, true, false>(idx, mt, nw))
                : (dump ? pick_shape<Fmt, false, true>(idx, mt, nw) : pick_shape<Fmt, false, false>(idx, mt, nw));
}
static_assert(kNumShapes == 10, "pick_shape covers every shape");

// The shape for nsb superblocks per row: the fewest steps (shortest waves, most of them)
// whose idle superblock slots stay within a quarter of the slots; DCQ_Q4K_SHAPE=<index>
// forces one (tuning).
int choose_shape(int nsb) {
    const int forced = knob(Knob::Q4KShape);
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

// Launch shape and waves per workgroup for the fused single-row decode. A decode GEMV streams
// each row once, and its time follows the most rows any one CU has to read (measured on
// MI355X at K = 2560: 32 rows per CU 4.7 us, 40 rows 5.7 us, 48 rows 6.0 us). Candidates: the
// shapes that leave at most a quarter of their superblock slots idle, in 4- or 5-wave
// workgroups. Many workgroups per CU cost more than their rows say (each quantizes the
// activation, and beyond what is resident they run in rounds): shapes within 15 % of the fewest
// busiest-CU rows that need at most 4 workgroups per CU come first (14336 x 4096: 60 rows in
// 3 workgroups per CU 9.05 us against 56 rows in 14, 9.74 us). Then the fewest busiest-CU rows;
// on a tie, up to 2 workgroups per CU with the most waves (9728 x 2560: 40 rows as 2 x 5 waves
// of 4 rows 4.54 us against 1 x 5 waves of 8 rows 4.68 us), else the fewest workgroups per CU
// (8192 x 2048: 32 rows as 1 workgroup 3.81 us against 4, 4.03 us). Measured with kernel
// arguments preloaded, over eight model shapes; the rule picks the fastest or within 0.15 us of
// it on each. Other variants keep choose_shape with 4 waves. (8- and 10-wave workgroups of
// 4-row waves, more waves for the same rows, measured slower: 6.3-7.0 us against 5.7 us at
// N = 9728.)
struct Launch {
    int idx, nw;
};
// nw5_max_per_cu: 5-wave candidates only up to that many workgroups per CU. Q5_K's steps hold
// 80 B per lane (Q4_K 48 B): with three or more 5-wave workgroups per CU they lose (14336 x 4096:
// {4,5} in 5 waves 13.8 us, in 4 waves 11.3 us), while at one or two per CU they still win
// (9728 x 2560 {4,3}: 5.62 against 6.01 us; 2560 x 9728 {8,5}: 6.82 against 7.79 us).
Launch choose_launch(int nsb, int64_t rows, bool nw5_ok, int64_t nw5_max_per_cu = INT64_MAX) {
    const int forced = knob(Knob::Q4KShape);
    if (forced >= 0) return {choose_shape(nsb), knob(Knob::Q4KWaves) == 5 ? 5 : 4};
    const int cus = cu_count();
    struct Cand {
        int idx, nw;
        int64_t busiest, per_cu;
    };
    Cand cands[2 * kNumShapes];
    int nc = 0;
    int64_t min_busiest = INT64_MAX;
    for (int i = 0; i < kNumShapes; ++i) {
        const int cap = kShapes[i].P * kShapes[i].NS;
        if (cap < nsb || 4 * (cap - nsb) > cap) continue;
        for (int nw = 4; nw <= (nw5_ok ? 5 : 4); ++nw) {
            const int64_t rpw = nw * (64 / (4 * kShapes[i].P));
            const int64_t wgs = (rows + rpw - 1) / rpw, per_cu = (wgs + cus - 1) / cus;
            if (nw == 5 && per_cu > nw5_max_per_cu) continue;
            cands[nc++] = {i, nw, per_cu * rpw, per_cu};
            min_busiest = cands[nc - 1].busiest < min_busiest ? cands[nc - 1].busiest : min_busiest;
        }
    }
    if (nc == 0) return {choose_shape(nsb), 4};
    auto preferred = [&](const Cand& c) { return c.per_cu <= 4 && 20 * c.busiest <= 23 * min_busiest; };
    bool any_preferred = false;
    for (int k = 0; k < nc; ++k) any_preferred |= preferred(cands[k]);
    // tie order: up to 2 workgroups per CU first, more waves per CU better; beyond, fewer workgroups
    auto tie_key = [](const Cand& c) { return c.per_cu <= 2 ? -c.per_cu * c.nw : 1000 + c.per_cu; };
    const Cand* best = nullptr;
    for (int k = 0; k < nc; ++k) {
        const Cand& c = cands[k];
        if (any_preferred && !preferred(c)) continue;
        if (!best || c.busiest < best->busiest || (c.busiest == best->busiest && tie_key(c) < tie_key(*best)))
            best = &c;
    }
    return {best->idx, best->nw};
}

// W2 != nullptr: the gate/up pair (Q4_K or Q5_K, fused activation, no block sums): Y = silu(W x) * (W2 x)
hipError_t launch_kq(int wtype, bool fuse, const void* W, const void* W2, int64_t w_row_bytes, int64_t n0, int64_t n1,
                     int64_t K, const float* X, int64_t x_stride, const PlanarBuffers* act, int64_t M, float* Y,
                     int64_t y_stride, int32_t* block_sums, int64_t sums_n_stride, hipStream_t st,
                     const float* R = nullptr, int64_t r_stride = 0) {
    const int nsb = (int)(K / 256);
    if (wtype != kTypeQ4_K && wtype != kTypeQ5_K && wtype != kTypeQ6_K) return hipErrorNotSupported;
    const bool glu = W2 != nullptr;
    if (glu && (wtype == kTypeQ6_K || !fuse || block_sums)) return hipErrorNotSupported;
    if (wtype != kTypeQ6_K ? (w_row_bytes % 16 != 0) : (w_row_bytes % 2 != 0)) return hipErrorNotSupported;
    // the 5-wave variants exist for the fused, sum-free single-row decode and the gate/up pair at
    // M = 1, which take the launch rule (the pair at config 2's shape: 7.44 -> 7.22 us with it,
    // kernel arguments preloaded); other variants keep choose_shape with 4 waves
    const bool single = fuse && !block_sums && M == 1;
    const Launch ln = single ? choose_launch(nsb, n1 - n0, true, wtype == kTypeQ5_K ? 2 : INT64_MAX)
                             : Launch{choose_shape(nsb), 4};
    const int idx = ln.idx;
    if (idx < 0) return hipErrorNotSupported;
    const int P = kShapes[idx].P;
    const int64_t per_row_sums = (wtype == kTypeQ6_K ? 1 : 2) * (K / 256);
    // validate every M tile before launching anything
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        if (act_lds_bytes_q8k(mt, K) > 64 * 1024) return hipErrorNotSupported;
        if (stage_chunks(P, kShapes[idx].NS, mt, fuse, ln.nw) > 16) return hipErrorNotSupported;
    }
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const size_t lds = act_lds_bytes_q8k(mt, K);
        const int nw = ln.nw;
        const int rows_per_block = nw * (64 / (4 * P));
        const unsigned grid = (unsigned)((n1 - n0 + rows_per_block - 1) / rows_per_block);
        DecodeFn fn = wtype == kTypeQ4_K   ? pick_fn<FmtQ4K>(fuse, block_sums != nullptr, glu, idx, mt, nw)
                      : wtype == kTypeQ5_K ? pick_fn<FmtQ5K>(fuse, block_sums != nullptr, glu, idx, mt, nw)
                                           : pick_fn<FmtQ6K>(fuse, block_sums != nullptr, false, idx, mt, nw);
        // rows beyond mc in an MT tile stage the last real activation row and are never stored
        hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * nw), lds, st, fuse ? X + m0 * x_stride : nullptr, x_stride,
                           (int)mc, nsb, (const uint8_t*)W, w_row_bytes, n0, n1, (const uint8_t*)W2,
                           fuse ? nullptr : act->qs + m0 * K, fuse ? nullptr : act->d + m0,
                           fuse ? nullptr : act->bs + m0 * (K / 16), fuse ? 0 : act->m_ld, Y + m0 * y_stride, y_stride,
                           block_sums ? block_sums + m0 * sums_n_stride * per_row_sums : nullptr, sums_n_stride,
                           R ? R + m0 * r_stride : nullptr, r_stride);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_kq(int wtype, const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                            const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                            int64_t sums_n_stride, hipStream_t st, const float* R, int64_t r_stride) {
    return launch_kq(wtype, false, W, nullptr, w_row_bytes, n0, n1, K, nullptr, 0, &act, M, Y, y_stride, block_sums,
                     sums_n_stride, st, R, r_stride);
}

hipError_t launch_decode_fused(int wtype, const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const float* X,
                               int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                               hipStream_t st, const float* R, int64_t r_stride) {
    if (knob(Knob::NoFuse)) return hipErrorNotSupported;
    if (wtype == kTypeQ8_0 || wtype == kTypeQ4_0 || wtype == kTypeQ8_0_RS)
        return launch_decode_fused_q8_0(q8_fmt(wtype), W, w_row_bytes, N, K, X, x_stride, M, Y, y_stride,
                                        block_sums, st, R, r_stride);
    if (wtype == kTypeQ6_K && !knob(Knob::Q6KDecode))
        return launch_decode_fused_q6k(W, w_row_bytes, N, K, X, x_stride, M, Y, y_stride, block_sums, st, R,
                                       r_stride);
    if (wtype != kTypeQ4_K && wtype != kTypeQ5_K && wtype != kTypeQ6_K) return hipErrorNotSupported;
    return launch_kq(wtype, true, W, nullptr, w_row_bytes, 0, N, K, X, x_stride, nullptr, M, Y, y_stride, block_sums,
                     N, st, R, r_stride);
}

hipError_t launch_decode_fused_glu(int wtype, const void* Wg, const void* Wu, int64_t w_row_bytes, int64_t N, int64_t K,
                                   const float* X, int64_t x_stride, int64_t M, float* Y, int64_t y_stride,
                                   hipStream_t st) {
    if (knob(Knob::NoFuse)) return hipErrorNotSupported;
    if (wtype == kTypeQ8_0 || wtype == kTypeQ4_0)
        return launch_decode_fused_q8_0_glu(q8_fmt(wtype), Wg, Wu, w_row_bytes, N, K, X, x_stride, M, Y,
                                            y_stride, st);
    if (wtype != kTypeQ4_K && wtype != kTypeQ5_K) return hipErrorNotSupported;
    return launch_kq(wtype, true, Wg, Wu, w_row_bytes, 0, N, K, X, x_stride, nullptr, M, Y, y_stride, nullptr, N, st);
}

}  // namespace dcq
