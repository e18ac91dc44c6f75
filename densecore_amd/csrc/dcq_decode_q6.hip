// dcq_decode_q6.hip — decode GEMV (M <= 8 per launch) for Q6_K weights, rows staged in LDS.
//
// Replaces the per-row vec_dot_q6_K_q8_K loop of cb_gemv_custom (core/src/inference.cpp:
// 896-923) and ggml's CPU MUL_MAT at small M (core/src/inference.cpp:1794-1797, executed at
// core/src/worker.cpp:544) for Q6_K weights. HBM-bound: each weight byte is read once.
//
// Why LDS. A Q6_K superblock is 210 bytes, so every other superblock of a row starts two
// bytes off a dword, and the pieces a lane needs (ql, qh, scales, d) lie 64..208 bytes
// apart: loading them straight into lanes spreads each wave instruction over many cache
// lines. Here each wave copies one weight row into LDS with direct-to-LDS loads (no
// registers held in flight): 16-byte loads (global_load_lds_dwordx4, 1 KB per wave
// instruction) over the row's 16-byte aligned interior, one dword load instruction each
// for the unaligned head and tail (global_load_lds_dword, 256 B, written over the same
// bytes the 16-byte loads write — equal values). The row's LDS image is placed so that
// 16-byte aligned global addresses land on 16-byte aligned LDS addresses. The planar Q8_K
// activation (qs, bsums, d) is staged once per workgroup, shared by its waves.
//
// Steps. Loads retire in order, so a wave computes superblocks 16k .. 16k+15 as soon as
// the loads holding their bytes have landed (s_waitcnt vmcnt on the count issued after
// them) while the rest of its row is still streaming.
//
// Dot. Lane = unit (superblock s, quarter c = (h, lh)): elements l in [16lh, 16lh+16) of
// half h for the four quarters t: ql low/high nibbles, 2 qh bits, q = (nibble | qh << 4) - 32
// with the -32 taken through the 16-element bsums:
//   iS = sum_t sc_t * (sum q6*q8 - 32 * bsum_t)                     (exact int32)
//   y += (d * dA) * iS                          (vec_dot_q6_K_q8_K's per-superblock form)
// Pieces are read from the dword at or below them and re-aligned with v_alignbyte; the
// 6-bit values are assembled with one v_bfi_b32 each from the nibble and the qh bit pair.
#include "dcq_common.h"
#include "dcq_kernels.h"

#include <stdlib.h>

#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list (see dma4)

namespace dcq {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Direct-to-LDS loads: lane l writes base + 4*l (dword) or base + 16*l (dwordx4), base
// wave-uniform in M0. Inline asm: the builtin form makes the compiler wait for all of them
// (vmcnt(0)) before any later use of an ordinary load. The compiler does not count these loads;
// the kernel waits with explicit s_waitcnt. M0 has no other use in the kernel.
// PRIVATE: the destination is the issuing wave's own row image, read only by that wave after its
// own counted wait, and the load may stay in flight across a workgroup barrier. The asm carries a
// "; wave-private" comment so that the assembly scan in tests/test_isa_hazards.py exempts it from
// the rule that a barrier must follow a wait for every earlier direct-to-LDS load.
template <bool PRIVATE = false>
__device__ __forceinline__ void dma4(const void* g, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    if constexpr (PRIVATE)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off ; wave-private" ::"v"(g), "s"(m0)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
// global address 16-byte aligned, base 16-byte aligned
template <bool PRIVATE = false>
__device__ __forceinline__ void dma16(const void* g, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    if constexpr (PRIVATE)
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off ; wave-private" ::"v"(g), "s"(m0)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}

// A 16-byte global load the compiler does not track, for loads that must sit in the same
// in-order queue as the direct-to-LDS loads above: its value may be read only after an explicit
// wait that covers it, followed by a sched_barrier (the compiler takes the result as ready).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 gload16_untracked(const void* g) {
    u32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(g) : "memory");
    return r;
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt fields at their maxima: no wait on them)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
// s_waitcnt vmcnt(n) for a wave-uniform n in [LO, HI]: binary search over the immediates
template <int LO, int HI>
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
    if constexpr (LO == HI) {
        wait_vmcnt<LO>();
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (n <= MID)
            wait_vmcnt_rt<LO, MID>(n);
        else
            wait_vmcnt_rt<MID + 1, HI>(n);
    }
}
// The counted wait for the loads issued before the last n. The ";dcq counted wait" comment after
// it marks its end in the assembly: the binary search has branches that the assembly scan in
// tests/test_isa_hazards.py cannot evaluate, so the scan takes the marker as the wait and checks
// that no instruction touches the registers of an untracked load, and no barrier follows a
// direct-to-LDS load, on any path before it.
__device__ __forceinline__ void counted_wait(int n) {
    wait_vmcnt_rt<0, 63>(n);
    asm volatile(";dcq counted wait");
}

// (a & m) | (b & ~m) as one v_bfi_b32 (the compiler otherwise re-derives the masks)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// 16 bytes at a 2-byte aligned LDS address p: five dwords from the dword at or below p
// (the fifth may lie past the piece: LDS rows are padded), shifted by (p & 2) bytes.
__device__ __forceinline__ void lds16_a2(const uint8_t* p, uint32_t (&out)[4]) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 2u;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
    out[0] = align_bytes(w1, w0, sh);
    out[1] = align_bytes(w2, w1, sh);
    out[2] = align_bytes(w3, w2, sh);
    out[3] = align_bytes(w4, w3, sh);
}
__device__ __forceinline__ void lds8_a2(const uint8_t* p, uint32_t (&out)[2]) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 2u;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    out[0] = align_bytes(w1, w0, sh);
    out[1] = align_bytes(w2, w1, sh);
}


// weight rows per workgroup: one per wave (kWaves, 4 at every launch)
constexpr int kSbStep = 16;    // superblocks per step: 4 lanes each, one wave
constexpr int kMaxNsb = 64;    // K <= 16384: the scales gather is one dword instruction
constexpr size_t kMaxLds = 160 * 1024;

// LDS carve-up, every region a whole number of its DMA instructions (lanes past a region's
// end write duplicates into its padding). Activation (shared): qs [MT][q_ld] (1 KB pieces),
// bsums [MT][b_ld bytes] (1 KB pieces), d [MT][64] floats; then one row image per wave.
struct Q6Lds {
    int q_ld, b_ld, pitch;
    size_t act_bytes, total;
    // nbuf: row images per wave (2 when a wave streams several rows: the next one lands while the
    // current one computes)
    __host__ __device__ Q6Lds(int nsb, int MT, int nw, int nbuf = 1) {
        q_ld = (int)round_up(256 * nsb, 1024);
        b_ld = (int)round_up(32 * nsb, 1024);
        // image at 16 - head (head < 16): 16 + 16-byte interior (1 KB pieces) + the tail dwords
        pitch = (int)round_up(16 + round_up(210 * nsb, 1024) + 256, 256);
        act_bytes = (size_t)MT * (q_ld + b_ld + 256);
        total = act_bytes + (size_t)nw * nbuf * pitch;
    }
};

}  // namespace

// FUSE: X is fp32 [M][x_stride] and the workgroup quantizes it to Q8_K in LDS (the same wave
// quantizer as the fused Q4_K decode: bit-identical bytes), saving the separate quantize
// launch. Its loads are untracked inline-asm loads issued before the row's direct-to-LDS
// loads: loads retire in order, so an explicit wait for all but the row's loads covers them,
// and the quantizer runs while the row streams. The first SW waves stage the activation, QC
// passes of 4 * SW (superblock, row) pairs; the other waves only stream their rows.
// The arguments the first loads need come first: the first 56 bytes of arguments are preloaded
// into scalar registers at dispatch (-amdgpu-kernarg-preload-count), the rest take a dependent
// scalar load.
template <int MT, bool DUMP, bool FUSE = false, int QC = 1, int kWaves = 4, int SW = kWaves>
__global__ void __launch_bounds__(64 * kWaves) decode_q6k_lds_kernel(
    const float* __restrict__ X, int64_t x_stride, const uint8_t* __restrict__ W, int64_t n0, int64_t n1,
    int w_row_bytes, int M, int nsb, int rpw, const int8_t* __restrict__ xqs, const float* __restrict__ xd,
    const int16_t* __restrict__ xbs, int64_t m_ld, float* Y, int64_t y_stride, int32_t* __restrict__ sums,
    int64_t sums_n_stride, const float* R, int64_t r_stride) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nbuf = rpw > 1 ? 2 : 1;
    const Q6Lds L(nsb, MT, kWaves, nbuf);
    const int K = 256 * nsb;
    const int row_bytes = 210 * nsb, row_dw = row_bytes / 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int8_t* aq = reinterpret_cast<int8_t*>(smem);
    int8_t* abb = reinterpret_cast<int8_t*>(smem + (size_t)MT * L.q_ld);
    float* ad = reinterpret_cast<float*>(smem + (size_t)MT * (L.q_ld + L.b_ld));
    uint8_t* const lw0 = smem + L.act_bytes + (size_t)wave * nbuf * L.pitch;
    // this wave's rows: row0 + j * kWaves for j < rpw (for a fixed j the workgroup's waves read
    // consecutive rows)
    const int64_t row0 = n0 + (int64_t)blockIdx.x * kWaves * rpw + wave;

    // ---- 1. activation share: qs and bsums in 1 KB pieces, the scales gathered ----
#pragma unroll
    for (int mi = 0; mi < (FUSE ? 0 : MT); ++mi) {
        const int m = mi < M ? mi : M - 1;
        const int8_t* qsrc = xqs + (int64_t)m * K;
        for (int part = wave; part * 1024 < K; part += kWaves) {
            const int c = 64 * part + lane, c_last = K / 16 - 1;
            dma16(qsrc + 16 * (c < c_last ? c : c_last), aq + mi * L.q_ld + 1024 * part);
        }
        const int8_t* bsrc = reinterpret_cast<const int8_t*>(xbs + (int64_t)m * (K / 16));
        for (int part = wave; part * 1024 < K / 8; part += kWaves) {
            const int c = 64 * part + lane, c_last = K / 128 - 1;
            dma16(bsrc + 16 * (c < c_last ? c : c_last), abb + mi * L.b_ld + 1024 * part);
        }
        if (wave == mi % kWaves) dma4(xd + (int64_t)(lane < nsb ? lane : nsb - 1) * m_ld + m, ad + 64 * mi);
    }

    // ---- 1b. fused: the fp32 activation, issued ahead of the row so that it lands first ----
    [[maybe_unused]] u32x4 xr[FUSE ? QC : 1][4];
    const bool stager = wave < SW;  // wave-uniform
    if constexpr (FUSE) {
        const int g = threadIdx.x & 15, last_pair = nsb * MT - 1;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            if (!stager) break;
            int pr = (threadIdx.x >> 4) + 4 * SW * i;
            pr = pr < last_pair ? pr : last_pair;
            const int s = pr / MT, m = pr % MT;  // MT is a power of two
            const float* xp = X + (int64_t)(m < M ? m : M - 1) * x_stride + 256 * s + 16 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[i][j] = gload16_untracked(xp + 4 * j);
        }
    }

    // ---- 2. this wave's row: head dwords, 16-byte interior, tail dwords ----
    // row byte b sits at img + b; img + head is 16-byte aligned like src + head
    struct RowImg {
        const uint8_t* src;
        uint8_t* lw;
        uint8_t* img;
        int head, nfull, nx4, issued;
    };
    auto row_image = [&](int64_t row, uint8_t* lw) {
        RowImg r;
        r.src = W + (row < n1 ? row : n1 - 1) * w_row_bytes;
        r.head = (int)((16u - ((uint32_t)(uintptr_t)r.src & 15u)) & 15u);
        r.lw = lw;
        r.img = lw + 16 - r.head;
        r.nfull = (row_bytes - r.head) / 16;  // whole 16-byte chunks after the head
        r.nx4 = (r.nfull + 63) / 64;
        r.issued = r.nx4 + 2;  // every row load, in issue order: head, pieces, tail
        return r;
    };
    const int tail0 = row_dw > 64 ? row_dw - 64 : 0;
    auto issue_head = [&](const RowImg& r) { dma4<true>(r.src + 4 * (lane < row_dw ? lane : row_dw - 1), r.img); };
    auto issue_pieces = [&](const RowImg& r, int j0, int j1) {
        for (int j = j0; j < j1; ++j) {
            const int c = 64 * j + lane;
            dma16<true>(r.src + r.head + 16 * (c < r.nfull ? c : r.nfull - 1), r.lw + 16 + 1024 * j);
        }
    };
    auto issue_tail = [&](const RowImg& r) {
        dma4<true>(r.src + 4 * (tail0 + lane < row_dw ? tail0 + lane : row_dw - 1), r.img + 4 * tail0);
    };
    RowImg cur = row_image(row0, lw0);
    const int issued = cur.issued;
    // fused workgroups of 8+ waves (K > 4096): only the head and the first 40 % of the row go
    // out before the activation is waited for (fewer loads ahead of it), the rest once it is
    // quantized (measured at M = 1: 2560 x 9728 9.5 -> 8.7 us; with 4-wave workgroups rows of
    // three 1 KB pieces lose: 1024 x 2560 3.8 -> 4.2 us)
    // Waves past the first SW stage nothing and issue the whole row at once. The launcher has
    // every wave stage: one quantizer pass each instead of three on four staging waves
    // (2560 x 9728: 7.94-8.04 -> 7.71-7.72 us; the early share of the row then measured best at
    // 40 %: 20 % 7.99, 50 % 7.86, 60 % 7.88, the whole row 8.40 us).
    constexpr bool split = FUSE && kWaves > 4;
    const int n_early = split && stager ? (2 * cur.nx4) / 5 : cur.nx4;
    issue_head(cur);
    issue_pieces(cur, 0, n_early);
    if (!split || !stager) issue_tail(cur);
    // One counted wait on every path. A staging wave of the fused form waits for its activation
    // loads only (issued before the row): it quantizes the activation while the row streams. Every
    // other wave waits for the activation share of the unfused form, issued before the row (in
    // the fused form such a wave issued none, and the wait lets its whole row stay in flight).
    counted_wait(FUSE && stager && split ? n_early + 1 : issued);
    if (FUSE && stager) {
        // quantize the activation (QC passes of 4 * SW (superblock, row) pairs, one per 16-lane
        // group)
        __builtin_amdgcn_sched_barrier(0);
        const int tid = threadIdx.x, g = tid & 15, last_pair = nsb * MT - 1;
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            int pr = (tid >> 4) + 4 * SW * i;
            pr = pr < last_pair ? pr : last_pair;
            const int s = pr / MT, m = pr % MT;
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[4 * j] = __uint_as_float(xr[i][j].x), x[4 * j + 1] = __uint_as_float(xr[i][j].y);
                x[4 * j + 2] = __uint_as_float(xr[i][j].z), x[4 * j + 3] = __uint_as_float(xr[i][j].w);
            }
            uint32_t packed[4];
            int bsum;
            float dval;
            quantize_q8k_row16(x, g, packed, bsum, dval);
            *reinterpret_cast<uint4*>(aq + m * L.q_ld + 256 * s + 16 * g) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
            reinterpret_cast<int16_t*>(abb + m * L.b_ld)[16 * s + g] = (int16_t)bsum;
            if (g == 0) ad[64 * m + s] = dval;
        }
        if constexpr (split) {
            __builtin_amdgcn_sched_barrier(0);
            issue_pieces(cur, n_early, cur.nx4);
            issue_tail(cur);
        }
    }
    __syncthreads();

    // ---- 3. per row: the next row's loads go out (two images per wave), then steps of 16
    // superblocks, each computed once its bytes are in; then the row's sum over the wave ----
    const int c4 = lane & 3, h = c4 >> 1, lh = c4 & 1;
    const int nsteps = (nsb + kSbStep - 1) / kSbStep;
    for (int jr = 0; jr < rpw; ++jr) {
        const int64_t row = row0 + (int64_t)jr * kWaves;
        const bool row_ok = row < n1;
        int after = 0;  // loads issued after this row's (the next row's)
        RowImg nxt = cur;
        if (jr + 1 < rpw) {
            // the next image overwrites the one of row jr - 1: its LDS reads have all returned
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) alone
            __builtin_amdgcn_sched_barrier(0);
            nxt = row_image(row + kWaves, lw0 + (size_t)((jr + 1) & 1) * L.pitch);
            issue_head(nxt);
            issue_pieces(nxt, 0, nxt.nx4);
            issue_tail(nxt);
            after = nxt.issued;
        }
        const uint8_t* img = cur.img;
        float acc[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;
        for (int k = 0; k < nsteps; ++k) {
            // loads holding row bytes < 210*16*(k+1): the head and the 16-byte pieces up to that
            // byte; the last step also needs the tail
            const int endb = 3360 * (k + 1) < row_bytes ? 3360 * (k + 1) : row_bytes;
            const int need = (endb - cur.head + 1023) / 1024;
            const int done = k == nsteps - 1 ? cur.issued : 1 + (need < cur.nx4 ? need : cur.nx4);
            counted_wait(cur.issued - done + after);
            const int s_raw = kSbStep * k + (lane >> 2);
            const bool valid = s_raw < nsb;
            const int s = valid ? s_raw : nsb - 1;
            const uint8_t* sb = img + 210 * s;
            uint32_t qa[4], qb[4], qh[4], scw[2];
            lds16_a2(sb + 64 * h + 16 * lh, qa);
            lds16_a2(sb + 64 * h + 32 + 16 * lh, qb);
            lds16_a2(sb + 128 + 32 * h + 16 * lh, qh);
            lds8_a2(sb + 192 + 8 * h, scw);
            const float dW = half_bits_to_float(*reinterpret_cast<const uint16_t*>(sb + 208));
            // scales of groups 8h + 2t + lh: bytes lh + 2t of the half's eight
            const uint32_t ssh = (uint32_t)lh * 8u;
            const int sc[4] = {(int)(int8_t)(scw[0] >> ssh), (int)(int8_t)(scw[0] >> (16 + ssh)),
                               (int)(int8_t)(scw[1] >> ssh), (int)(int8_t)(scw[1] >> (16 + ssh))};
            // 6-bit values of the four quarters t for each dword i (4 elements):
            //   t = 0: ql_a low nibble | qh bits 0-1 << 4     t = 2: ql_a high nibble | qh bits 4-5
            //   t = 1: ql_b low nibble | qh bits 2-3 << 2     t = 3: ql_b high nibble | qh bits 6-7 >> 2
            uint32_t q6[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 0x0F0F0F0Fu;
                const uint32_t ev = qh[i] & 0x33333333u, od = qh[i] & 0xCCCCCCCCu;
                q6[0][i] = bfi(m, qa[i], ev << 4);
                q6[1][i] = bfi(m, qb[i], od << 2);
                q6[2][i] = bfi(m, qa[i] >> 4, ev);
                q6[3][i] = bfi(m, qb[i] >> 4, od >> 2);
            }
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                const int8_t* ap = aq + mi * L.q_ld + 256 * s + 128 * h + 16 * lh;
                // bsums of groups 8h + 2t + lh, t = 0..3: every other int16 of [16s + 8h, +8)
                const uint4 bq = *reinterpret_cast<const uint4*>(abb + mi * L.b_ld + 32 * s + 16 * h);
                const uint32_t bsh = (uint32_t)lh * 16u;
                const int bs[4] = {(int)(int16_t)(bq.x >> bsh), (int)(int16_t)(bq.y >> bsh),
                                   (int)(int16_t)(bq.z >> bsh), (int)(int16_t)(bq.w >> bsh)};
                int iS = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint4 av = *reinterpret_cast<const uint4*>(ap + 32 * t);
                    int I = sdot4((int)q6[t][0], (int)av.x, 0);
                    I = sdot4((int)q6[t][1], (int)av.y, I);
                    I = sdot4((int)q6[t][2], (int)av.z, I);
                    I = sdot4((int)q6[t][3], (int)av.w, I);
                    iS += __mul24(sc[t], I - 32 * bs[t]);  // |sc| < 128, |I - 32 bs| < 2^18
                }
                if (DUMP && valid && row_ok && mi < M)
                    atomicAdd(sums + ((int64_t)mi * sums_n_stride + (row - n0)) * nsb + s, iS);
                const float v = (dW * ad[64 * mi + s]) * (float)iS;
                acc[mi] = valid ? acc[mi] + v : acc[mi];
            }
        }
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            const float v = lanes_sum<64>(acc[mi]);
            if (lane == 0 && row_ok && mi < M)  // R (optional, may alias Y): Y = W x + R
                Y[(int64_t)mi * y_stride + (row - n0)] = R ? v + R[(int64_t)mi * r_stride + (row - n0)] : v;
        }
        cur = nxt;
    }
}

// ---------------------------------------------------------------- tall matrices on the MFMA
// Matrices of many rows (an LM head: 151936) at M <= 8: the weight rows go through the int8 MFMA
// in tiles of 32, v_mfma_i32_32x32x16_i8 per 16-element group with the activation as the A
// operand (MFMA rows m; rows >= M repeat the last real one and are never stored) and 32 weight
// rows as the B operand (columns n). Lane (n, hl) of the result holds rows m = 4 hl + v, v < 4,
// of column n: iS += sc_g * I_g is MV (= min(M tile, 4)) v_mad_i32_i24 per group for 32 rows,
// where the lane-per-superblock kernel above spends its VALU on one row at a time (and at
// K = 2560 leaves 24 of 64 lanes idle). The weight bytes are unpacked to signed q - 32 in
// registers (a v_perm table lookup for the two qh bits, v_bfi for the ql nibble).
//
// Staging: each wave streams its tiles superblock by superblock through two LDS buffers (32
// rows x 264 bytes: 8-byte aligned rows, 8-byte reads of the 32 rows conflict-free). A row's
// superblock is one direct-to-LDS instruction: lanes 0..52 the 53 dwords from the dword at or
// below it (lanes 53..63 repeat lane 52's dword into the row's padding), so an odd superblock
// (210 s = 2 mod 4) sits 2 bytes into its LDS row; the next superblock's 32 loads are in flight
// while the current one computes. The activation (planar Q8_K: qs and d; the bsums
// are not needed, the -32 is in the operand) is staged once per workgroup. A workgroup owns tiles
// blockIdx.x + k * gridDim.x; its 8 waves take work from an LDS counter, so the tiles of a CU
// spread over its waves whatever their count.
//
// Halves (PAIR): with whole tiles as the unit of work, a head of fewer tiles than waves (32768
// rows: 1024 tiles for 2048 waves) leaves waves idle. With PAIR the unit is half a tile's
// superblocks; the wave finishing a tile's first half parks its partial sums in an
// LDS slot (kTallSlots slots, tile k in slot k % kTallSlots once its earlier occupants are done),
// and the wave finishing the second half adds the two (a two-term fp32 sum: the same bits
// whichever half finishes first) and stores Y. A wave waits (s_sleep) only for a slot's earlier
// tile, whose second half another wave is computing, or for the partner's partial being written.
constexpr int kTallWaves = 8;
constexpr int kTallPitch = 264;             // LDS bytes per staged row (66 dwords)
constexpr int kTallBuf = 32 * kTallPitch;   // one superblock of a 32-row tile
constexpr int64_t kTallMinRows = 32768;     // rows from which the MFMA form is used

__host__ __device__ inline size_t tall_act_bytes(int MT, int nsb) {
    return (size_t)round_up((int64_t)MT * 256 * nsb + (int64_t)nsb * MT * 4 + 16, 256);
}
constexpr int kTallSlots = 8;  // PAIR: parked half-tile partials (64 lanes x 4 floats each)
constexpr size_t kTallPairBytes = (size_t)kTallSlots * 1024 + 3 * kTallSlots * 4;
__host__ __device__ inline size_t tall_lds_bytes(int MT, int nsb, bool pair) {
    return tall_act_bytes(MT, nsb) + (size_t)kTallWaves * 2 * kTallBuf + (pair ? kTallPairBytes : 0);
}
// Bounded spin of one lane on an LDS word (an exit every wave reaches, whatever the word holds:
// 2^22 sleeps, far beyond any wait here)
__device__ __forceinline__ void lds_spin_until(const int* p, int v) {
    for (int it = 0; it < (1 << 22); ++it) {
        if (__hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == v) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// one dword per lane from global memory (uniform base `g` + per-lane offset) into LDS at
// lds_base + 4 * lane; the base is an SGPR pair, M0 the LDS base. Used for the waves' own tile
// buffers only ("; wave-private", as dma4<true>).
__device__ __forceinline__ void dma4s(const void* g, uint32_t off, const void* lds_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1 ; wave-private" ::"v"(off), "s"(g), "s"(m0)
                 : "memory", "m0");
}

typedef int v16i_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i_t mfma_32x32x16(long a, long b) {
    v16i_t z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, z, 0, 0, 0);
}

// Signed q - 32 bytes of four 6-bit quants: ql nibbles in bits 0-3 of each byte, the two high
// bits in bits 0-1 of each byte of qh2 ((qh2 - 2) << 4 is byte qh2 of the table 0x1000F0E0).
// Plain code, not the inline-asm bfi above: the result is an MFMA operand, and the compiler places
// the wait states between a VALU write and an MFMA read of it only for instructions it can see.
__device__ __forceinline__ uint32_t q6_signed(uint32_t ql, uint32_t qh2) {
    return (ql & 0x0F0F0F0Fu) | (__builtin_amdgcn_perm(0u, 0x1000F0E0u, qh2) & 0xF0F0F0F0u);
}

// 8 bytes at p + SH (p 8-byte aligned, SH 0 or 2): one ds_read_b64, or three dwords realigned
template <int SH>
__device__ __forceinline__ uint2 lds8_sh(const uint8_t* p) {
    if constexpr (SH == 0) {
        return *reinterpret_cast<const uint2*>(p);
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
        return make_uint2(align_bytes(w1, w0, 2), align_bytes(w2, w1, 2));
    }
}

// One superblock s of a 32-row tile: the lane's column n = col (LDS row `row`, superblock byte 0
// at row + SH), activation rows min(col, MT - 1) as the A operand.
template <int MT, int SH>
__device__ __forceinline__ void tall_superblock(const uint8_t* row, const int8_t* arow, int hl, int (&ai)[4]) {
    constexpr int MV = MT < 4 ? MT : 4;
    uint32_t scw[4];
    if constexpr (SH == 0) {  // rows are 8-byte aligned: two 8-byte reads
        const uint2 v0 = *reinterpret_cast<const uint2*>(row + 192), v1 = *reinterpret_cast<const uint2*>(row + 200);
        scw[0] = v0.x, scw[1] = v0.y, scw[2] = v1.x, scw[3] = v1.y;
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(row + 192);
        const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
        scw[0] = align_bytes(w1, w0, 2), scw[1] = align_bytes(w2, w1, 2);
        scw[2] = align_bytes(w3, w2, 2), scw[3] = align_bytes(w4, w3, 2);
    }
    // Four blocks (h, gg) of four groups each, software-pipelined: the MFMAs of block i run while
    // the operands of block i + 1 are read and unpacked, then block i's results are consumed.
    // The compiler let the VALU read these MFMAs' results and overwrite their operand registers a
    // few cycles after issue (wrong sums from the later MFMAs of a block), so the order is pinned
    // with scheduling barriers, the operands and all 16 result registers of each MFMA are kept
    // allocated until consumed, and at least the unpacking of the next block (plus 8 wait
    // states; 48 after the last block) separates an MFMA from the read of its result.
    long aw[2][4], bw[2][4];
    auto prep = [&](int blk, long (&a)[4], long (&b)[4]) {
        const int h = blk >> 1, gg = blk & 1, l = 16 * gg + 8 * hl;
        const uint2 qa = lds8_sh<SH>(row + 64 * h + l);       // quarters 0 (low nibbles), 2 (high)
        const uint2 qb = lds8_sh<SH>(row + 64 * h + 32 + l);  // quarters 1, 3
        const uint2 qh = lds8_sh<SH>(row + 128 + 32 * h + l);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int g = 8 * h + 2 * t + gg;  // group of elements 128h + 32t + 16gg + [0, 16)
            const uint2 src = (t & 1) ? qb : qa;
            const uint32_t nsh = 4u * (uint32_t)(t >> 1), hsh = 2u * (uint32_t)t;
            const uint32_t b0 = q6_signed(src.x >> nsh, (qh.x >> hsh) & 0x03030303u);
            const uint32_t b1 = q6_signed(src.y >> nsh, (qh.y >> hsh) & 0x03030303u);
            b[t] = (long)(((uint64_t)b1 << 32) | b0);
            a[t] = *reinterpret_cast<const long*>(arow + 16 * g);
        }
    };
    prep(0, aw[0], bw[0]);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
        const int cur = blk & 1;
        v16i_t D[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) D[t] = mfma_32x32x16(aw[cur][t], bw[cur][t]);
        __builtin_amdgcn_sched_barrier(0);
        if (blk < 3) {
            prep(blk + 1, aw[cur ^ 1], bw[cur ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 7");
        } else {
            asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15");
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) asm volatile("" ::"v"(aw[cur][t]), "v"(bw[cur][t]));
        __builtin_amdgcn_sched_barrier(0);
        const int h = blk >> 1, gg = blk & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int g = 8 * h + 2 * t + gg;
            const int sc = __builtin_amdgcn_sbfe((int)scw[g >> 2], 8 * (g & 3), 8);
#pragma unroll
            for (int v = 0; v < MV; ++v) ai[v] = __mul24(sc, D[t][v]) + ai[v];  // |I_g| < 2^16
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) asm volatile("" ::"v"(D[t]));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// FUSE: X is fp32 [M][x_stride] and every workgroup quantizes the rows it needs to Q8_K itself (the
// shared 16-lane quantizer: the same bytes as the quantize kernel), saving that launch; else the
// planar workspace (xqs, xd).
template <int MT, bool DUMP, bool FUSE, bool PAIR>
__global__ void __launch_bounds__(64 * kTallWaves, 1) decode_q6k_mfma_kernel(
    const uint8_t* __restrict__ W, int64_t w_row_bytes, int64_t n0, int64_t n1, int nsb,
    const int8_t* __restrict__ xqs, const float* __restrict__ xd, int64_t m_ld, const float* __restrict__ X,
    int64_t x_stride, int M, float* Y, int64_t y_stride, int32_t* __restrict__ sums, int64_t sums_n_stride,
    const float* R, int64_t r_stride) {
    constexpr int MV = MT < 4 ? MT : 4;
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = nsb * 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, hl = lane >> 5;
    int8_t* aq = reinterpret_cast<int8_t*>(smem);                        // [MT][K]
    float* ad = reinterpret_cast<float*>(smem + (size_t)MT * K);         // [nsb][MT]
    int* ctr = reinterpret_cast<int*>(smem + (size_t)MT * K + (size_t)nsb * MT * 4);
    uint8_t* wb = smem + tall_act_bytes(MT, nsb) + (size_t)wave * 2 * kTallBuf;
    // PAIR: parked partials [slot][lane] (float4), then per slot: arrivals, partial ready, generation
    uint8_t* pair_base = smem + tall_act_bytes(MT, nsb) + (size_t)kTallWaves * 2 * kTallBuf;
    float4* parked = reinterpret_cast<float4*>(pair_base);
    int* slot_cnt = reinterpret_cast<int*>(pair_base + kTallSlots * 1024);
    int* slot_ready = slot_cnt + kTallSlots;
    int* slot_gen = slot_ready + kTallSlots;

    // ---- activation: MT rows of qs (rows >= M repeat row M - 1) and the superblock scales ----
    if constexpr (FUSE) {
        // (superblock, row) pairs, one per 16-lane group (32 groups a pass)
        const int g = tid & 15;
        for (int pr = tid >> 4; pr < nsb * MT; pr += 4 * kTallWaves) {
            const int sb = pr / MT, m = pr % MT;
            const float4* xp = reinterpret_cast<const float4*>(X + (int64_t)(m < M ? m : M - 1) * x_stride + 256 * sb + 16 * g);
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = xp[j];
                x[4 * j] = v.x, x[4 * j + 1] = v.y, x[4 * j + 2] = v.z, x[4 * j + 3] = v.w;
            }
            uint32_t packed[4];
            int bsum;
            float dval;
            quantize_q8k_row16(x, g, packed, bsum, dval);
            *reinterpret_cast<uint4*>(aq + (size_t)m * K + 256 * sb + 16 * g) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
            if (g == 0) ad[sb * MT + m] = dval;
        }
    } else {
        for (int i = tid; i < MT * K / 16; i += 64 * kTallWaves) {
            const int m = i / (K / 16), c = i % (K / 16);
            *reinterpret_cast<uint4*>(aq + (size_t)m * K + 16 * c) =
                *reinterpret_cast<const uint4*>(xqs + (int64_t)(m < M ? m : M - 1) * K + 16 * c);
        }
        for (int i = tid; i < nsb * MT; i += 64 * kTallWaves) ad[i] = xd[(int64_t)(i / MT) * m_ld + i % MT];
    }
    if (tid == 0) *ctr = 0;
    if (PAIR && tid < 3 * kTallSlots) slot_cnt[tid] = 0;
    __syncthreads();

    const int64_t tiles = (n1 - n0 + 31) / 32;
    const int G = gridDim.x, c0 = blockIdx.x;
    const int cnt = (int)((tiles - c0 + G - 1) / G);  // this workgroup's tiles: c0 + k * G
    auto claim = [&]() {
        int v = 0;
        if (lane == 0) v = atomicAdd(ctr, 1);
        return __builtin_amdgcn_readfirstlane(v);
    };
    // 53 dwords of row r of the tile (superblock s, from the dword at or below it) into buffer b;
    // rows past n1 (the last tile) repeat row n1 - 1
    const uint32_t dma_off = 4u * (uint32_t)(lane < 53 ? lane : 52);
    // (rows r0 .. r1 - 1 of the tile: the loop issues 31 rows, waits, then the last one, so that
    // at most 63 loads are ever outstanding, what vmcnt counts)
    auto issue = [&](int k, int s, int b, int r0, int r1) {
        const int64_t rbase = n0 + (int64_t)(c0 + (int64_t)k * G) * 32;
        const int64_t sboff = 210 * (int64_t)s - ((210 * s) & 3);
        uint8_t* dst = wb + b * kTallBuf;
        if (rbase + 32 <= n1) {
            const uint8_t* src = W + rbase * w_row_bytes + sboff;
#pragma unroll 8
            for (int r = r0; r < r1; ++r) dma4s(src + r * w_row_bytes, dma_off, dst + r * kTallPitch);
        } else {
            for (int r = r0; r < r1; ++r) {
                const int64_t row = rbase + r < n1 ? rbase + r : n1 - 1;
                dma4s(W + row * w_row_bytes + sboff, dma_off, dst + r * kTallPitch);
            }
        }
    };

    // units: whole tiles, or (PAIR) halves: unit u is tile u >> 1, superblocks from (u & 1) * per
    const int per = PAIR ? nsb / 2 : nsb;
    const int units = PAIR ? 2 * cnt : cnt;
    auto tile_of = [&](int u) { return PAIR ? u >> 1 : u; };
    auto sb0_of = [&](int u) { return PAIR ? (u & 1) * per : 0; };
    int u_cur = claim();
    if (u_cur >= units) return;  // no barrier follows: a wave without work may leave
    int u_next = claim();
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int ai[4] = {0, 0, 0, 0};
    const int8_t* arow = aq + (size_t)(col < MT ? col : MT - 1) * K + 8 * hl;
    issue(tile_of(u_cur), sb0_of(u_cur), 0, 0, 32);
    int i = 0, b = 0;  // superblock i of the unit, in buffer b
    for (;;) {
        const bool last_sb = i + 1 == per;
        const bool more = !last_sb || u_next < units;
        const int s = sb0_of(u_cur) + i;
        if (more) {
            const int nu = last_sb ? u_next : u_cur, ns = last_sb ? sb0_of(u_next) : s + 1;
            // the other buffer's previous reads have returned (lgkmcnt(0)) before it is refilled
            __builtin_amdgcn_s_waitcnt(0xC07F);
            issue(tile_of(nu), ns, b ^ 1, 0, 31);
            wait_vmcnt<31>();  // this superblock's 32 loads (issued before the next one's) are in
            issue(tile_of(nu), ns, b ^ 1, 31, 32);
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* row = wb + b * kTallBuf + col * kTallPitch;
        if ((210 * s) & 3)
            tall_superblock<MT, 2>(row, arow + 256 * s, hl, ai);
        else
            tall_superblock<MT, 0>(row, arow + 256 * s, hl, ai);
        const float dW = half_bits_to_float(*reinterpret_cast<const uint16_t*>(row + 208 + ((210 * s) & 3)));
        const int k = tile_of(u_cur);
        const int64_t n = n0 + (int64_t)(c0 + (int64_t)k * G) * 32 + col;
#pragma unroll
        for (int v = 0; v < MV; ++v) {
            const int m = 4 * hl + v;
            acc[v] = fmaf(dW * ad[s * MT + (m < MT ? m : MT - 1)], (float)ai[v], acc[v]);
            if (DUMP && m < M && n < n1) sums[((int64_t)m * sums_n_stride + (n - n0)) * nsb + s] = ai[v];
            ai[v] = 0;
        }
        if (last_sb) {
            bool store = true;
            if constexpr (PAIR) {
                const int j = k % kTallSlots, gen = k / kTallSlots;
                // the slot's earlier tiles are done
                if (lane == 0) lds_spin_until(slot_gen + j, gen);
                int first = 0;
                if (lane == 0) first = atomicAdd(slot_cnt + j, 1) == 0;
                first = __builtin_amdgcn_readfirstlane(first);
                if (first) {
                    parked[j * 64 + lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // the partial is in LDS
                    if (lane == 0) __hip_atomic_store(slot_ready + j, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                    store = false;
                } else {
                    if (lane == 0) lds_spin_until(slot_ready + j, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("" ::: "memory");
                    const float4 o = parked[j * 64 + lane];
                    acc[0] += o.x, acc[1] += o.y, acc[2] += o.z, acc[3] += o.w;
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // the partial has been read
                    if (lane == 0) {
                        slot_cnt[j] = 0;
                        slot_ready[j] = 0;
                        __hip_atomic_store(slot_gen + j, gen + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                    }
                }
            }
            if (store && n < n1) {
#pragma unroll
                for (int v = 0; v < MV; ++v) {
                    const int m = 4 * hl + v;
                    if (m < M)  // R (optional, may alias Y): Y = W x + R
                        Y[(int64_t)m * y_stride + (n - n0)] =
                            R ? acc[v] + R[(int64_t)m * r_stride + (n - n0)] : acc[v];
                }
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[v] = 0.0f;
            if (!more) break;
            u_cur = u_next;
            u_next = claim();
            i = 0;
        } else {
            ++i;
        }
        b ^= 1;
    }
}

namespace {

using Q6Fn = void (*)(const float*, int64_t, const uint8_t*, int64_t, int64_t, int, int, int, int, const int8_t*,
                      const float*, const int16_t*, int64_t, float*, int64_t, int32_t*, int64_t, const float*,
                      int64_t);

// fused activation: M <= 2 rows, nsb <= 64. Every wave stages: at most 8 passes of 16 (superblock,
// row) pairs in 4-wave workgroups, at most 4 passes of 4 * NW pairs in 8..12-wave ones (64
// registers of activation per lane)
constexpr int q6_stage_waves(int nw) { return nw; }
template <int MT, bool DUMP, int NW, int QC>
Q6Fn q6_fused_qc(int qc) {
    constexpr int SW = q6_stage_waves(NW);
    if constexpr (QC > (NW > 4 ? 4 : 8)) {
        return nullptr;
    } else {
        if (qc == QC) return decode_q6k_lds_kernel<MT, DUMP, true, QC, NW, SW>;
        return q6_fused_qc<MT, DUMP, NW, QC + 1>(qc);
    }
}
template <bool DUMP, int NW>
Q6Fn q6_fused_nw(int mt, int qc) {
    return mt == 1 ? q6_fused_qc<1, DUMP, NW, 1>(qc) : mt == 2 ? q6_fused_qc<2, DUMP, NW, 1>(qc) : nullptr;
}
template <bool DUMP>
Q6Fn q6_pick_fused(int mt, int qc, int nw) {
    switch (nw) {
        case 4: return q6_fused_nw<DUMP, 4>(mt, qc);
        case 8: return q6_fused_nw<DUMP, 8>(mt, qc);
        case 10: return q6_fused_nw<DUMP, 10>(mt, qc);
        case 12: return q6_fused_nw<DUMP, 12>(mt, qc);
        default: return nullptr;
    }
}

// Rows per wave of the 4-wave kernels. One row per wave while the grid is a few workgroups per
// CU; for very tall matrices (LM heads: 151936 rows) every workgroup would otherwise restage
// (and, fused, re-quantize) the whole activation for four rows, so each wave streams several
// rows through two LDS images, keeping about 16 workgroups per CU over the launch.
int q6_rows_per_wave(int64_t rows, int nw) {
    int rpw = knob(Knob::Q6KRows);
    if (rpw < 1) {
        const int64_t per_wave = rows / ((int64_t)nw * cu_count() * 16);
        rpw = per_wave >= 8 ? 8 : per_wave >= 4 ? 4 : per_wave >= 2 ? 2 : 1;
    }
    return rpw > 16 ? 16 : rpw;
}

using TallFn = void (*)(const uint8_t*, int64_t, int64_t, int64_t, int, const int8_t*, const float*, int64_t,
                        const float*, int64_t, int, float*, int64_t, int32_t*, int64_t, const float*, int64_t);

template <bool DUMP, bool FUSE, bool PAIR>
TallFn tall_pick(int mt) {
    switch (mt) {
        case 1: return decode_q6k_mfma_kernel<1, DUMP, FUSE, PAIR>;
        case 2: return decode_q6k_mfma_kernel<2, DUMP, FUSE, PAIR>;
        case 4: return decode_q6k_mfma_kernel<4, DUMP, FUSE, PAIR>;
        default: return decode_q6k_mfma_kernel<8, DUMP, FUSE, PAIR>;
    }
}
template <bool DUMP, bool FUSE>
TallFn tall_pick(int mt, bool pair) {
    return pair ? tall_pick<DUMP, FUSE, true>(mt) : tall_pick<DUMP, FUSE, false>(mt);
}

// Tall matrices: the MFMA kernel over rows [n0, n1), M tiled by 8; X (fp32, quantized in every
// workgroup) or the planar activation `act`.
hipError_t launch_tall_q6k(const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K, const float* X,
                           int64_t x_stride, const PlanarBuffers* act, int64_t M, float* Y, int64_t y_stride,
                           int32_t* block_sums, int64_t sums_n_stride, hipStream_t st, const float* R, int64_t r_stride) {
    const int nsb = (int)(K / 256);
    const int64_t tiles = (n1 - n0 + 31) / 32;
    const unsigned grid = (unsigned)(tiles < cu_count() ? tiles : cu_count());
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const bool fuse = X != nullptr;
        // halves where whole tiles would leave waves idle and the slots fit in LDS (151936 x 2560:
        // 2.3 tiles per wave, halves 63.6 -> 64.8 us; 32768 x 4096: 0.5, halves 32.1 -> 27.5 us)
        const bool pair = tiles < (int64_t)grid * kTallWaves && tall_lds_bytes(mt, nsb, true) <= kMaxLds;
        TallFn fn = block_sums ? (fuse ? tall_pick<true, true>(mt, pair) : tall_pick<true, false>(mt, pair))
                               : (fuse ? tall_pick<false, true>(mt, pair) : tall_pick<false, false>(mt, pair));
        hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * kTallWaves), tall_lds_bytes(mt, nsb, pair), st, (const uint8_t*)W,
                           w_row_bytes, n0, n1, nsb, fuse ? nullptr : act->qs + m0 * K, fuse ? nullptr : act->d + m0,
                           fuse ? (int64_t)0 : act->m_ld, fuse ? X + m0 * x_stride : nullptr, x_stride, (int)mc,
                           Y + m0 * y_stride, y_stride, block_sums ? block_sums + m0 * sums_n_stride * nsb : nullptr,
                           sums_n_stride, R ? R + m0 * r_stride : nullptr, r_stride);
    }
    return hipGetLastError();
}

// The MFMA form for tall matrices (DCQ_Q6K_MFMA=0 keeps the lane-per-superblock kernels): an even
// number of superblocks (the 53-dword staging of an even superblock reads 2 bytes into the next)
// and the activation tile within the LDS left by the weight buffers.
bool q6_use_mfma(int64_t rows, int nsb, int64_t M) {
    if (rows < kTallMinRows || nsb % 2 != 0 || knob(Knob::Q6KMfma) == 0) return false;
    // one activation row up to 16 superblocks: the fused LDS kernel (four rows per wave) stays
    // faster below 65536 rows (49152 x 4096: 36.8 against 40.8 us per step; 32768 x 4096 26.0
    // against 26.7 us), the MFMA kernel from there (65536 x 2048: 27.6 against 30.6 us)
    if (M == 1 && nsb <= kSbStep && rows < 65536) return false;
    const int mt = M == 1 ? 1 : M == 2 ? 2 : M <= 4 ? 4 : 8;
    return tall_lds_bytes(mt, nsb, false) <= kMaxLds;
}

template <bool DUMP>
Q6Fn q6_pick(int mt) {
    switch (mt) {
        case 1: return decode_q6k_lds_kernel<1, DUMP>;
        case 2: return decode_q6k_lds_kernel<2, DUMP>;
        case 4: return decode_q6k_lds_kernel<4, DUMP>;
        default: return decode_q6k_lds_kernel<8, DUMP>;
    }
}

}  // namespace

hipError_t launch_decode_q6k_lds(const void* W, int64_t w_row_bytes, int64_t n0, int64_t n1, int64_t K,
                                 const PlanarBuffers& act, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                                 int64_t sums_n_stride, hipStream_t st, const float* R, int64_t r_stride) {
    const int nsb = (int)(K / 256);
    // dword-granular head/tail loads: the row's bytes and its stride must be whole dwords;
    // the weight base is 16-byte aligned (checked by the C ABI)
    if (nsb % 2 != 0 || w_row_bytes % 4 != 0 || nsb > kMaxNsb || w_row_bytes > INT32_MAX)
        return hipErrorNotSupported;
    if (knob(Knob::Q6KLdsOff)) return hipErrorNotSupported;
    if (q6_use_mfma(n1 - n0, nsb, M))
        return launch_tall_q6k(W, w_row_bytes, n0, n1, K, nullptr, 0, &act, M, Y, y_stride, block_sums, sums_n_stride,
                               st, R, r_stride);
    const int nw = 4;  // 5-wave workgroups (rows spread more evenly) measured no faster here
    // several rows per wave only where a step of 16 superblocks covers the row (the waits count
    // two rows' loads)
    const int rpw = nsb <= kSbStep ? q6_rows_per_wave(n1 - n0, nw) : 1;
    const int nbuf = rpw > 1 ? 2 : 1;
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        if (Q6Lds(nsb, mt, nw, nbuf).total > kMaxLds) return hipErrorNotSupported;
    }
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mc = M - m0 < 8 ? M - m0 : 8;
        const int mt = mc == 1 ? 1 : mc == 2 ? 2 : mc <= 4 ? 4 : 8;
        const unsigned grid = (unsigned)((n1 - n0 + (int64_t)nw * rpw - 1) / ((int64_t)nw * rpw));
        Q6Fn fn = block_sums ? q6_pick<true>(mt) : q6_pick<false>(mt);
        hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * nw), Q6Lds(nsb, mt, nw, nbuf).total, st, (const float*)nullptr,
                           (int64_t)0, (const uint8_t*)W, n0, n1, (int)w_row_bytes, (int)mc, nsb, rpw,
                           act.qs + m0 * K, act.d + m0, act.bs + m0 * (K / 16), act.m_ld, Y + m0 * y_stride,
                           y_stride, block_sums ? block_sums + m0 * sums_n_stride * nsb : nullptr, sums_n_stride,
                           R ? R + m0 * r_stride : nullptr, r_stride);
    }
    return hipGetLastError();
}

hipError_t launch_decode_fused_q6k(const void* W, int64_t w_row_bytes, int64_t N, int64_t K, const float* X,
                                   int64_t x_stride, int64_t M, float* Y, int64_t y_stride, int32_t* block_sums,
                                   hipStream_t st, const float* R, int64_t r_stride) {
    const int nsb = (int)(K / 256);
    if (nsb % 2 != 0 || w_row_bytes % 4 != 0 || nsb > kMaxNsb || w_row_bytes > INT32_MAX)
        return hipErrorNotSupported;
    if (knob(Knob::Q6KLdsOff) != 0 || knob(Knob::Q6KNoFuse) != 0) return hipErrorNotSupported;
    // tall matrices (M <= 8): the MFMA kernel, every workgroup quantizing the activation
    if (M <= 8 && q6_use_mfma(N, nsb, M))
        return launch_tall_q6k(W, w_row_bytes, 0, N, K, X, x_stride, nullptr, M, Y, y_stride, block_sums, N, st, R,
                               r_stride);
    if (M > 2) return hipErrorNotSupported;
    // Workgroup width (one row per wave). Up to K = 4096, 4 waves (measured at M = 1 against
    // quantize + decode: 2560 x 4096 5.7 vs 7.2 us; 1024 x 2560 3.8 vs 5.8 us). Beyond, every
    // workgroup re-reads and re-quantizes the whole activation (39 KB at K = 9728: 4-wave
    // workgroups 12.3 us against 10.5 us unfused), so a workgroup takes all rows of its CU
    // instead, 8 to 12 waves, one workgroup per CU (2560 x 9728: 10 waves 9.3 us, 12 waves
    // 9.5 us). Outside 8..12 rows per CU the separate quantize kernel stays.
    int nw = 4;
    if (nsb > 16) {
        const int cus = cu_count();
        const int64_t per_cu = (N + cus - 1) / cus;
        if (per_cu < 8 || per_cu > 12) return hipErrorNotSupported;
        nw = per_cu <= 8 ? 8 : per_cu <= 10 ? 10 : 12;
    }
    if (knob(Knob::Q6KFuseWaves) > 0) nw = knob(Knob::Q6KFuseWaves);  // tuning override: 4, 8, 10 or 12
    const int kWaves = nw;
    const int mt = M == 1 ? 1 : 2;
    const int sw = q6_stage_waves(kWaves);
    const int qc = (nsb * mt + 4 * sw - 1) / (4 * sw);
    // Rows per wave of the fused 4-wave kernel: every workgroup quantizes the activation again, so
    // from 6144 rows fewer, longer workgroups win, four rows per wave from 128 k superblocks (per
    // step, 1 / 2 / 4 rows per wave: 8192 x 2048 6.98 / 6.50 / 7.24 us; 8192 x 4096 9.0 / 9.6 /
    // 8.6 us; 24576 x 2048 16.9 / 14.9 / 14.2 us; 32000 x 2048 21.3 / 18.0 / 16.7 us; M = 2,
    // 8192 x 4096 13.9 / 12.5 / 10.9 us; below 6144 rows one row per wave: 2048 x 2048 3.8 / 4.2 /
    // 6.1 us)
    int rpw = 1;
    if (kWaves == 4 && nsb <= kSbStep) {
        rpw = (int64_t)N * nsb >= 131072 ? 4 : N >= 6144 ? 2 : 1;
        if (knob(Knob::Q6KRows) >= 1) rpw = q6_rows_per_wave(N, kWaves);
    }
    const Q6Lds lds(nsb, mt, kWaves, rpw > 1 ? 2 : 1);
    if (lds.total > kMaxLds) return hipErrorNotSupported;
    Q6Fn fn = block_sums ? q6_pick_fused<true>(mt, qc, kWaves) : q6_pick_fused<false>(mt, qc, kWaves);
    if (!fn) return hipErrorNotSupported;
    const unsigned grid = (unsigned)((N + (int64_t)kWaves * rpw - 1) / ((int64_t)kWaves * rpw));
    hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * kWaves), lds.total, st, X, x_stride, (const uint8_t*)W, (int64_t)0,
                       N, (int)w_row_bytes, (int)M, nsb, rpw, (const int8_t*)nullptr, (const float*)nullptr,
                       (const int16_t*)nullptr, (int64_t)0, Y, y_stride, block_sums, N, R, r_stride);
    return hipGetLastError();
}

}  // namespace dcq
