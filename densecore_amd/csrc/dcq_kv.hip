// dcq_kv.hip — DenseCore's paged KV cache on the device, and the attention that reads it.
//
// Arena layout (the reference's PagedKVCache bytes, core/src/kv_cache.cpp:341-409): slot
// (block, layer, s) at ((block * n_layer + layer) * 16 + s) * slot_bytes, slot_bytes =
// row_size(cache_type, n_head_kv * head_dim); a slot holds one token's row for all KV heads,
// head h at h * head_dim elements into the row.
//
// Kernels:
//   kv_write_kernel   WriteKSlot/WriteVSlot (core/src/kv_cache.cpp:565-598): F32 copy, F16
//                     round-to-nearest-even, Q8_0 quantize_row_q8_0_ref (d = amax/127,
//                     id = 1/d, roundf). Bit-exact; compiled without fp contraction.
//   kv_gather_kernel  cb_kv_update_and_gather's output (core/src/inference.cpp:748-784):
//                     history read from the arena, batch rows appended in fp32.
//   attn_kernel       the standard attention path (core/src/inference.cpp:1577-1746) fused
//                     over the arena: scores, scale, causal mask, softmax and the V product in
//                     one pass with an online softmax, reading Q8_0/F16/F32 slots directly
//                     (the reference first gathers the whole history into fp32).
//   attn_combine_kernel  merges key-range splits (decode spreads the keys over workgroups).
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

constexpr int kKvBlock = 16;

__device__ __forceinline__ const uint8_t* kv_slot(const uint8_t* arena, int blk, int n_layer, int layer, int slot,
                                                  int64_t sb) {
    return arena + (((int64_t)blk * n_layer + layer) * kKvBlock + slot) * sb;
}

// ---------------------------------------------------------------- write
// One workgroup per token row. Units: a 32-element block (Q8_0), 2 elements (F16), 4 (F32).
__global__ void __launch_bounds__(256) kv_write_kernel(int ct, uint8_t* __restrict__ arena, int n_blocks,
                                                       int n_layer, int layer, int64_t row_elems, int64_t sb,
                                                       const int32_t* __restrict__ table, int pos0,
                                                       const float* __restrict__ src, int64_t src_stride) {
#pragma clang fp contract(off)
    const int i = blockIdx.x;
    const int pos = pos0 + i;
    const int blk = table[pos / kKvBlock];
    if (blk < 0 || blk >= n_blocks) return;  // the reference skips a null slot pointer
    uint8_t* dst = const_cast<uint8_t*>(kv_slot(arena, blk, n_layer, layer, pos % kKvBlock, sb));
    const float* x = src + (int64_t)i * src_stride;
    if (ct == kTypeQ8_0) {
        for (int64_t b = threadIdx.x; b < row_elems / 32; b += blockDim.x) {
            const float4* xb = reinterpret_cast<const float4*>(x + b * 32);
            float v[32];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float4 f = xb[j];
                v[4 * j] = f.x, v[4 * j + 1] = f.y, v[4 * j + 2] = f.z, v[4 * j + 3] = f.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
            const float d = amax / 127.f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint16_t* p16 = reinterpret_cast<uint16_t*>(dst + b * 34);
            p16[0] = float_to_half_bits(d);
#pragma unroll
            for (int j = 0; j < 32; j += 2) {
                const float q0 = fminf(fmaxf(roundf(v[j] * id), -128.f), 127.f);
                const float q1 = fminf(fmaxf(roundf(v[j + 1] * id), -128.f), 127.f);
                p16[1 + j / 2] =
                    (uint16_t)(((uint32_t)(int32_t)q0 & 0xFFu) | (((uint32_t)(int32_t)q1 & 0xFFu) << 8));
            }
        }
    } else if (ct == kTypeF16) {
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
        for (int64_t u = threadIdx.x; u < row_elems / 2; u += blockDim.x) {
            const float2 f = reinterpret_cast<const float2*>(x)[u];
            d32[u] = (uint32_t)float_to_half_bits(f.x) | ((uint32_t)float_to_half_bits(f.y) << 16);
        }
    } else {
        float4* d4 = reinterpret_cast<float4*>(dst);
        for (int64_t u = threadIdx.x; u < row_elems / 4; u += blockDim.x) d4[u] = reinterpret_cast<const float4*>(x)[u];
    }
}

// ---------------------------------------------------------------- gather
// One workgroup per output row t of [n_past + N, row_elems].
__global__ void __launch_bounds__(256) kv_gather_kernel(int ct, const uint8_t* __restrict__ arena, int n_blocks,
                                                        int n_layer, int layer, int64_t row_elems, int64_t sb,
                                                        const int32_t* __restrict__ table, int n_table, int n_past,
                                                        const float* __restrict__ cur, int64_t cur_stride,
                                                        float* __restrict__ dst, int64_t dst_stride) {
    const int t = blockIdx.x;
    float4* out = reinterpret_cast<float4*>(dst + (int64_t)t * dst_stride);
    const int64_t n4 = row_elems / 4;
    if (t >= n_past) {
        const float4* x = reinterpret_cast<const float4*>(cur + (int64_t)(t - n_past) * cur_stride);
        for (int64_t u = threadIdx.x; u < n4; u += blockDim.x) out[u] = x[u];
        return;
    }
    const int lb = t / kKvBlock;
    const int blk = lb < n_table ? table[lb] : -1;
    if (blk < 0 || blk >= n_blocks) {  // no block: zeros, as the reference's missing-block path
        for (int64_t u = threadIdx.x; u < n4; u += blockDim.x) out[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const uint8_t* s = kv_slot(arena, blk, n_layer, layer, t % kKvBlock, sb);
    for (int64_t u = threadIdx.x; u < n4; u += blockDim.x) {
        float4 f;
        if (ct == kTypeQ8_0) {
            const uint8_t* b = s + (u / 8) * 34;
            const float d = half_bits_to_float(ldu16(b));
            const int o = 2 + 4 * (int)(u % 8);
            const uint32_t lo = ldu16(b + o), hi = ldu16(b + o + 2);
            f.x = d * (float)(int8_t)(lo & 0xFF);
            f.y = d * (float)(int8_t)(lo >> 8);
            f.z = d * (float)(int8_t)(hi & 0xFF);
            f.w = d * (float)(int8_t)(hi >> 8);
        } else if (ct == kTypeF16) {
            const uint2 h = reinterpret_cast<const uint2*>(s)[u];
            f.x = half_bits_to_float(h.x & 0xFFFF);
            f.y = half_bits_to_float(h.x >> 16);
            f.z = half_bits_to_float(h.y & 0xFFFF);
            f.w = half_bits_to_float(h.y >> 16);
        } else {
            f = reinterpret_cast<const float4*>(s)[u];
        }
        out[u] = f;
    }
}

// ---------------------------------------------------------------- attention
// Workgroup: 4 waves, one KV head's group of query heads (HPW of them) for NQ query tokens
// (R = NQ * HPW <= RMAX rows), over a range of key chunks. A chunk is KC = 8192 / HD keys.
//   scores: wave w takes keys [w*KPW, (w+1)*KPW) of the chunk; LPK = HD/32 lanes per key,
//           each lane one 32-element block of the key row, summed across the LPK lanes;
//   softmax: wave w owns rows w, w+4, ...: chunk max, running max M, rescale alpha, p = 2^(s-M);
//   V:       wave w again takes its KPW keys; lanes over dims (DPL = HD/64 each), R rows.
// Scores are kept in base 2: s = (q . k) * scale * log2(e), p = exp2(s - M).
template <int HD>
struct AttnShape {
    static constexpr int LPK = HD / 32;
    static constexpr int KPW = 64 / LPK;
    static constexpr int KC = 4 * KPW;
    static constexpr int DPL = HD / 64;
};
// Row capacity of a workgroup: 4 for decode-sized calls (one token's query heads of one KV
// head, n_rep <= 4: rows unrolled, a quarter of the LDS), else 16 (8 at head_dim 256).
template <int HD>
constexpr int attn_rmax_large() { return HD >= 256 ? 8 : 16; }

struct AttnArgs {
    const uint8_t* k_arena;
    const uint8_t* v_arena;
    int n_blocks, n_layer, layer;
    int64_t sb;  // slot bytes
    const int32_t* table;
    int n_table;
    const float* q;
    int64_t q_stride;  // floats between query tokens
    const float* k_cur;
    const float* v_cur;
    int64_t kv_stride;  // floats between current K (V) rows
    float* out;
    int64_t out_stride;
    float* ws_o;  // [splits][N][n_head][HD]
    float* ws_ml;  // [splits][N][n_head][2]
    int n_tokens, n_past, n_head, n_head_kv, hpw, nq;
    int nch_hist, nch_total, cps;  // chunks of history, all chunks, chunks per split
    int splits, groups;
    float scale_log2e;
};

// DPL consecutive dims of a value row, starting at element e0 of the head.
template <int CT, int DPL>
__device__ __forceinline__ void load_value_dims(const uint8_t* head, int e0, float (&v)[DPL]) {
    if constexpr (CT == kTypeQ8_0) {
        const uint8_t* b = head + (e0 / 32) * 34;
        const float d = half_bits_to_float(ldu16(b));
        const uint8_t* qs = b + 2 + (e0 % 32);
        if constexpr (DPL == 1) {
            v[0] = d * (float)(int8_t)qs[0];
        } else {
#pragma unroll
            for (int k = 0; k < DPL; k += 2) {
                const uint32_t h = ldu16(qs + k);
                v[k] = d * (float)(int8_t)(h & 0xFF);
                v[k + 1] = d * (float)(int8_t)(h >> 8);
            }
        }
    } else if constexpr (CT == kTypeF16) {
        // 2*DPL bytes at a multiple of 2*DPL (head pieces are 8-byte aligned): one load
        const uint8_t* h = head + 2 * e0;
        if constexpr (DPL == 1) {
            v[0] = half_bits_to_float(ldu16(h));
        } else if constexpr (DPL == 2) {
            const uint32_t w = ld1(h);
            v[0] = half_bits_to_float(w & 0xFFFF), v[1] = half_bits_to_float(w >> 16);
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(h);
            v[0] = half_bits_to_float(w.x & 0xFFFF), v[1] = half_bits_to_float(w.x >> 16);
            v[2] = half_bits_to_float(w.y & 0xFFFF), v[3] = half_bits_to_float(w.y >> 16);
        }
    } else {
        // 4*DPL bytes at a multiple of 4*DPL (fp32 rows are 16-byte aligned): one load
        const float* f = reinterpret_cast<const float*>(head) + e0;
        if constexpr (DPL == 1) {
            v[0] = f[0];
        } else if constexpr (DPL == 2) {
            const float2 w = *reinterpret_cast<const float2*>(f);
            v[0] = w.x, v[1] = w.y;
        } else {
            const float4 w = *reinterpret_cast<const float4*>(f);
            v[0] = w.x, v[1] = w.y, v[2] = w.z, v[3] = w.w;
        }
    }
}

// F16 / F32: the words holding DPL consecutive dims of a value row from element e0 (as
// load_value_dims), unconverted; value_from_raw converts them (zeros where `ok` is false).
template <int CT, int DPL>
__device__ __forceinline__ void load_value_raw(const uint8_t* head, int e0, uint32_t (&w)[CT == kTypeF16 ? (DPL + 1) / 2 : DPL]) {
    static_assert(CT == kTypeF16 || CT == kTypeF32, "Q8_0 values are staged through LDS");
    if constexpr (CT == kTypeF16) {
        const uint8_t* h = head + 2 * e0;
        if constexpr (DPL == 1) {
            w[0] = ldu16(h);
        } else if constexpr (DPL == 2) {
            w[0] = ld1(h);
        } else {
            const uint2 u = *reinterpret_cast<const uint2*>(h);
            w[0] = u.x, w[1] = u.y;
        }
    } else {
        const uint8_t* f = head + 4 * e0;
        if constexpr (DPL == 1) {
            w[0] = ld1(f);
        } else if constexpr (DPL == 2) {
            const uint2 u = *reinterpret_cast<const uint2*>(f);
            w[0] = u.x, w[1] = u.y;
        } else {
            const uint4 u = *reinterpret_cast<const uint4*>(f);
            w[0] = u.x, w[1] = u.y, w[2] = u.z, w[3] = u.w;
        }
    }
}
template <int CT, int DPL>
__device__ __forceinline__ void value_from_raw(const uint32_t (&w)[CT == kTypeF16 ? (DPL + 1) / 2 : DPL], bool ok,
                                               float (&v)[DPL]) {
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
        float x;
        if constexpr (CT == kTypeF16)
            x = half_bits_to_float((w[k / 2] >> (16 * (k & 1))) & 0xFFFFu);
        else
            x = __uint_as_float(w[k]);
        v[k] = ok ? x : 0.0f;
    }
}

template <int CT>
__device__ __forceinline__ int64_t head_bytes(int hd) {
    return CT == kTypeQ8_0 ? (int64_t)(hd / 32) * 34 : (int64_t)hd * (CT == kTypeF16 ? 2 : 4);
}

__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// LDS of one attention workgroup.
template <int HD, int RM>
struct AttnSmem {
    using S = AttnShape<HD>;
    static constexpr int HBW = (HD / 32) * 34 / 4;  // dwords per Q8_0 head piece
    static constexpr int NST = (S::KPW * HBW + 63) / 64;
    alignas(16) float q[RM][HD];  // 16-byte aligned: the score loop reads it as float4
    float p[RM][S::KC];
    float m[RM], l[RM], alpha[RM];
    float o[4][RM][HD];  // running V sums of each wave's keys
    // Q8_0 history: each wave stages its KPW keys' V head pieces (2176 bytes per wave for every
    // head_dim) with dword loads, then reads its dims from LDS
    uint32_t v[4][NST * 64];
};

// Per-workgroup constants of the attention kernel.
struct AttnTile {
    int tid, wave, lane, h_kv, i0, R;
    int64_t hb;  // bytes of one KV head's piece in a slot
};

// One chunk of KC keys: kbase .. kbase + KC - 1 (below klim), from the arena in format SRC
// (history) or from the current fp32 rows (SRC = F32, from_cur). Updates the running softmax
// state (m, l) and each wave's V sums. On the first chunk the query rows go to LDS after the
// chunk's loads are issued, so their latency overlaps.
template <int SRC, bool FROM_CUR, int HD, int RM, int QPT>
__device__ __forceinline__ void attn_chunk(const AttnArgs& a, const AttnTile& w, AttnSmem<HD, RM>& sm, int kbase,
                                           int klim, bool& q_stored, const float (&qreg)[QPT], int blk_pre = -2) {
    using S = AttnShape<HD>;
    constexpr int LPK = S::LPK, KPW = S::KPW, KC = S::KC, DPL = S::DPL;
    constexpr int HBW = AttnSmem<HD, RM>::HBW, NST = AttnSmem<HD, RM>::NST;
    constexpr bool STAGED = SRC == kTypeQ8_0 && !FROM_CUR;
    // F16 / F32 history: K and V loaded as raw words by every lane of a wave with a present key,
    // converted at use (see the loads below)
    constexpr bool RAWV = !STAGED && !FROM_CUR;
    const int wave = w.wave, lane = w.lane;

    // ---- this lane's key (score mapping) and where its head piece lives: a byte offset into
    // the arenas (K and V share the layout) or into the current rows
    const int t = wave * KPW + lane / LPK, b = lane % LPK;
    const int kt = kbase + t;
    int64_t off = 0;
    bool have = kt < klim;
    if (!FROM_CUR) {
        const int lb = kt / kKvBlock;
        // blk_pre >= -1: this lane's table entry, already loaded by the caller (the first chunk)
        const int blk = blk_pre >= -1 ? blk_pre : have && lb < a.n_table ? a.table[lb] : -1;
        have = blk >= 0 && blk < a.n_blocks;
        off = (((int64_t)blk * a.n_layer + a.layer) * kKvBlock + kt % kKvBlock) * a.sb + w.h_kv * w.hb;
    } else {
        off = ((int64_t)(kt - a.n_past) * a.kv_stride + (int64_t)w.h_kv * HD) * 4;
    }
    if (!have) off = 0;
    // key tt of this wave is present iff bit tt*LPK; a missing key's values are zero
    const uint64_t present = __ballot(have);

    // ---- issue every load of the chunk: the lane's K block (a Q8_0 block stays packed and is
    // unpacked per row below), then the V of the wave's KPW keys
    const uint8_t* kbase_p = FROM_CUR ? reinterpret_cast<const uint8_t*>(a.k_cur) : a.k_arena;
    const uint8_t* vbase_p = FROM_CUR ? reinterpret_cast<const uint8_t*>(a.v_cur) : a.v_arena;
    // raw words only: a conversion here would wait for the K loads before the V loads issue
    constexpr int KRAW = STAGED ? 2 : (SRC == kTypeF16 ? 4 : 8);  // 16-byte words of the block
    uint4 kraw[KRAW];
    float sc = 0.0f;
    if constexpr (STAGED) {
        if (have) {
            const uint8_t* p = kbase_p + off + b * 34;
            sc = half_bits_to_float(ldu16(p));
            uint32_t w[8];
            ld16_a2(p + 2, w);
            ld16_a2(p + 18, w + 4);
            kraw[0] = make_uint4(w[0], w[1], w[2], w[3]);
            kraw[1] = make_uint4(w[4], w[5], w[6], w[7]);
        } else {
            kraw[0] = kraw[1] = make_uint4(0u, 0u, 0u, 0u);
        }
    } else if (RAWV ? present != 0 : have) {
        // the key's piece as 16-byte words, interleaved over its LPK lanes (word b + LPK*j to
        // lane b): each load instruction reads contiguous bytes across the lanes of a key. History:
        // every lane of a wave with a present key loads (a missing key's offset is 0, in bounds),
        // and its values are zeroed when converted, so that no branch splits the loads (the waits
        // below then count exactly).
        sc = 1.0f;
        const uint8_t* p = kbase_p + off + 16 * b;
#pragma unroll
        for (int j = 0; j < KRAW; ++j) kraw[j] = ld16(p + 16 * LPK * j);
    } else {
#pragma unroll
        for (int j = 0; j < KRAW; ++j) kraw[j] = make_uint4(0u, 0u, 0u, 0u);
    }
    // F16 / F32: the K loads stay ahead of the V loads (the scheduler otherwise issues the V loads
    // first, and the scores would wait for both); they are waited for first (loads retire in order)
    if constexpr (RAWV) __builtin_amdgcn_sched_barrier(0);
    float v[KPW][DPL];
    // F16 / F32: the raw words of each key's DPL dims, converted after the softmax (a conversion
    // here would make each key's load wait for the one before)
    constexpr int VRW = SRC == kTypeF16 ? (DPL + 1) / 2 : DPL;
    uint32_t vraw[RAWV ? KPW : 1][VRW];
    const int e0 = DPL * lane;
    uint32_t vst[STAGED ? NST : 1];
    if constexpr (STAGED) {
        // A wave's KPW keys start on a multiple of min(KPW, kKvBlock) (kbase is a multiple of
        // KC = 4 KPW), so key pk lies in the wave's KV block pk / kKvBlock at position
        // pk % kKvBlock past that block's first key of the wave: its slot offset is that key's
        // (one scalar read per block) plus (pk % kKvBlock) slots, no lane exchange per load.
        constexpr int NB = KPW > kKvBlock ? KPW / kKvBlock : 1;
        static_assert(KPW % kKvBlock == 0 || kKvBlock % KPW == 0, "keys of a wave tile KV blocks");
        int64_t ob[NB];
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
            const int src = bb * kKvBlock * LPK;  // the lane of key bb * kKvBlock (compile-time)
            ob[bb] = ((int64_t)__builtin_amdgcn_readlane((int)(off >> 32), src) << 32) |
                     (uint32_t)__builtin_amdgcn_readlane((int)off, src);
        }
#pragma unroll
        for (int j = 0; j < NST; ++j) {
            const int f = lane + 64 * j, pk = f / HBW, dw = f - pk * HBW;
            const int pkc = pk < KPW ? pk : 0, bb = NB > 1 ? pkc / kKvBlock : 0;
            int64_t o0 = ob[0];
#pragma unroll
            for (int k = 1; k < NB; ++k) o0 = bb == k ? ob[k] : o0;
            const int64_t op = o0 + (int64_t)(pkc % kKvBlock) * a.sb;
            const bool ok = f < KPW * HBW && ((present >> (pkc * LPK)) & 1);
            vst[j] = ok ? ld1(vbase_p + op + 4 * dw) : 0u;
        }
    } else if constexpr (RAWV) {
        if (present != 0) {
#pragma unroll
            for (int tt = 0; tt < KPW; ++tt) {
                // every lane loads: a missing key's offset is 0, in bounds (masked when converted)
                const int64_t o_tt = ((int64_t)__builtin_amdgcn_readlane((int)(off >> 32), tt * LPK) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane((int)off, tt * LPK);
                load_value_raw<SRC, DPL>(vbase_p + o_tt, e0, vraw[tt]);
            }
        } else {
#pragma unroll
            for (int tt = 0; tt < KPW; ++tt)
#pragma unroll
                for (int k = 0; k < VRW; ++k) vraw[tt][k] = 0u;
        }
    } else {
#pragma unroll
        for (int tt = 0; tt < KPW; ++tt) {
            const int64_t o_tt = ((int64_t)__builtin_amdgcn_readlane((int)(off >> 32), tt * LPK) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)off, tt * LPK);
            if ((present >> (tt * LPK)) & 1) {
                load_value_dims<SRC, DPL>(vbase_p + o_tt, e0, v[tt]);
            } else {
#pragma unroll
                for (int k = 0; k < DPL; ++k) v[tt][k] = 0.0f;
            }
        }
    }

    // this lane's 32 key values (Q8_0: 8 packed dwords, one block, unpacked per row in the score
    // loop; F16 / F32: the elements of its interleaved words, see kelem below)
    float x[STAGED ? 1 : 32];
    uint32_t kw[STAGED ? 8 : 1];
    if constexpr (STAGED) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            kw[4 * j] = kraw[j].x, kw[4 * j + 1] = kraw[j].y, kw[4 * j + 2] = kraw[j].z, kw[4 * j + 3] = kraw[j].w;
    } else if constexpr (SRC == kTypeF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t hw[4] = {have ? kraw[j].x : 0u, have ? kraw[j].y : 0u, have ? kraw[j].z : 0u,
                                    have ? kraw[j].w : 0u};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x[8 * j + 2 * k] = half_bits_to_float(hw[k] & 0xFFFF);
                x[8 * j + 2 * k + 1] = half_bits_to_float(hw[k] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[4 * j] = have ? __uint_as_float(kraw[j].x) : 0.0f, x[4 * j + 1] = have ? __uint_as_float(kraw[j].y) : 0.0f;
            x[4 * j + 2] = have ? __uint_as_float(kraw[j].z) : 0.0f, x[4 * j + 3] = have ? __uint_as_float(kraw[j].w) : 0.0f;
        }
    }

    if (!q_stored) {  // first chunk: publish the query rows (and the row state) to all waves
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int e = w.tid + 256 * u;
            sm.q[e / HD][e % HD] = qreg[u];
        }
        q_stored = true;
        __syncthreads();
    }

    // ---- scores. Element of x[4g .. 4g+3] within the head: Q8_0 32b + 4g (the lane's block);
    // F16 / F32 the interleaved 16-byte words (E16 = 8 or 4 elements per word)
    constexpr int E16 = SRC == kTypeF16 ? 8 : 4;
    auto kelem = [&](int g) { return STAGED ? 32 * b + 4 * g : (b + LPK * (4 * g / E16)) * E16 + (4 * g) % E16; };
    auto score_row = [&](int r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 qv = *reinterpret_cast<const float4*>(&sm.q[r][kelem(j)]);
            float x0, x1, x2, x3;
            if constexpr (STAGED) {
                x0 = (float)(int32_t)__builtin_amdgcn_sbfe(kw[j], 0, 8);
                x1 = (float)(int32_t)__builtin_amdgcn_sbfe(kw[j], 8, 8);
                x2 = (float)(int32_t)__builtin_amdgcn_sbfe(kw[j], 16, 8);
                x3 = (float)(int32_t)__builtin_amdgcn_sbfe(kw[j], 24, 8);
            } else {
                x0 = x[4 * j], x1 = x[4 * j + 1], x2 = x[4 * j + 2], x3 = x[4 * j + 3];
            }
            acc = fmaf(x0, qv.x, acc);
            acc = fmaf(x1, qv.y, acc);
            acc = fmaf(x2, qv.z, acc);
            acc = fmaf(x3, qv.w, acc);
        }
        acc = lanes_sum<LPK>(acc * sc);
        const int i = w.i0 + r / a.hpw;
        const bool vis = kt < klim && kt <= a.n_past + i;
        if (b == 0) sm.p[r][t] = vis ? acc * a.scale_log2e : -INFINITY;
    };
    if constexpr (RM <= 4) {
#pragma unroll
        for (int r = 0; r < RM; ++r)
            if (r < w.R) score_row(r);
    } else {
#pragma unroll 1
        for (int r = 0; r < w.R; ++r) score_row(r);
    }
    __syncthreads();

    // ---- softmax statistics; wave w owns rows w, w+4, ...
    for (int r = wave; r < w.R; r += 4) {
        float s[(KC + 63) / 64];
        float mc = -INFINITY;
#pragma unroll
        for (int u = 0; u < (KC + 63) / 64; ++u) {
            const int tu = lane + 64 * u;
            s[u] = tu < KC ? sm.p[r][tu] : -INFINITY;
            mc = fmaxf(mc, s[u]);
        }
        mc = wave_max(mc);
        const float m_old = sm.m[r];
        const float m_new = fmaxf(m_old, mc);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_old - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int u = 0; u < (KC + 63) / 64; ++u) {
            const int tu = lane + 64 * u;
            const float p = m_new == -INFINITY ? 0.0f : exp2f(s[u] - m_new);
            if (tu < KC) sm.p[r][tu] = p;
            ls += p;
        }
        ls = lanes_sum<64>(ls);
        if (lane == 0) {
            sm.m[r] = m_new;
            sm.l[r] = sm.l[r] * alpha + ls;
            sm.alpha[r] = alpha;
        }
    }
    __syncthreads();

    // ---- V: this wave's KPW keys, lanes over dims
    if constexpr (STAGED) {  // the wave's own LDS region: written and read by this wave only
#pragma unroll
        for (int j = 0; j < NST; ++j) sm.v[wave][lane + 64 * j] = vst[j];
        __builtin_amdgcn_wave_barrier();
        const uint8_t* vb = reinterpret_cast<const uint8_t*>(&sm.v[wave][0]);
#pragma unroll
        for (int tt = 0; tt < KPW; ++tt) load_value_dims<kTypeQ8_0, DPL>(vb + tt * HBW * 4, e0, v[tt]);
    }
    if constexpr (RAWV) {
#pragma unroll
        for (int tt = 0; tt < KPW; ++tt) value_from_raw<SRC, DPL>(vraw[tt], ((present >> (tt * LPK)) & 1) != 0, v[tt]);
    }
    auto v_row = [&](int r) {
        float acc[DPL];
        const float al = sm.alpha[r];
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[k] = sm.o[wave][r][DPL * lane + k] * al;
#pragma unroll
        for (int tt = 0; tt < KPW; ++tt) {
            const float p = sm.p[r][wave * KPW + tt];
#pragma unroll
            for (int k = 0; k < DPL; ++k) acc[k] = fmaf(p, v[tt][k], acc[k]);
        }
#pragma unroll
        for (int k = 0; k < DPL; ++k) sm.o[wave][r][DPL * lane + k] = acc[k];
    };
    if constexpr (RM <= 4) {
#pragma unroll
        for (int r = 0; r < RM; ++r)
            if (r < w.R) v_row(r);
    } else {
#pragma unroll 1
        for (int r = 0; r < w.R; ++r) v_row(r);
    }
    __syncthreads();
}

// The fields the query and block-table loads need come as scalar arguments ahead of the struct:
// the first 56 bytes of arguments are preloaded into scalar registers at dispatch
// (-amdgpu-kernarg-preload-count), so those loads issue without waiting for the struct's.
// hpw_nq = hpw | nq << 8; rep = n_head / n_head_kv.
template <int CT, int HD, int RMAX>
__global__ void __launch_bounds__(256, RMAX <= 4 ? 3 : 1) attn_kernel(const int32_t* table, const float* q,
                                                                    int64_t q_stride, int n_table, int n_tokens,
                                                                    int n_past, int splits, int groups, int cps,
                                                                    int rep, int hpw_nq, AttnArgs a) {
    using S = AttnShape<HD>;
    constexpr int KC = S::KC, DPL = S::DPL;
    __shared__ AttnSmem<HD, RMAX> sm;
    a.table = table, a.q = q, a.q_stride = q_stride, a.n_table = n_table, a.n_tokens = n_tokens;
    a.n_past = n_past, a.splits = splits, a.groups = groups, a.cps = cps;
    a.hpw = hpw_nq & 0xFF, a.nq = hpw_nq >> 8;
    a.nch_hist = (n_past + KC - 1) / KC;  // as the host's plan, with KC = 8192 / HD
    a.nch_total = a.nch_hist + (n_tokens + KC - 1) / KC;

    AttnTile w;
    w.tid = threadIdx.x, w.wave = w.tid >> 6, w.lane = w.tid & 63;
    const int tid = w.tid, wave = w.wave, lane = w.lane;
    // Workgroup -> (split, group, query tile), XCD-aware: workgroup ids are dealt to the 8 XCDs
    // round-robin (id % 8), and each XCD has its own L2. With the keys split, the groups of one
    // split share its slots' cache lines (a head's piece does not fill them), so the split's low
    // three bits come from id % 8 and all its groups land on one XCD. Without splitting, the
    // query tiles of one group share its K/V and the group index is id % groups.
    int split, group, qt;
    {
        const int id = blockIdx.x;
        if (a.splits > 1) {
            const int rest = id >> 3, sblk = (a.splits + 7) >> 3;
            group = rest % a.groups;
            split = ((rest / a.groups) % sblk) * 8 + (id & 7);
            qt = (rest / a.groups) / sblk;
            if (split >= a.splits) return;  // padding to a multiple of 8 splits: the whole group
        } else {
            split = 0;
            group = id % a.groups;
            qt = id / a.groups;
        }
    }
    const int groups_per_kv = rep / a.hpw;
    w.h_kv = group / groups_per_kv;
    const int h0 = w.h_kv * rep + (group % groups_per_kv) * a.hpw;
    w.i0 = qt * a.nq;
    w.R = a.nq * a.hpw;
    w.hb = head_bytes<CT>(HD);
    const int i_last = min(w.i0 + a.nq, a.n_tokens) - 1;

    // query rows r -> token i0 + r / hpw, head h0 + r % hpw (zeros past the last token), loaded
    // into registers now and stored to LDS by the first chunk after its loads are issued
    constexpr int QPT = RMAX * HD / 256;
    float qreg[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int e = tid + 256 * u, r = e / HD, d = e % HD;
        const int i = w.i0 + r / a.hpw, h = h0 + r % a.hpw;
        qreg[u] = r < w.R && i < a.n_tokens ? a.q[(int64_t)i * a.q_stride + (int64_t)h * HD + d] : 0.0f;
    }
    if (tid < RMAX) {
        sm.m[tid] = -INFINITY;
        sm.l[tid] = 0.0f;
    }
    for (int r = 0; r < w.R; ++r)
#pragma unroll
        for (int k = 0; k < DPL; ++k) sm.o[wave][r][DPL * lane + k] = 0.0f;

    // chunks this workgroup visits: its split's range, cut at the last key its last token sees
    // (keys 0 .. n_past + i_last are visible to some row; the last of them is a current row)
    const int c_begin = split * a.cps;
    const int c_vis = a.nch_hist + i_last / KC;
    const int c_end = min(min(c_begin + a.cps, a.nch_total), c_vis + 1);
    // the first chunk's block-table entry, loaded from the preloaded arguments before anything
    // waits for the struct's fields (the same lookup attn_chunk makes for a history chunk)
    int blk_first = -1;
    if (c_begin < c_end && c_begin < a.nch_hist) {
        const int kt = c_begin * KC + wave * S::KPW + lane / S::LPK, lb = kt / kKvBlock;
        blk_first = kt < n_past && lb < n_table ? table[lb] : -1;
    }
    bool q_stored = false;
    for (int c = c_begin; c < c_end; ++c) {
        if (c < a.nch_hist)
            attn_chunk<CT, false, HD, RMAX, QPT>(a, w, sm, c * KC, a.n_past, q_stored, qreg,
                                                 c == c_begin ? blk_first : -2);
        else
            attn_chunk<kTypeF32, true, HD, RMAX, QPT>(a, w, sm, a.n_past + (c - a.nch_hist) * KC, a.n_past + a.n_tokens,
                                                q_stored, qreg);
    }

    // ---- merge the four waves' partial sums and write (after a chunk's closing barrier; with no
    // chunk, after the zeroing above)
    if (c_begin >= c_end) __syncthreads();
    const bool direct = a.ws_o == nullptr;
    for (int e = tid; e < w.R * HD; e += 256) {
        const int r = e / HD, d = e % HD;
        const int i = w.i0 + r / a.hpw, h = h0 + r % a.hpw;
        if (i >= a.n_tokens) continue;
        const float sum = ((sm.o[0][r][d] + sm.o[1][r][d]) + sm.o[2][r][d]) + sm.o[3][r][d];
        if (direct) {
            a.out[(int64_t)i * a.out_stride + (int64_t)h * HD + d] = sum / sm.l[r];
        } else {
            const int64_t row = ((int64_t)split * a.n_tokens + i) * a.n_head + h;
            a.ws_o[row * HD + d] = sum;
            if (d == 0) {
                a.ws_ml[2 * row] = sm.m[r];
                a.ws_ml[2 * row + 1] = sm.l[r];
            }
        }
    }
}

// out[i][h][:] from the splits' (m, l, o): M = max m, L = sum l 2^(m-M), out = sum o 2^(m-M) / L.
// A split that saw no key of row (i, h) has m = -inf and l = 0 and drops out. Workgroup: one row,
// 32 dims, the splits dealt to 8 groups of 32 threads. Each thread merges its splits online
// (running max, rescaled sums), so its loads do not wait on one another; the 8 groups are then
// merged the same way.
__device__ __forceinline__ void merge_online(float& m, float& l, float& acc, float ms, float lv, float ov) {
    const float mn = fmaxf(m, ms);
    const float c0 = mn == -INFINITY ? 1.0f : exp2f(m - mn);  // m = -inf below a finite mn: 0
    const float c1 = ms == -INFINITY ? 0.0f : exp2f(ms - mn);
    l = l * c0 + lv * c1;
    acc = acc * c0 + ov * c1;
    m = mn;
}

__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml, int splits,
                                                           int n_tokens, int n_head, int hd, float* __restrict__ out,
                                                           int64_t out_stride) {
    __shared__ float pm[8][32], pl[8][32], pa[8][32];
    const int row = blockIdx.x;  // i * n_head + h
    const int i = row / n_head, h = row % n_head;
    const int64_t rows = (int64_t)n_tokens * n_head;
    const int tid = threadIdx.x, d = blockIdx.y * 32 + (tid & 31), g = tid >> 5;
    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    for (int s0 = g; s0 < splits; s0 += 8 * 16) {  // 16 splits per thread per pass, loads first
        float mv[16], lv[16], ov[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int s = s0 + 8 * k;
            const int64_t r = (int64_t)s * rows + row;
            mv[k] = s < splits ? ws_ml[2 * r] : -INFINITY;
            lv[k] = s < splits ? ws_ml[2 * r + 1] : 0.0f;
            ov[k] = s < splits ? ws_o[r * hd + d] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) merge_online(m, l, acc, mv[k], lv[k], ov[k]);
    }
    pm[g][tid & 31] = m, pl[g][tid & 31] = l, pa[g][tid & 31] = acc;
    __syncthreads();
    if (tid < 32) {
        float mm = -INFINITY, ll = 0.0f, aa = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) merge_online(mm, ll, aa, pm[k][tid], pl[k][tid], pa[k][tid]);
        out[(int64_t)i * out_stride + (int64_t)h * hd + d] = aa / ll;
    }
}

// Few splits over many rows (prompts): one thread per 4 consecutive output elements (head_dim a
// multiple of 4: the MFMA kernel's 64 and 128), the splits' loads issued together (S <= 16).
// Two passes over the splits: the row maximum, then the weighted sums, so a thread evaluates
// S powers of two for its 4 elements (the sequential merge took 2 S per element).
template <int S>
__global__ void __launch_bounds__(256) attn_combine_few_kernel(const float* __restrict__ ws_o,
                                                               const float* __restrict__ ws_ml, int splits,
                                                               int n_tokens, int n_head, int hd,
                                                               float* __restrict__ out, int64_t out_stride) {
    const int64_t rows = (int64_t)n_tokens * n_head;
    const int q4 = hd / 4;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * q4) return;
    const int64_t row = idx / q4;
    const int d = (int)(idx % q4) * 4;
    float mv[S], lv[S];
    float4 ov[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t r = (int64_t)s * rows + row;
        mv[s] = s < splits ? ws_ml[2 * r] : -INFINITY;
        lv[s] = s < splits ? ws_ml[2 * r + 1] : 0.0f;
        ov[s] = s < splits ? *reinterpret_cast<const float4*>(ws_o + r * hd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < S; ++s) m = fmaxf(m, mv[s]);  // finite: every row sees at least one key
    float l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const float c = mv[s] == -INFINITY ? 0.0f : exp2f(mv[s] - m);  // a split without keys adds 0
        l = fmaf(lv[s], c, l);
        acc.x = fmaf(ov[s].x, c, acc.x);
        acc.y = fmaf(ov[s].y, c, acc.y);
        acc.z = fmaf(ov[s].z, c, acc.z);
        acc.w = fmaf(ov[s].w, c, acc.w);
    }
    const float inv = 1.0f / l;
    const int i = (int)(row / n_head), h = (int)(row % n_head);
    float* o = out + (int64_t)i * out_stride + (int64_t)h * hd + d;
    o[0] = acc.x * inv;
    o[1] = acc.y * inv;
    o[2] = acc.z * inv;
    o[3] = acc.w * inv;
}

// Many splits over few rows (decode): the splits of each 4-element output are dealt to P
// consecutive lanes (lane p takes splits p, p + P, ..., at most NS of them, all loads issued
// together), and the lanes combine by exchange (DPP inside 16-lane rows, one lane permute
// across rows): the row maximum first, then the weighted sums, one exp2 per split. A decode call at n_past = 4095 (65 splits over 32 rows x 32 quads) runs
// 32768 threads with at most three splits each: 15.4 us per call with the attention kernel,
// against 15.7 us with 16 lanes per output and 16.7 us with the workgroup-per-row kernel.
template <int P, int NS>
__global__ void __launch_bounds__(256) attn_combine_lanes_kernel(const float* __restrict__ ws_o,
                                                                 const float* __restrict__ ws_ml, int splits,
                                                                 int n_tokens, int n_head, int hd,
                                                                 float* __restrict__ out, int64_t out_stride) {
    static_assert(P <= 64 && (P & (P - 1)) == 0, "a unit's lanes share a wave");
    const int64_t rows = (int64_t)n_tokens * n_head;
    const int q4 = hd / 4;
    const int64_t unit = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / P;  // row * q4 + quad
    const int p = threadIdx.x & (P - 1);
    const bool ok = unit < rows * q4;  // uniform over the unit's 16 lanes
    const int64_t row = ok ? unit / q4 : 0;
    const int d = ok ? (int)(unit % q4) * 4 : 0;
    float2 ml[NS];
    float4 ov[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int s = p + P * k;
        const int64_t r = (int64_t)s * rows + row;
        const bool have = ok && s < splits;
        ml[k] = have ? *reinterpret_cast<const float2*>(ws_ml + 2 * r) : make_float2(-INFINITY, 0.0f);
        ov[k] = have ? *reinterpret_cast<const float4*>(ws_o + r * hd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NS; ++k) m = fmaxf(m, ml[k].x);
    m = lanes_max<P>(m);  // finite for a real row
    float l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const float c = ml[k].x == -INFINITY ? 0.0f : exp2f(ml[k].x - m);  // a split without keys adds 0
        l = fmaf(ml[k].y, c, l);
        acc.x = fmaf(ov[k].x, c, acc.x);
        acc.y = fmaf(ov[k].y, c, acc.y);
        acc.z = fmaf(ov[k].z, c, acc.z);
        acc.w = fmaf(ov[k].w, c, acc.w);
    }
    l = lanes_sum<P>(l);
    acc.x = lanes_sum<P>(acc.x);
    acc.y = lanes_sum<P>(acc.y);
    acc.z = lanes_sum<P>(acc.z);
    acc.w = lanes_sum<P>(acc.w);
    if (!ok || p != 0) return;
    const float inv = 1.0f / l;
    const int i = (int)(row / n_head), h = (int)(row % n_head);
    float* o = out + (int64_t)i * out_stride + (int64_t)h * hd + d;
    o[0] = acc.x * inv;
    o[1] = acc.y * inv;
    o[2] = acc.z * inv;
    o[3] = acc.w * inv;
}

// ---------------------------------------------------------------- prompt attention on fp32 MFMA
// For prompts (head_dim 64 or 128, query-head groups that divide into fours): a workgroup is 4
// waves = 4 query heads of one KV head over the same 32 query tokens; it walks the keys its
// tile sees in blocks of 32 with the online softmax in base 2 of the VALU kernel above.
//   Per block the workgroup stages K ([key][dim]) and V transposed ([dim][key]) in LDS as fp32
//   (Q8_0 / F16 slots decoded, the batch's own rows copied), shared by its four heads.
//   S^T = K Q^T (keys x queries) by v_mfma_f32_32x32x2f32 over head_dim in HD/2 steps: in step
//   s lane l supplies key l%32 and query l%32 at dim HD/2 * (l/32) + s. In the 32x32 result
//   lane l holds S^T[8(i/4) + 4(l/32) + i%4][l%32], i = 0..15: sixteen keys of ONE query row,
//   so the row's max and sum are the lane's own plus one exchange with the other half-wave.
//   O^T += V^T P^T (dims x queries) in 32-dim tiles and 16 steps over the block's keys: step s
//   takes key 8(s/4) + 4(l/32) + s%4, which is the lane's own P value i = s, so P needs no
//   transpose and the rescale of O^T by the row's alpha is lane-local.
// The products are fp32 and the sums fp32 (in the MFMA's order), as in the VALU kernel.
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int kAttnMfmaMinTokens = 32;

template <int HD>
struct __align__(16) MfmaAttnSmem {
    static constexpr int KP = HD + 4;  // K row pitch (floats), keeps rows 16-byte aligned
    static constexpr int VP = 36;      // V^T row pitch: 32 keys + 4
    float k[32][KP];
    float vt[HD][VP];
};

// E consecutive elements e0 .. e0+E-1 of a head's piece (E = 8 or 16: inside one Q8_0 block)
template <int CT, int E>
__device__ __forceinline__ void load_head_elems(const uint8_t* head, int e0, float (&out)[E]) {
    if constexpr (CT == kTypeQ8_0) {
        const uint8_t* b = head + (e0 / 32) * 34;
        const float d = half_bits_to_float(ldu16(b));
        const uint8_t* qs = b + 2 + (e0 % 32);  // 2-byte aligned
        uint32_t w[E / 4];
        if constexpr (E == 16) {
            ld16_a2(qs, w);
        } else {
#pragma unroll
            for (int j = 0; j < E / 4; ++j) w[j] = ldu16(qs + 4 * j) | (ldu16(qs + 4 * j + 2) << 16);
        }
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = d * (float)(int32_t)__builtin_amdgcn_sbfe(w[j / 4], 8 * (j % 4), 8);
    } else if constexpr (CT == kTypeF16) {
#pragma unroll
        for (int j = 0; j < E / 8; ++j) {
            const uint4 h = ld16(head + 2 * e0 + 16 * j);
            const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                out[8 * j + 2 * k] = half_bits_to_float(hw[k] & 0xFFFF);
                out[8 * j + 2 * k + 1] = half_bits_to_float(hw[k] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < E / 4; ++j) {
            const float4 f = *reinterpret_cast<const float4*>(head + 4 * e0 + 16 * j);
            out[4 * j] = f.x, out[4 * j + 1] = f.y, out[4 * j + 2] = f.z, out[4 * j + 3] = f.w;
        }
    }
}

template <int CT, int HD>
__global__ void __launch_bounds__(256, 2) attn_mfma_kernel(AttnArgs a) {
    constexpr int E = HD / 8;     // elements per staging thread
    constexpr int HALF = HD / 2;  // steps of the score product
    constexpr int NT = HD / 32;   // 32-dim tiles of the output
    __shared__ MfmaAttnSmem<HD> sm;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int p = lane >> 5, c32 = lane & 31;
    const int rep = a.n_head / a.n_head_kv, quads = rep / 4;
    const int n_qt = (a.n_tokens + 31) / 32;
    const int per_tile = a.n_head_kv * quads;
    const int id = blockIdx.x;
    const int grp = id % per_tile;
    const int split = (id / per_tile) % a.splits;
    // query tiles see 1, 2, ... key blocks: the first half of the launch order takes the largest
    // tiles, descending, the second half the smallest, ascending, so that the two workgroups a
    // CU receives (one from each half, in dispatch order) carry about the same keys together
    const int rank = id / per_tile / a.splits, half = (n_qt + 1) / 2;
    const int qt = rank < half ? n_qt - 1 - rank : rank - half;
    const int h_kv = grp / quads;
    const int h = h_kv * rep + (grp % quads) * 4 + wave;
    const int i0 = qt * 32;
    const int iq = i0 + c32;  // this lane's query token
    const bool q_ok = iq < a.n_tokens;
    const int64_t hb = head_bytes<CT>(HD);

    // the lane's query row at dims HALF*p .. HALF*p + HALF - 1, pre-scaled to base-2 scores
    float qr[HALF];
    {
        const float4* qp = reinterpret_cast<const float4*>(a.q + (int64_t)(q_ok ? iq : 0) * a.q_stride +
                                                           (int64_t)h * HD + HALF * p);
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const float4 v = qp[j];
            qr[4 * j] = q_ok ? v.x * a.scale_log2e : 0.0f;
            qr[4 * j + 1] = q_ok ? v.y * a.scale_log2e : 0.0f;
            qr[4 * j + 2] = q_ok ? v.z * a.scale_log2e : 0.0f;
            qr[4 * j + 3] = q_ok ? v.w * a.scale_log2e : 0.0f;
        }
    }
    v16f o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    // keys 0 .. n_past + last token are visible to some row of the tile; with key splits this
    // workgroup takes blocks [split * cps, split * cps + cps) of them (possibly none)
    const int last_tok = min(i0 + 31, a.n_tokens - 1);
    const int nblk = (a.n_past + last_tok + 1 + 31) / 32;
    const int b_begin = split * a.cps, b_end = min(nblk, b_begin + a.cps);
    const int skey = tid & 31, se0 = E * (tid >> 5);  // staging: one key, E elements
    for (int bi = b_begin; bi < b_end; ++bi) {
        const int kb = 32 * bi;
        // ---- stage the block's K and V^T: history slots (missing blocks read as zeros), the
        // batch's own fp32 rows, zeros past the last key
        {
            const int kk = kb + skey;
            float kv[E], vv[E];
#pragma unroll
            for (int j = 0; j < E; ++j) kv[j] = vv[j] = 0.0f;
            if (kk < a.n_past) {
                const int lb = kk / kKvBlock;
                const int blk = lb < a.n_table ? a.table[lb] : -1;
                if (blk >= 0 && blk < a.n_blocks) {
                    const int64_t off = (((int64_t)blk * a.n_layer + a.layer) * kKvBlock + kk % kKvBlock) * a.sb +
                                        (int64_t)h_kv * hb;
                    load_head_elems<CT, E>(a.k_arena + off, se0, kv);
                    load_head_elems<CT, E>(a.v_arena + off, se0, vv);
                }
            } else if (kk < a.n_past + a.n_tokens) {
                const int64_t off = ((int64_t)(kk - a.n_past) * a.kv_stride + (int64_t)h_kv * HD) * 4;
                load_head_elems<kTypeF32, E>(reinterpret_cast<const uint8_t*>(a.k_cur) + off, se0, kv);
                load_head_elems<kTypeF32, E>(reinterpret_cast<const uint8_t*>(a.v_cur) + off, se0, vv);
            }
#pragma unroll
            for (int j = 0; j < E; j += 4)
                *reinterpret_cast<float4*>(&sm.k[skey][se0 + j]) = make_float4(kv[j], kv[j + 1], kv[j + 2], kv[j + 3]);
#pragma unroll
            for (int j = 0; j < E; ++j) sm.vt[se0 + j][skey] = vv[j];
        }
        __syncthreads();

        // ---- S^T = K Q^T
        v16f sc;
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[v] = 0.0f;
#pragma unroll
        for (int c = 0; c < HALF / 16; ++c) {
            float kr[16];
            const float4* kp = reinterpret_cast<const float4*>(&sm.k[c32][HALF * p + 16 * c]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = kp[j];
                kr[4 * j] = v.x, kr[4 * j + 1] = v.y, kr[4 * j + 2] = v.z, kr[4 * j + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[j], qr[16 * c + j], sc, 0, 0, 0);
        }

        // ---- causal mask and the online softmax of row iq
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kk = kb + 8 * (i >> 2) + 4 * p + (i & 3);
            sc[i] = kk <= a.n_past + iq ? sc[i] : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
        float pv[16], ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pv[i] = m_new == -INFINITY ? 0.0f : exp2f(sc[i] - m_new);
            ls += pv[i];
        }
        ls += __shfl_xor(ls, 32, 64);
        l_run = l_run * alpha + ls;
        m_run = m_new;

        // ---- O^T = alpha O^T + V^T P^T
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) o[t][v] *= alpha;
            float vr[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = *reinterpret_cast<const float4*>(&sm.vt[32 * t + c32][8 * j + 4 * p]);
                vr[4 * j] = v.x, vr[4 * j + 1] = v.y, vr[4 * j + 2] = v.z, vr[4 * j + 3] = v.w;
            }
#pragma unroll
            for (int st = 0; st < 16; ++st) o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vr[st], pv[st], o[t], 0, 0, 0);
        }
        __syncthreads();  // the next block overwrites the staging
    }

    // ---- the lane's query row: dims 32t + 8(v/4) + 4p + v%4 of O^T / l, or with key splits
    // the unnormalised sums and (m, l) for the combine kernel (m = -inf, l = 0 if no key)
    if (q_ok) {
        if (a.splits == 1) {
            float* orow = a.out + (int64_t)iq * a.out_stride + (int64_t)h * HD;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) orow[32 * t + 8 * (v >> 2) + 4 * p + (v & 3)] = o[t][v] / l_run;
        } else {
            const int64_t row = ((int64_t)split * a.n_tokens + iq) * a.n_head + h;
            float* orow = a.ws_o + row * HD;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<float4*>(orow + 32 * t + 8 * j + 4 * p) =
                        make_float4(o[t][4 * j], o[t][4 * j + 1], o[t][4 * j + 2], o[t][4 * j + 3]);
            if (p == 0) {
                a.ws_ml[2 * row] = m_run;
                a.ws_ml[2 * row + 1] = l_run;
            }
        }
    }
}

// ---------------------------------------------------------------- launchers
hipError_t launch_kv_write(int ct, void* arena, int n_blocks, int n_layer, int layer, int64_t row_elems, int64_t sb,
                           const int32_t* table, int pos0, const float* src, int64_t src_stride, int n_tokens,
                           hipStream_t st) {
    if (n_tokens <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)n_tokens), dim3(256), 0, st, ct,
                       static_cast<uint8_t*>(arena), n_blocks, n_layer, layer, row_elems, sb, table, pos0, src,
                       src_stride);
    return hipGetLastError();
}

hipError_t launch_kv_gather(int ct, const void* arena, int n_blocks, int n_layer, int layer, int64_t row_elems,
                            int64_t sb, const int32_t* table, int n_table, int n_past, const float* cur,
                            int64_t cur_stride, int n_tokens, float* dst, int64_t dst_stride, hipStream_t st) {
    const int rows = n_past + n_tokens;
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)rows), dim3(256), 0, st, ct,
                       static_cast<const uint8_t*>(arena), n_blocks, n_layer, layer, row_elems, sb, table, n_table,
                       n_past, cur, cur_stride, dst, dst_stride);
    return hipGetLastError();
}

// Work decomposition shared by the workspace query and the launch.
struct AttnPlan {
    int kc, rmax, hpw, nq, nch_hist, nch_total, cps, splits, qtiles, groups;
};

static int attn_kc(int hd) { return 8192 / hd; }

static AttnPlan attn_plan(int hd, int n_head, int n_head_kv, int n_tokens, int n_past) {
    AttnPlan p{};
    p.kc = attn_kc(hd);
    const int rep = n_head / n_head_kv;
    p.rmax = rep <= 4 && (int64_t)n_tokens * rep <= 4 ? 4 : (hd >= 256 ? 8 : 16);
    p.hpw = 1;
    for (int d = 1; d <= rep && d <= p.rmax; ++d)
        if (rep % d == 0) p.hpw = d;
    p.nq = p.rmax / p.hpw;
    if (p.nq > n_tokens) p.nq = n_tokens;
    p.nch_hist = (n_past + p.kc - 1) / p.kc;
    p.nch_total = p.nch_hist + (n_tokens + p.kc - 1) / p.kc;
    p.qtiles = (n_tokens + p.nq - 1) / p.nq;
    p.groups = n_head / p.hpw;
    // spread the keys over workgroups until about 1024 of them are in flight
    const int64_t base = (int64_t)p.qtiles * p.groups;
    int want = (int)((1024 + base - 1) / base);
    if (want > p.nch_total) want = p.nch_total;
    if (want < 1) want = 1;
    p.cps = (p.nch_total + want - 1) / want;
    p.splits = (p.nch_total + p.cps - 1) / p.cps;
    return p;
}

// Prompts take the MFMA kernel: head_dim 64 or 128, query-head groups that divide into fours,
// at least kAttnMfmaMinTokens tokens.
static bool attn_use_mfma(int hd, int n_head, int n_head_kv, int n_tokens) {
    return (hd == 64 || hd == 128) && (n_head / n_head_kv) % 4 == 0 && n_tokens >= kAttnMfmaMinTokens &&
           knob(Knob::AttnNoMfma) == 0;
}

// Key splits of the MFMA kernel: about 512 workgroups in flight (two per CU), at least 8 key
// blocks of 32 per split (the last query tile's count) so the combine stays small.
struct MfmaPlan {
    int splits, bps;  // splits, key blocks per split
};
static MfmaPlan attn_mfma_plan(int n_head, int n_tokens, int n_past) {
    const int64_t base = (int64_t)((n_tokens + 31) / 32) * (n_head / 4);
    const int nblk_max = (n_past + n_tokens + 31) / 32;
    int want = (int)((512 + base - 1) / base);
    const int cap = (nblk_max + 7) / 8;
    if (want > cap) want = cap;
    if (want < 1) want = 1;
    MfmaPlan m;
    m.bps = (nblk_max + want - 1) / want;
    m.splits = (nblk_max + m.bps - 1) / m.bps;
    return m;
}

size_t attn_workspace_bytes(int hd, int n_head, int n_head_kv, int n_tokens, int n_past) {
    if (attn_use_mfma(hd, n_head, n_head_kv, n_tokens)) {
        const MfmaPlan m = attn_mfma_plan(n_head, n_tokens, n_past);
        if (m.splits <= 1) return 0;
        const size_t rows = (size_t)m.splits * n_tokens * n_head;
        return round_up((int64_t)(rows * hd * 4), 256) + round_up((int64_t)(rows * 2 * 4), 256);
    }
    const AttnPlan p = attn_plan(hd, n_head, n_head_kv, n_tokens, n_past);
    if (p.splits <= 1) return 0;
    const size_t rows = (size_t)p.splits * n_tokens * n_head;
    return round_up((int64_t)(rows * hd * 4), 256) + round_up((int64_t)(rows * 2 * 4), 256);
}

template <int CT, int HD>
static void launch_attn_t(const AttnArgs& a, int rmax, dim3 grid, hipStream_t st) {
    const int rep = a.n_head / a.n_head_kv, hpw_nq = a.hpw | a.nq << 8;
#define DCQ_ATTN_ARGS a.table, a.q, a.q_stride, a.n_table, a.n_tokens, a.n_past, a.splits, a.groups, a.cps, rep, hpw_nq, a
    if (rmax == 4)
        hipLaunchKernelGGL((attn_kernel<CT, HD, 4>), grid, dim3(256), 0, st, DCQ_ATTN_ARGS);
    else
        hipLaunchKernelGGL((attn_kernel<CT, HD, attn_rmax_large<HD>()>), grid, dim3(256), 0, st, DCQ_ATTN_ARGS);
#undef DCQ_ATTN_ARGS
}

// The merge of the key splits: one thread per 4 output elements for up to 16 splits (prompts:
// many rows), 32 lanes per 4 elements for up to 128 (decode: few rows, many splits), else the
// workgroup-per-row kernel.
static hipError_t launch_attn_combine(const float* ws_o, const float* ws_ml, int splits, int n_tokens, int n_head,
                                      int hd, float* out, int64_t out_stride, hipStream_t st) {
    const int64_t quads = (int64_t)n_tokens * n_head * (hd / 4);
    const dim3 few_grid((unsigned)((quads + 255) / 256)), lane_grid((unsigned)((32 * quads + 255) / 256));
#define DCQ_COMBINE(KERNEL, GRID) \
    hipLaunchKernelGGL(KERNEL, GRID, dim3(256), 0, st, ws_o, ws_ml, splits, n_tokens, n_head, hd, out, out_stride)
    if (splits <= 4)
        DCQ_COMBINE(attn_combine_few_kernel<4>, few_grid);
    else if (splits <= 8)
        DCQ_COMBINE(attn_combine_few_kernel<8>, few_grid);
    else if (splits <= 16)
        DCQ_COMBINE(attn_combine_few_kernel<16>, few_grid);
    else if (splits <= 64)
        DCQ_COMBINE((attn_combine_lanes_kernel<32, 2>), lane_grid);
    else if (splits <= 96)
        DCQ_COMBINE((attn_combine_lanes_kernel<32, 3>), lane_grid);
    else if (splits <= 128)
        DCQ_COMBINE((attn_combine_lanes_kernel<32, 4>), lane_grid);
    else
        DCQ_COMBINE(attn_combine_kernel, dim3((unsigned)(n_tokens * n_head), (unsigned)(hd / 32)));
#undef DCQ_COMBINE
    return hipGetLastError();
}

hipError_t launch_kv_attention(int ct, const void* k_arena, const void* v_arena, int n_blocks, int n_layer, int layer,
                               int64_t sb, const int32_t* table, int n_table, int n_head, int n_head_kv, int hd,
                               const float* q, int64_t q_stride, const float* k_cur, const float* v_cur,
                               int64_t kv_stride, int n_tokens, int n_past, float scale, float* out,
                               int64_t out_stride, void* ws, size_t ws_bytes, hipStream_t st) {
    const bool mfma = attn_use_mfma(hd, n_head, n_head_kv, n_tokens);
    const AttnPlan p = attn_plan(hd, n_head, n_head_kv, n_tokens, n_past);
    if (ws_bytes < attn_workspace_bytes(hd, n_head, n_head_kv, n_tokens, n_past)) return hipErrorInvalidValue;
    AttnArgs a{};
    a.k_arena = static_cast<const uint8_t*>(k_arena);
    a.v_arena = static_cast<const uint8_t*>(v_arena);
    a.n_blocks = n_blocks, a.n_layer = n_layer, a.layer = layer, a.sb = sb;
    a.table = table, a.n_table = n_table;
    a.q = q, a.q_stride = q_stride, a.k_cur = k_cur, a.v_cur = v_cur, a.kv_stride = kv_stride;
    a.out = out, a.out_stride = out_stride;
    a.n_tokens = n_tokens, a.n_past = n_past, a.n_head = n_head, a.n_head_kv = n_head_kv;
    a.hpw = p.hpw, a.nq = p.nq, a.nch_hist = p.nch_hist, a.nch_total = p.nch_total, a.cps = p.cps;
    a.splits = p.splits, a.groups = p.groups;
    a.scale_log2e = scale * 1.4426950408889634f;
    if (mfma) {
        const MfmaPlan m = attn_mfma_plan(n_head, n_tokens, n_past);
        a.splits = m.splits, a.cps = m.bps;
        if (m.splits > 1) {
            const size_t rows = (size_t)m.splits * n_tokens * n_head;
            a.ws_o = static_cast<float*>(ws);
            a.ws_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + round_up((int64_t)(rows * hd * 4), 256));
        }
        const int64_t wgs = (int64_t)((n_tokens + 31) / 32) * (n_head / 4) * m.splits;
        if (wgs > INT32_MAX) return hipErrorInvalidValue;
        const dim3 grid((unsigned)wgs);
#define DCQ_ATTN_MFMA_CASE(C, H)                                                  \
    if (ct == C && hd == H) {                                                     \
        hipLaunchKernelGGL((attn_mfma_kernel<C, H>), grid, dim3(256), 0, st, a); \
    } else
        DCQ_ATTN_MFMA_CASE(kTypeQ8_0, 128)
        DCQ_ATTN_MFMA_CASE(kTypeQ8_0, 64)
        DCQ_ATTN_MFMA_CASE(kTypeF16, 128)
        DCQ_ATTN_MFMA_CASE(kTypeF16, 64)
        DCQ_ATTN_MFMA_CASE(kTypeF32, 128)
        DCQ_ATTN_MFMA_CASE(kTypeF32, 64)
        return hipErrorNotSupported;
#undef DCQ_ATTN_MFMA_CASE
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || m.splits <= 1) return e;
        return launch_attn_combine(a.ws_o, a.ws_ml, m.splits, n_tokens, n_head, hd, out, out_stride, st);
    }
    if (p.splits > 1) {
        const size_t rows = (size_t)p.splits * n_tokens * n_head;
        a.ws_o = static_cast<float*>(ws);
        a.ws_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + round_up((int64_t)(rows * hd * 4), 256));
    }
    const int64_t wgs = (int64_t)(p.splits > 1 ? (p.splits + 7) / 8 * 8 : 1) * p.groups * p.qtiles;
    if (wgs > INT32_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)wgs);
#define DCQ_ATTN_CASE(C, H)           \
    if (ct == C && hd == H) {         \
        launch_attn_t<C, H>(a, p.rmax, grid, st); \
    } else
    DCQ_ATTN_CASE(kTypeQ8_0, 128)
    DCQ_ATTN_CASE(kTypeQ8_0, 64)
    DCQ_ATTN_CASE(kTypeQ8_0, 256)
    DCQ_ATTN_CASE(kTypeF16, 128)
    DCQ_ATTN_CASE(kTypeF16, 64)
    DCQ_ATTN_CASE(kTypeF16, 256)
    DCQ_ATTN_CASE(kTypeF32, 128)
    DCQ_ATTN_CASE(kTypeF32, 64)
    DCQ_ATTN_CASE(kTypeF32, 256)
    return hipErrorNotSupported;
#undef DCQ_ATTN_CASE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.splits <= 1) return e;
    return launch_attn_combine(a.ws_o, a.ws_ml, p.splits, n_tokens, n_head, hd, out, out_stride, st);
}

}  // namespace dcq
