/*
 * dcq_oracle.c — scalar CPU restatement of the quantized mul_mat hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see dcq_oracle.h): the checker for the HIP
 * library, never part of it. Built with -ffp-contract=off so every fp32
 * multiply and add rounds separately, as the reference's C does on a target
 * without FMA contraction.
 *
 * Reference call sites this follows (paths relative to /root/reference):
 *   core/src/inference.cpp:887-894   from_float(X -> vec_dot_type) once per call
 *   core/src/inference.cpp:916-923   vec_dot(K, &y[n], W + n*nb1, Xq, ...) per row
 *   core/src/inference.cpp:970-984   vec_dot_type selection via type traits
 *   core/src/simd_ops.cpp:140-171    row-range contract, output relative to k_start
 *   core/include/simd_ops.h:3298-3305 weight -> activation type mapping
 *   core/shaders/quantized_gemv.metal:85-88  block_q8_0 {half; int8[32]}
 * The block arithmetic is ggml's (absent submodule, .gitmodules:1-3),
 * restated from the GGUF block definitions.
 */
#include "dcq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* Block layouts (GGUF). Sizes are part of the on-disk format.               */
/* ------------------------------------------------------------------------ */
#define QK8_0 32
#define QK_K 256

typedef struct {
    uint16_t d;
    int8_t qs[QK8_0];
} blk_q8_0;
typedef struct {
    uint16_t d;
    uint8_t qs[QK8_0 / 2]; /* element j: low nibble of qs[j]; element j + 16: its high nibble */
} blk_q4_0;
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[QK_K / 2];
} blk_q4_K;
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qh[QK_K / 8]; /* bit j of qh[l]: the fifth bit of element l of sub-block j */
    uint8_t qs[QK_K / 2]; /* the low four bits, packed as in Q4_K */
} blk_q5_K;
typedef struct {
    uint8_t ql[QK_K / 2];
    uint8_t qh[QK_K / 4];
    int8_t scales[QK_K / 16];
    uint16_t d;
} blk_q6_K;
typedef struct {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
} blk_q8_K;

_Static_assert(sizeof(blk_q8_0) == 34, "Q8_0 block is 34 bytes");
_Static_assert(sizeof(blk_q4_0) == 18, "Q4_0 block is 18 bytes");
_Static_assert(sizeof(blk_q4_K) == 144, "Q4_K block is 144 bytes");
_Static_assert(sizeof(blk_q5_K) == 176, "Q5_K block is 176 bytes");
_Static_assert(sizeof(blk_q6_K) == 210, "Q6_K block is 210 bytes");
_Static_assert(sizeof(blk_q8_K) == 292, "Q8_K block is 292 bytes");

int64_t dcqo_block_size(int type) {
    switch (type) {
        case DCQO_TYPE_F32: return 1;
        case DCQO_TYPE_F16: return 1;
        case DCQO_TYPE_Q4_0:
        case DCQO_TYPE_Q8_0: return QK8_0;
        case DCQO_TYPE_Q4_K:
        case DCQO_TYPE_Q5_K:
        case DCQO_TYPE_Q6_K:
        case DCQO_TYPE_Q8_K: return QK_K;
        default: return 0;
    }
}

int64_t dcqo_type_size(int type) {
    switch (type) {
        case DCQO_TYPE_F32: return 4;
        case DCQO_TYPE_F16: return 2;
        case DCQO_TYPE_Q4_0: return (int64_t)sizeof(blk_q4_0);
        case DCQO_TYPE_Q8_0: return (int64_t)sizeof(blk_q8_0);
        case DCQO_TYPE_Q4_K: return (int64_t)sizeof(blk_q4_K);
        case DCQO_TYPE_Q5_K: return (int64_t)sizeof(blk_q5_K);
        case DCQO_TYPE_Q6_K: return (int64_t)sizeof(blk_q6_K);
        case DCQO_TYPE_Q8_K: return (int64_t)sizeof(blk_q8_K);
        default: return 0;
    }
}

int64_t dcqo_row_size(int type, int64_t k) {
    int64_t bs = dcqo_block_size(type);
    if (bs <= 0 || k % bs) return 0;
    return (k / bs) * dcqo_type_size(type);
}

/* core/include/simd_ops.h:3298-3305: Q4_K/Q5_K/Q6_K -> Q8_K, Q8_0 -> Q8_0; Q4_0 -> Q8_0 is
 * ggml's type trait for the Q4_0 the reference's quantize tool emits (core/src/quantize.cpp:71-72) */
int dcqo_vec_dot_type(int type) {
    switch (type) {
        case DCQO_TYPE_Q4_0:
        case DCQO_TYPE_Q8_0: return DCQO_TYPE_Q8_0;
        case DCQO_TYPE_Q4_K:
        case DCQO_TYPE_Q5_K:
        case DCQO_TYPE_Q6_K: return DCQO_TYPE_Q8_K;
        default: return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32. fp32->fp16 is IEEE round-to-nearest-even (what F16C        */
/* `vcvtps2ph imm=0` and ggml's generic bit-trick both produce).             */
/* Pinned by: numpy float16 conversion over random values and every tie.     */
/* ------------------------------------------------------------------------ */
static uint32_t rne_shr(uint32_t v, int s) {
    if (s <= 0) return v;
    if (s >= 32) return 0;
    uint32_t q = v >> s;
    uint32_t rem = v & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return q;
}

uint16_t dcqo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan (quiet the nan) */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    uint32_t e = ax >> 23;
    uint32_t mant = ax & 0x7fffffu;
    if (e >= 113) { /* fp16 normal range (or overflow via carry) */
        if (e >= 143) return sign | 0x7c00u;
        uint32_t v = ((e - 112u) << 23) | mant;
        uint32_t h = rne_shr(v, 13);
        if (h >= 0x7c00u) h = 0x7c00u;
        return sign | (uint16_t)h;
    }
    if (e == 0) return sign; /* fp32 subnormal: far below fp16 resolution */
    /* fp16 subnormal: value = M * 2^(e-150) = m16 * 2^-24 -> m16 = M >> (126-e) */
    uint32_t M = mant | 0x800000u;
    uint32_t h = rne_shr(M, (int)(126u - e));
    return sign | (uint16_t)h;
}

float dcqo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void dcqo_fp32_to_fp16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = dcqo_fp32_to_fp16(x[i]);
}
void dcqo_fp16_to_fp32_array(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = dcqo_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Activation quantizers (the `from_float` of the vec_dot_type).             */
/* ------------------------------------------------------------------------ */

/* ggml's nearest_int: add 1.5*2^23 and read the mantissa; for |v| < 2^22 this
 * is round-half-even of the (already rounded) fp32 argument. */
static int nearest_int(float v) {
    float t = v + 12582912.f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/*
 * Q8_0 from_float. Invoked at core/src/inference.cpp:891-892 through the type
 * traits; DCQO_Q8_0_X86 is the x86 SIMD semantics that a GGML_NATIVE x86 build
 * executes: amax over |x|, d = amax/127 (fp32 divide) stored as fp16 (RNE),
 * id = 127/amax (0 for amax == 0), q = round-half-even(x*id), saturated to int8.
 * DCQO_Q8_0_REF is quantize_row_q8_0_ref (also ggml_quantize_chunk's Q8_0,
 * core/src/kv_cache.cpp:572-579): id = 1/d, q = roundf(x*id).
 * Pins: zero block -> d = 0, q = 0; single non-zero -> q = +-127; exact .5
 * ties separate the two variants; |x - d*q| <= d/2 (plus fp16 rounding of d).
 */
void dcqo_quantize_row_q8_0(const float* x, void* vy, int64_t k, int variant) {
    blk_q8_0* y = (blk_q8_0*)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; ++i) {
        const float* xb = x + i * QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.f;
        y[i].d = dcqo_fp32_to_fp16(d);
        if (variant == DCQO_Q8_0_REF) {
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < QK8_0; ++j) {
                float v = roundf(xb[j] * id);
                if (v > 127.f) v = 127.f;
                if (v < -128.f) v = -128.f;
                y[i].qs[j] = (int8_t)v;
            }
        } else {
            const float id = amax != 0.0f ? 127.f / amax : 0.0f;
            for (int j = 0; j < QK8_0; ++j) {
                float v = rintf(xb[j] * id);
                if (v > 127.f) v = 127.f;
                if (v < -128.f) v = -128.f;
                y[i].qs[j] = (int8_t)v;
            }
        }
    }
}

/*
 * Q8_K from_float (quantize_row_q8_K_ref; x86 has no SIMD variant). Per
 * 256-block: `max` is the first element of largest |x| (strict >, so the
 * earliest wins a tie); iscale = -127/max; q = min(127, nearest_int(iscale*x));
 * bsums[g] = sum of q[16g .. 16g+15]; d = 1/iscale (fp32, may be negative).
 * An all-zero block gives d = 0 and q = 0; ggml leaves its bsums unwritten,
 * this restatement (and the GPU) writes 0, the value sum(q) defines.
 * Pins: extreme maps to -127; bsums invariant; |x - d*q| <= |d|/2.
 */
void dcqo_quantize_row_q8_K(const float* x, void* vy, int64_t k) {
    blk_q8_K* y = (blk_q8_K*)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float* xb = x + i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; ++j) {
            float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(blk_q8_K));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) {
            int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < QK_K / 16; ++g) {
            int s = 0;
            for (int t = 0; t < 16; ++t) s += y[i].qs[16 * g + t];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void dcqo_quantize_rows(int vdt, const float* x, int64_t m, int64_t k, int64_t x_stride, void* y,
                        int variant) {
    const int64_t rs = dcqo_row_size(vdt, k);
    for (int64_t r = 0; r < m; ++r) {
        char* yr = (char*)y + r * rs;
        if (vdt == DCQO_TYPE_Q8_0)
            dcqo_quantize_row_q8_0(x + r * x_stride, yr, k, variant);
        else if (vdt == DCQO_TYPE_Q8_K)
            dcqo_quantize_row_q8_K(x + r * x_stride, yr, k);
    }
}

/* ------------------------------------------------------------------------ */
/* Weight quantizers (ggml_quantize_chunk equivalents; core/src/quantize.cpp */
/* :214,285 calls them). Only used to generate synthetic weights: both the   */
/* GPU and the oracle then consume the same bytes, so their byte-exactness   */
/* against ggml does not enter mul_mat parity (parity unpinned).             */
/* ------------------------------------------------------------------------ */
#define GROUP_MAX_EPS 1e-15f

void dcqo_quantize_row_q8_0_weights(const float* x, void* y, int64_t k) {
    dcqo_quantize_row_q8_0(x, y, k, DCQO_Q8_0_REF);
}

/* quantize_row_q4_0_ref: max = the first element of largest |x| (strict '<' scan), d = max / -8,
 * id = 1/d (0 for an all-zero block), q = min(15, (int8)(x*id + 8.5)) truncated toward zero; the
 * element of largest magnitude maps to 0, i.e. to -8 once the 8 is taken off. */
void dcqo_quantize_row_q4_0(const float* x, void* vy, int64_t k) {
    blk_q4_0* y = (blk_q4_0*)vy;
    for (int64_t i = 0; i < k / QK8_0; ++i) {
        const float* xb = x + i * QK8_0;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK8_0; ++j) {
            if (amax < fabsf(xb[j])) {
                amax = fabsf(xb[j]);
                max = xb[j];
            }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = dcqo_fp32_to_fp16(d);
        for (int j = 0; j < QK8_0 / 2; ++j) {
            const float x0 = xb[j] * id, x1 = xb[QK8_0 / 2 + j] * id;
            const int q0 = (int)(int8_t)(x0 + 8.5f), q1 = (int)(int8_t)(x1 + 8.5f);
            y[i].qs[j] = (uint8_t)((q0 < 15 ? q0 : 15) | ((q1 < 15 ? q1 : 15) << 4));
        }
    }
}

/* weighted least-squares fit of x ~ scale*L + min, L in [0,nmax], min <= 0: the best of the
 * rounding at iscale = nmax/(max-min) and the nstep+1 grid points iscale = (rmin + rdelta*is +
 * nmax)/(max-min), each refitted by weighted least squares (min clamped to <= 0).
 * flags (test hooks only, 0 in the quantizers): DCQO_PLANT_NO_MIN_CLAMP drops the clamp of the
 * refitted min. */
static float make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L,
                              float* the_min, uint8_t* Laux, float rmin, float rdelta, int nstep, int flags) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : (l > nmax ? nmax : l));
        float diff = scale * L[i] + min - x[i];
        best_error += weights[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0 && !(flags & DCQO_PLANT_NO_MIN_CLAMP)) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                mad += weights[i] * (diff * diff);
            }
            if (mad < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* the 12-byte packing of eight 6-bit (scale, min) pairs that get_scale_min_k4 reads back:
 * j < 4 in the low 6 bits of bytes j and j+4; j >= 4 as nibbles of byte j+4, with their top two
 * bits in the high bits of bytes j-4 (scale) and j (min) */
void dcqo_pack_scale_min_k4(const uint8_t ls[8], const uint8_t lm[8], uint8_t s[12]) {
    memset(s, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            s[j] = ls[j];
            s[j + 4] = lm[j];
        } else {
            s[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            s[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            s[j - 0] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
}

static void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* One superblock of quantize_row_q4_K_ref / quantize_row_q5_K_ref: a make_qkx2_quants fit per
 * 32-element sub-block (weights av_x + |x_i|; nmax 15, rmin -1, nstep 20 for Q4_K; nmax 31,
 * rmin -0.5, nstep 15 for Q5_K; rdelta 0.1), the fits' scales and mins as 6-bit multiples of
 * d = max scale / 63 and dmin = max min / 63, then every element re-rounded against its stored
 * scale and min: L = clamp(nearest_int((x + dmin*m) / (d*sc)), 0, nmax). A sub-block whose stored
 * scale is 0 keeps its fit's own levels. */
static void kquant_superblock(const float* x, int nmax, float rmin, int nstep, uint8_t L[QK_K],
                              uint8_t scales[12], uint16_t* dh, uint16_t* dminh) {
    uint8_t Laux[32];
    float weights[32], mins[QK_K / 32], sc_f[QK_K / 32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < QK_K / 32; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        sc_f[j] = make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, rmin, 0.1f,
                                   nstep, 0);
        if (sc_f[j] > max_scale) max_scale = sc_f[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t ls[QK_K / 32], lm[QK_K / 32];
    for (int j = 0; j < QK_K / 32; ++j) {
        const int a = nearest_int(inv_scale * sc_f[j]);
        const int b = nearest_int(inv_min * mins[j]);
        ls[j] = (uint8_t)(a < 63 ? a : 63);
        lm[j] = (uint8_t)(b < 63 ? b : 63);
    }
    dcqo_pack_scale_min_k4(ls, lm, scales);
    *dh = dcqo_fp32_to_fp16(max_scale / 63.f);
    *dminh = dcqo_fp32_to_fp16(max_min / 63.f);
    for (int j = 0; j < QK_K / 32; ++j) {
        uint8_t sc, m;
        get_scale_min_k4(j, scales, &sc, &m);
        const float d = dcqo_fp16_to_fp32(*dh) * sc;
        if (!d) continue;
        const float dm = dcqo_fp16_to_fp32(*dminh) * m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > nmax ? nmax : l));
        }
    }
}

void dcqo_quantize_row_q4_K(const float* x, void* vy, int64_t k) {
    blk_q4_K* y = (blk_q4_K*)vy;
    uint8_t L[QK_K];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        kquant_superblock(x, 15, -1.f, 20, L, y[i].scales, &y[i].d, &y[i].dmin);
        /* sub-block 2c in the low nibbles of qs[32c .. 32c+31], sub-block 2c+1 in the high ones */
        uint8_t* q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

void dcqo_quantize_row_q5_K(const float* x, void* vy, int64_t k) {
    blk_q5_K* y = (blk_q5_K*)vy;
    uint8_t L[QK_K];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        kquant_superblock(x, 31, -0.5f, 15, L, y[i].scales, &y[i].d, &y[i].dmin);
        /* the low four bits packed as Q4_K's nibbles; bit 4 of element l of sub-block j in bit j of
         * qh[l] */
        memset(y[i].qh, 0, sizeof(y[i].qh));
        uint8_t* q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) {
                const int l1 = L[j + l], l2 = L[j + l + 32];
                q[l] = (uint8_t)((l1 & 0xF) | ((l2 & 0xF) << 4));
                y[i].qh[l] |= (uint8_t)(((l1 >> 4) << (j / 32)) | ((l2 >> 4) << (j / 32 + 1)));
            }
            q += 32;
        }
        x += QK_K;
    }
}

/* least-squares symmetric fit, L in [-nmax, nmax-1] stored offset by nmax: the best, by the
 * x^2-weighted fit quality (sum w x l)^2 / sum w l^2, of the rounding at iscale = -nmax/max and at
 * iscale = -(nmax + 0.1*is)/max for is in [-9, 9], is != 0.
 * flags (test hooks only, 0 in the quantizer): DCQO_PLANT_UNIT_WEIGHTS weighs every element 1,
 * DCQO_PLANT_GRID_8 searches is in [-8, 8] only. */
static float make_qx_quants(int n, int nmax, const float* x, int8_t* L, int flags) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        float w = (flags & DCQO_PLANT_UNIT_WEIGHTS) ? 1.0f : x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    const int grid = (flags & DCQO_PLANT_GRID_8) ? 8 : 9;
    for (int is = -grid; is <= grid; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            float w = (flags & DCQO_PLANT_UNIT_WEIGHTS) ? 1.0f : x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(l + nmax);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

void dcqo_quantize_row_q6_K(const float* x, void* vy, int64_t k) {
    blk_q6_K* y = (blk_q6_K*)vy;
    const int64_t nb = k / QK_K;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < nb; ++i) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 0);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(blk_q6_K));
            x += QK_K;
            continue;
        }
        float iscale = -128.f / max_scale;
        y[i].d = dcqo_fp32_to_fp16(1 / iscale);
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            int v = nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            float d = dcqo_fp16_to_fp32(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t* ql = y[i].ql;
        uint8_t* qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                  ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

/* ---- test hooks: the quantizers' inner fits, for the optimality checks of the tests ---- */
float dcqo_make_qkx2_quants(int n, int nmax, const float* x, const float* weights, uint8_t* L, float* the_min,
                            float rmin, float rdelta, int nstep, int flags) {
    uint8_t Laux[256];
    if (n <= 0 || n > 256) return 0.0f;
    return make_qkx2_quants(n, nmax, x, weights, L, the_min, Laux, rmin, rdelta, nstep, flags);
}

float dcqo_make_qx_quants(int n, int nmax, const float* x, int8_t* L, int flags) {
    return make_qx_quants(n, nmax, x, L, flags);
}

/* ---- threaded matrix quantization (pure data-parallel over rows) ---- */
typedef struct {
    int type;
    const float* x;
    int64_t k;
    void* y;
    int64_t r0, r1;
} qm_job;

static void* qm_worker(void* p) {
    qm_job* j = (qm_job*)p;
    const int64_t rs = dcqo_row_size(j->type, j->k);
    for (int64_t r = j->r0; r < j->r1; ++r) {
        const float* xr = j->x + r * j->k;
        void* yr = (char*)j->y + r * rs;
        if (j->type == DCQO_TYPE_Q8_0)
            dcqo_quantize_row_q8_0_weights(xr, yr, j->k);
        else if (j->type == DCQO_TYPE_Q4_0)
            dcqo_quantize_row_q4_0(xr, yr, j->k);
        else if (j->type == DCQO_TYPE_Q4_K)
            dcqo_quantize_row_q4_K(xr, yr, j->k);
        else if (j->type == DCQO_TYPE_Q5_K)
            dcqo_quantize_row_q5_K(xr, yr, j->k);
        else if (j->type == DCQO_TYPE_Q6_K)
            dcqo_quantize_row_q6_K(xr, yr, j->k);
    }
    return NULL;
}

static int auto_threads(int nthreads) {
    if (nthreads > 0) return nthreads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > 64) n = 64;
    return (int)n;
}

int dcqo_quantize_matrix(int type, const float* x, int64_t n, int64_t k, void* y, int nthreads) {
    if (type != DCQO_TYPE_Q8_0 && type != DCQO_TYPE_Q4_0 && type != DCQO_TYPE_Q4_K && type != DCQO_TYPE_Q5_K &&
        type != DCQO_TYPE_Q6_K)
        return -1;
    if (dcqo_row_size(type, k) <= 0) return -2;
    int nt = auto_threads(nthreads);
    if (nt > n) nt = (int)(n > 0 ? n : 1);
    pthread_t th[64];
    qm_job jobs[64];
    int64_t per = (n + nt - 1) / nt;
    for (int t = 0; t < nt; ++t) {
        jobs[t] = (qm_job){type, x, k, y, t * per, (t + 1) * per < n ? (t + 1) * per : n};
        pthread_create(&th[t], NULL, qm_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; ++t) pthread_join(th[t], NULL);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dequantization (ggml to_float semantics).                                 */
/* ------------------------------------------------------------------------ */

/* element e (0..255) of a Q4_K superblock: 4-bit quant and its sub-block */
static int q4k_quant(const blk_q4_K* b, int e) {
    int c = e / 64, w = e % 64, l = w % 32;
    uint8_t byte = b->qs[32 * c + l];
    return (w >= 32) ? (byte >> 4) : (byte & 0xF);
}
/* element e (0..255) of a Q5_K superblock: the 4-bit part as Q4_K's, plus 16 * bit (e/32) of
 * qh[e % 32] */
static int q5k_quant(const blk_q5_K* b, int e) {
    int c = e / 64, w = e % 64, l = w % 32;
    uint8_t byte = b->qs[32 * c + l];
    int lo = (w >= 32) ? (byte >> 4) : (byte & 0xF);
    return lo + 16 * ((b->qh[l] >> (e / 32)) & 1);
}
/* element j (0..31) of a Q4_0 block: unsigned 4-bit quant q (the value is d * (q - 8)) */
static int q4_0_quant(const blk_q4_0* b, int j) {
    return j < 16 ? (b->qs[j] & 0xF) : (b->qs[j - 16] >> 4);
}
/* element e of a Q6_K superblock: signed 6-bit quant q - 32 */
static int q6k_quant(const blk_q6_K* b, int e) {
    int h = e / 128, ep = e % 128, t = ep / 32, l = ep % 32;
    int lo = (b->ql[64 * h + l + 32 * (t & 1)] >> (4 * (t >> 1))) & 0xF;
    int hi = (b->qh[32 * h + l] >> (2 * t)) & 3;
    return (lo | (hi << 4)) - 32;
}

int dcqo_dequantize_row(int type, const void* vx, float* y, int64_t k) {
    if (dcqo_row_size(type, k) <= 0) return -1;
    if (type == DCQO_TYPE_Q8_0) {
        const blk_q8_0* x = (const blk_q8_0*)vx;
        for (int64_t i = 0; i < k / QK8_0; ++i) {
            float d = dcqo_fp16_to_fp32(x[i].d);
            for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = x[i].qs[j] * d;
        }
    } else if (type == DCQO_TYPE_Q4_0) {
        /* dequantize_row_q4_0: (q - 8) * d */
        const blk_q4_0* x = (const blk_q4_0*)vx;
        for (int64_t i = 0; i < k / QK8_0; ++i) {
            float d = dcqo_fp16_to_fp32(x[i].d);
            for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = (q4_0_quant(&x[i], j) - 8) * d;
        }
    } else if (type == DCQO_TYPE_Q4_K) {
        const blk_q4_K* x = (const blk_q4_K*)vx;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            float d = dcqo_fp16_to_fp32(x[i].d), dmin = dcqo_fp16_to_fp32(x[i].dmin);
            for (int e = 0; e < QK_K; ++e) {
                uint8_t sc, m;
                get_scale_min_k4(e / 32, x[i].scales, &sc, &m);
                y[i * QK_K + e] = d * sc * q4k_quant(&x[i], e) - dmin * m;
            }
        }
    } else if (type == DCQO_TYPE_Q5_K) {
        /* dequantize_row_q5_K: (d * sc) * q - dmin * m, q in [0, 31] */
        const blk_q5_K* x = (const blk_q5_K*)vx;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            float d = dcqo_fp16_to_fp32(x[i].d), dmin = dcqo_fp16_to_fp32(x[i].dmin);
            for (int e = 0; e < QK_K; ++e) {
                uint8_t sc, m;
                get_scale_min_k4(e / 32, x[i].scales, &sc, &m);
                y[i * QK_K + e] = d * sc * q5k_quant(&x[i], e) - dmin * m;
            }
        }
    } else if (type == DCQO_TYPE_Q6_K) {
        const blk_q6_K* x = (const blk_q6_K*)vx;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            float d = dcqo_fp16_to_fp32(x[i].d);
            for (int e = 0; e < QK_K; ++e) y[i * QK_K + e] = d * x[i].scales[e / 16] * q6k_quant(&x[i], e);
        }
    } else if (type == DCQO_TYPE_Q8_K) {
        const blk_q8_K* x = (const blk_q8_K*)vx;
        for (int64_t i = 0; i < k / QK_K; ++i)
            for (int e = 0; e < QK_K; ++e) y[i * QK_K + e] = x[i].d * x[i].qs[e];
    } else {
        return -1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* vec_dot in ggml's generic (scalar) order.                                 */
/* ------------------------------------------------------------------------ */
static float vec_dot_q8_0_q8_0(int64_t n, const blk_q8_0* x, const blk_q8_0* y) {
    float sumf = 0;
    for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
        int sumi = 0;
        for (int j = 0; j < QK8_0; ++j) sumi += x[ib].qs[j] * y[ib].qs[j];
        sumf += sumi * (dcqo_fp16_to_fp32(x[ib].d) * dcqo_fp16_to_fp32(y[ib].d));
    }
    return sumf;
}

/* vec_dot_q4_0_q8_0 (generic): per block the integer sum of (q - 8) * q8 over both halves, then
 * sumf += (sumi * dx) * dy, the products in that order */
static float vec_dot_q4_0_q8_0(int64_t n, const blk_q4_0* x, const blk_q8_0* y) {
    float sumf = 0;
    for (int64_t ib = 0; ib < n / QK8_0; ++ib) {
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < QK8_0 / 2; ++j) {
            sumi0 += ((x[ib].qs[j] & 0x0F) - 8) * y[ib].qs[j];
            sumi1 += ((x[ib].qs[j] >> 4) - 8) * y[ib].qs[j + QK8_0 / 2];
        }
        const int sumi = sumi0 + sumi1;
        sumf += sumi * dcqo_fp16_to_fp32(x[ib].d) * dcqo_fp16_to_fp32(y[ib].d);
    }
    return sumf;
}

/* integer parts of one Q4_K (qh == NULL) or Q5_K x Q8_K superblock, as the generic kernels form
 * them: aux32[8] lanes of sum sc_j*q*q8 and the mins sum over bsums. q is the nibble, plus 16
 * where bit j of qh[l] is set for element l of sub-block j (Q5_K). */
static void kq_superblock_ints(const uint8_t* qs, const uint8_t* qh, const uint8_t* scales,
                               const blk_q8_K* y, int32_t aux32[8], int32_t* mins_sum) {
    int8_t a[QK_K];
    const uint8_t* q4 = qs;
    int8_t* p = a;
    uint8_t mbit = 1;
    for (int j = 0; j < QK_K / 64; ++j) {
        for (int l = 0; l < 32; ++l) p[l] = (int8_t)((q4[l] & 0xF) + (qh && (qh[l] & mbit) ? 16 : 0));
        p += 32;
        mbit <<= 1;
        for (int l = 0; l < 32; ++l) p[l] = (int8_t)((q4[l] >> 4) + (qh && (qh[l] & mbit) ? 16 : 0));
        p += 32;
        mbit <<= 1;
        q4 += 32;
    }
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) get_scale_min_k4(j, scales, &sc[j], &mn[j]);
    int32_t sumi = 0;
    for (int j = 0; j < QK_K / 16; ++j) sumi += y->bsums[j] * mn[j / 2];
    *mins_sum = sumi;
    for (int l = 0; l < 8; ++l) aux32[l] = 0;
    const int8_t* q8 = y->qs;
    p = a;
    for (int j = 0; j < QK_K / 32; ++j) {
        int32_t scale = sc[j];
        for (int g = 0; g < 4; ++g) {
            for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * p[l]);
            q8 += 8;
            p += 8;
        }
    }
}

static void q4k_superblock_ints(const blk_q4_K* x, const blk_q8_K* y, int32_t aux32[8], int32_t* mins_sum) {
    kq_superblock_ints(x->qs, NULL, x->scales, y, aux32, mins_sum);
}
static void q5k_superblock_ints(const blk_q5_K* x, const blk_q8_K* y, int32_t aux32[8], int32_t* mins_sum) {
    kq_superblock_ints(x->qs, x->qh, x->scales, y, aux32, mins_sum);
}

/* vec_dot_q4_K_q8_K and vec_dot_q5_K_q8_K (generic): the same float steps over their integer
 * parts (the 4-byte d/dmin header sits at the start of both blocks) */
static float vec_dot_kq_q8_K(int wtype, int64_t n, const void* vx, const blk_q8_K* y) {
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t i = 0; i < n / QK_K; ++i) {
        int32_t aux32[8], mins_sum;
        uint16_t xd, xdmin;
        if (wtype == DCQO_TYPE_Q5_K) {
            const blk_q5_K* x = (const blk_q5_K*)vx + i;
            q5k_superblock_ints(x, &y[i], aux32, &mins_sum);
            xd = x->d, xdmin = x->dmin;
        } else {
            const blk_q4_K* x = (const blk_q4_K*)vx + i;
            q4k_superblock_ints(x, &y[i], aux32, &mins_sum);
            xd = x->d, xdmin = x->dmin;
        }
        const float d = dcqo_fp16_to_fp32(xd) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = dcqo_fp16_to_fp32(xdmin) * y[i].d;
        sumf -= dmin * mins_sum;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static void q6k_superblock_ints(const blk_q6_K* x, const blk_q8_K* y, int32_t aux32[8]) {
    int8_t a[QK_K];
    const uint8_t* q4 = x->ql;
    const uint8_t* qh = x->qh;
    int8_t* p = a;
    for (int j = 0; j < QK_K; j += 128) {
        for (int l = 0; l < 32; ++l) {
            p[l + 0] = (int8_t)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            p[l + 32] = (int8_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            p[l + 64] = (int8_t)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            p[l + 96] = (int8_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        }
        p += 128;
        q4 += 64;
        qh += 32;
    }
    for (int l = 0; l < 8; ++l) aux32[l] = 0;
    const int8_t* q8 = y->qs;
    p = a;
    for (int j = 0; j < QK_K / 16; ++j) {
        int scale = x->scales[j];
        for (int g = 0; g < 2; ++g) {
            for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * p[l]);
            q8 += 8;
            p += 8;
        }
    }
}

static float vec_dot_q6_K_q8_K(int64_t n, const blk_q6_K* x, const blk_q8_K* y) {
    float sums[8] = {0};
    for (int64_t i = 0; i < n / QK_K; ++i) {
        int32_t aux32[8];
        q6k_superblock_ints(&x[i], &y[i], aux32);
        const float d = dcqo_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

float dcqo_vec_dot(int wtype, int64_t k, const void* w, const void* xq) {
    switch (wtype) {
        case DCQO_TYPE_Q8_0: return vec_dot_q8_0_q8_0(k, (const blk_q8_0*)w, (const blk_q8_0*)xq);
        case DCQO_TYPE_Q4_0: return vec_dot_q4_0_q8_0(k, (const blk_q4_0*)w, (const blk_q8_0*)xq);
        case DCQO_TYPE_Q4_K:
        case DCQO_TYPE_Q5_K: return vec_dot_kq_q8_K(wtype, k, w, (const blk_q8_K*)xq);
        case DCQO_TYPE_Q6_K: return vec_dot_q6_K_q8_K(k, (const blk_q6_K*)w, (const blk_q8_K*)xq);
        default: return 0.0f;
    }
}

int64_t dcqo_block_sums_per_row(int wtype, int64_t k) {
    switch (wtype) {
        case DCQO_TYPE_Q4_0:
        case DCQO_TYPE_Q8_0: return k / QK8_0;
        case DCQO_TYPE_Q4_K:
        case DCQO_TYPE_Q5_K: return 2 * (k / QK_K);
        case DCQO_TYPE_Q6_K: return k / QK_K;
        default: return 0;
    }
}

int dcqo_block_sums(int wtype, int64_t k, const void* w, const void* xq, int32_t* out) {
    if (dcqo_row_size(wtype, k) <= 0) return -1;
    if (wtype == DCQO_TYPE_Q8_0) {
        const blk_q8_0* x = (const blk_q8_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t ib = 0; ib < k / QK8_0; ++ib) {
            int s = 0;
            for (int j = 0; j < QK8_0; ++j) s += x[ib].qs[j] * y[ib].qs[j];
            out[ib] = s;
        }
    } else if (wtype == DCQO_TYPE_Q4_0) {
        const blk_q4_0* x = (const blk_q4_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t ib = 0; ib < k / QK8_0; ++ib) {
            int s = 0;
            for (int j = 0; j < QK8_0 / 2; ++j)
                s += ((x[ib].qs[j] & 0x0F) - 8) * y[ib].qs[j] + ((x[ib].qs[j] >> 4) - 8) * y[ib].qs[j + 16];
            out[ib] = s;
        }
    } else if (wtype == DCQO_TYPE_Q4_K || wtype == DCQO_TYPE_Q5_K) {
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            int32_t aux32[8], mins_sum, s = 0;
            if (wtype == DCQO_TYPE_Q5_K)
                q5k_superblock_ints((const blk_q5_K*)w + i, &y[i], aux32, &mins_sum);
            else
                q4k_superblock_ints((const blk_q4_K*)w + i, &y[i], aux32, &mins_sum);
            for (int l = 0; l < 8; ++l) s += aux32[l];
            out[2 * i] = s;
            out[2 * i + 1] = mins_sum;
        }
    } else if (wtype == DCQO_TYPE_Q6_K) {
        const blk_q6_K* x = (const blk_q6_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            int32_t aux32[8], s = 0;
            q6k_superblock_ints(&x[i], &y[i], aux32);
            for (int l = 0; l < 8; ++l) s += aux32[l];
            out[i] = s;
        }
    } else {
        return -1;
    }
    return 0;
}

/* First principles: element-wise integer products, int64, no bsums, no
 * unpacking loops shared with the functions above. */
int dcqo_block_sums_bruteforce(int wtype, int64_t k, const void* w, const void* xq, int64_t* out) {
    if (dcqo_row_size(wtype, k) <= 0) return -1;
    if (wtype == DCQO_TYPE_Q8_0) {
        const blk_q8_0* x = (const blk_q8_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t e0 = 0; e0 < k; e0 += QK8_0) {
            int64_t s = 0;
            for (int64_t e = e0; e < e0 + QK8_0; ++e)
                s += (int64_t)x[e / QK8_0].qs[e % QK8_0] * y[e / QK8_0].qs[e % QK8_0];
            out[e0 / QK8_0] = s;
        }
    } else if (wtype == DCQO_TYPE_Q4_0) {
        const blk_q4_0* x = (const blk_q4_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t e0 = 0; e0 < k; e0 += QK8_0) {
            int64_t s = 0;
            for (int64_t e = e0; e < e0 + QK8_0; ++e)
                s += (int64_t)(q4_0_quant(&x[e / QK8_0], (int)(e % QK8_0)) - 8) * y[e / QK8_0].qs[e % QK8_0];
            out[e0 / QK8_0] = s;
        }
    } else if (wtype == DCQO_TYPE_Q4_K || wtype == DCQO_TYPE_Q5_K) {
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            const blk_q4_K* x4 = (const blk_q4_K*)w + i;
            const blk_q5_K* x5 = (const blk_q5_K*)w + i;
            const uint8_t* scales = wtype == DCQO_TYPE_Q5_K ? x5->scales : x4->scales;
            int64_t a = 0, b = 0;
            for (int e = 0; e < QK_K; ++e) {
                uint8_t sc, m;
                get_scale_min_k4(e / 32, scales, &sc, &m);
                const int q = wtype == DCQO_TYPE_Q5_K ? q5k_quant(x5, e) : q4k_quant(x4, e);
                a += (int64_t)sc * q * y[i].qs[e];
                b += (int64_t)m * y[i].qs[e];
            }
            out[2 * i] = a;
            out[2 * i + 1] = b;
        }
    } else if (wtype == DCQO_TYPE_Q6_K) {
        const blk_q6_K* x = (const blk_q6_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t i = 0; i < k / QK_K; ++i) {
            int64_t a = 0;
            for (int e = 0; e < QK_K; ++e)
                a += (int64_t)x[i].scales[e / 16] * q6k_quant(&x[i], e) * y[i].qs[e];
            out[i] = a;
        }
    } else {
        return -1;
    }
    return 0;
}

double dcqo_vec_dot_f64(int wtype, int64_t k, const void* w, const void* xq) {
    double s = 0.0;
    if (wtype == DCQO_TYPE_Q8_0) {
        const blk_q8_0* x = (const blk_q8_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t e = 0; e < k; ++e) {
            double wv = (double)dcqo_fp16_to_fp32(x[e / 32].d) * x[e / 32].qs[e % 32];
            double av = (double)dcqo_fp16_to_fp32(y[e / 32].d) * y[e / 32].qs[e % 32];
            s += wv * av;
        }
    } else if (wtype == DCQO_TYPE_Q4_0) {
        const blk_q4_0* x = (const blk_q4_0*)w;
        const blk_q8_0* y = (const blk_q8_0*)xq;
        for (int64_t e = 0; e < k; ++e) {
            double wv = (double)dcqo_fp16_to_fp32(x[e / 32].d) * (q4_0_quant(&x[e / 32], (int)(e % 32)) - 8);
            double av = (double)dcqo_fp16_to_fp32(y[e / 32].d) * y[e / 32].qs[e % 32];
            s += wv * av;
        }
    } else if (wtype == DCQO_TYPE_Q4_K) {
        const blk_q4_K* x = (const blk_q4_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t e = 0; e < k; ++e) {
            const blk_q4_K* b = &x[e / QK_K];
            uint8_t sc, m;
            get_scale_min_k4((int)(e % QK_K) / 32, b->scales, &sc, &m);
            double wv = (double)dcqo_fp16_to_fp32(b->d) * sc * q4k_quant(b, (int)(e % QK_K)) -
                        (double)dcqo_fp16_to_fp32(b->dmin) * m;
            double av = (double)y[e / QK_K].d * y[e / QK_K].qs[e % QK_K];
            s += wv * av;
        }
    } else if (wtype == DCQO_TYPE_Q5_K) {
        const blk_q5_K* x = (const blk_q5_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t e = 0; e < k; ++e) {
            const blk_q5_K* b = &x[e / QK_K];
            uint8_t sc, m;
            get_scale_min_k4((int)(e % QK_K) / 32, b->scales, &sc, &m);
            double wv = (double)dcqo_fp16_to_fp32(b->d) * sc * q5k_quant(b, (int)(e % QK_K)) -
                        (double)dcqo_fp16_to_fp32(b->dmin) * m;
            double av = (double)y[e / QK_K].d * y[e / QK_K].qs[e % QK_K];
            s += wv * av;
        }
    } else if (wtype == DCQO_TYPE_Q6_K) {
        const blk_q6_K* x = (const blk_q6_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t e = 0; e < k; ++e) {
            const blk_q6_K* b = &x[e / QK_K];
            double wv = (double)dcqo_fp16_to_fp32(b->d) * b->scales[(e % QK_K) / 16] *
                        q6k_quant(b, (int)(e % QK_K));
            double av = (double)y[e / QK_K].d * y[e / QK_K].qs[e % QK_K];
            s += wv * av;
        }
    }
    return s;
}

double dcqo_vec_dot_l1(int wtype, int64_t k, const void* w, const void* xq) {
    double s = 0.0;
    if (wtype == DCQO_TYPE_Q8_0 || wtype == DCQO_TYPE_Q4_0) {
        /* the block terms dW * dA * I_b (the 2-byte fp16 d opens both block layouts) */
        const size_t wbs = wtype == DCQO_TYPE_Q8_0 ? sizeof(blk_q8_0) : sizeof(blk_q4_0);
        const blk_q8_0* y = (const blk_q8_0*)xq;
        int32_t* ib = (int32_t*)malloc(sizeof(int32_t) * (size_t)(k / 32));
        dcqo_block_sums(wtype, k, w, xq, ib);
        for (int64_t b = 0; b < k / 32; ++b) {
            uint16_t dw;
            memcpy(&dw, (const char*)w + b * wbs, 2);
            s += fabs((double)dcqo_fp16_to_fp32(dw) * dcqo_fp16_to_fp32(y[b].d) * ib[b]);
        }
        free(ib);
    } else if (wtype == DCQO_TYPE_Q4_K || wtype == DCQO_TYPE_Q5_K) {
        /* the terms vec_dot_q4_K_q8_K / vec_dot_q5_K_q8_K add in fp32: the eight lane sums
         * d * aux32[l] of each superblock (they can cancel to a much smaller superblock total)
         * and the mins term */
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t b = 0; b < k / QK_K; ++b) {
            int32_t aux32[8], mins_sum;
            uint16_t xd, xdmin;
            if (wtype == DCQO_TYPE_Q5_K) {
                const blk_q5_K* x = (const blk_q5_K*)w + b;
                q5k_superblock_ints(x, &y[b], aux32, &mins_sum);
                xd = x->d, xdmin = x->dmin;
            } else {
                const blk_q4_K* x = (const blk_q4_K*)w + b;
                q4k_superblock_ints(x, &y[b], aux32, &mins_sum);
                xd = x->d, xdmin = x->dmin;
            }
            const double d = (double)dcqo_fp16_to_fp32(xd) * y[b].d;
            for (int l = 0; l < 8; ++l) s += fabs(d * aux32[l]);
            s += fabs((double)dcqo_fp16_to_fp32(xdmin) * y[b].d * mins_sum);
        }
    } else if (wtype == DCQO_TYPE_Q6_K) {
        /* the eight lane sums d * aux32[l] of each superblock, as vec_dot_q6_K_q8_K adds them */
        const blk_q6_K* x = (const blk_q6_K*)w;
        const blk_q8_K* y = (const blk_q8_K*)xq;
        for (int64_t b = 0; b < k / QK_K; ++b) {
            int32_t aux32[8];
            q6k_superblock_ints(&x[b], &y[b], aux32);
            const double d = (double)dcqo_fp16_to_fp32(x[b].d) * y[b].d;
            for (int l = 0; l < 8; ++l) s += fabs(d * aux32[l]);
        }
    }
    return s;
}

int dcqo_dot_rows(int wtype, const void* w, size_t row_stride, const void* xq, int64_t k, float* y,
                  int64_t n0, int64_t n1) {
    if (dcqo_vec_dot_type(wtype) < 0 || dcqo_row_size(wtype, k) <= 0) return -1;
    for (int64_t r = n0; r < n1; ++r) y[r - n0] = dcqo_vec_dot(wtype, k, (const char*)w + r * row_stride, xq);
    return 0;
}

/* ---- threaded mul_mat driver ---- */
typedef struct {
    int wtype;
    const void* w;
    int64_t k;
    size_t w_row_bytes;
    const void* xq;
    size_t xq_row_bytes;
    int64_t m;
    float* y;
    int64_t y_stride;
    float* l1;
    int64_t n0, n1;
} mm_job;

static void* mm_worker(void* p) {
    mm_job* j = (mm_job*)p;
    for (int64_t r = j->n0; r < j->n1; ++r) {
        const void* wr = (const char*)j->w + r * j->w_row_bytes;
        for (int64_t mi = 0; mi < j->m; ++mi) {
            const void* xr = (const char*)j->xq + mi * j->xq_row_bytes;
            j->y[mi * j->y_stride + r] = dcqo_vec_dot(j->wtype, j->k, wr, xr);
            if (j->l1) j->l1[mi * j->y_stride + r] = (float)dcqo_vec_dot_l1(j->wtype, j->k, wr, xr);
        }
    }
    return NULL;
}

int dcqo_mul_mat(int wtype, const void* w, int64_t n, int64_t k, size_t w_row_bytes, const float* x,
                 int64_t m, int64_t x_stride, float* y, int64_t y_stride, float* l1, int variant,
                 int nthreads) {
    const int vdt = dcqo_vec_dot_type(wtype);
    if (vdt < 0) return -1;
    const int64_t xrs = dcqo_row_size(vdt, k);
    if (xrs <= 0 || dcqo_row_size(wtype, k) <= 0) return -2;
    void* xq = malloc((size_t)(xrs * (m > 0 ? m : 1)));
    if (!xq) return -3;
    /* quantize all of X first, then the dots (race-free form of
     * core/src/inference.cpp:887-923) */
    dcqo_quantize_rows(vdt, x, m, k, x_stride, xq, variant);
    int nt = auto_threads(nthreads);
    if (nt > n) nt = (int)(n > 0 ? n : 1);
    pthread_t th[64];
    mm_job jobs[64];
    int64_t per = (n + nt - 1) / nt; /* row partition of core/src/inference.cpp:896-902 */
    for (int t = 0; t < nt; ++t) {
        int64_t a = t * per, b = (t + 1) * per < n ? (t + 1) * per : n;
        jobs[t] = (mm_job){wtype, w, k, w_row_bytes, xq, (size_t)xrs, m, y, y_stride, l1, a, b};
        pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; ++t) pthread_join(th[t], NULL);
    free(xq);
    return 0;
}
