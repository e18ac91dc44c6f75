/*
 * dcq_cpu_simd.c — the timed CPU baseline: a SIMD restatement of the reference CPU path.
 *
 * TEST / MEASUREMENT INFRASTRUCTURE ONLY. Loaded by tests/ (checked against the scalar oracle)
 * and by the cpu_baseline leg of bench.py. The product library never links or calls it.
 *
 * What is timed. The reference's quantized mul_mat runs in ggml's CPU backend (an un-vendored,
 * unpinned submodule, /root/reference/.gitmodules:1-3) built with GGML_NATIVE / -march=native
 * (core/CMakeLists.txt:101-103, 472-475), with one worker thread per physical core
 * (core/src/worker.cpp:63-77). ggml cannot be built here, so this file restates that path
 * ("CPU restatement (not ggml)"):
 *   - every X row is quantized once to the vec_dot_type (the oracle's x86 Q8_0 / Q8_K
 *     from_float), before any dot (the race-free form of core/src/inference.cpp:887-923);
 *   - then row-partitioned dots, one W row against one X row at a time
 *     (core/src/inference.cpp:896-923; ggml's x86 vec_dot with nrc = 1), tiled 16 W rows x
 *     64 X rows so a tile's operands stay in the core's caches;
 *   - int8 dot products with AVX2 (vpmaddubsw / vpmaddwd) or AVX-512 VNNI (vpdpbusd), chosen at
 *     run time by CPUID because this library is built here and run on the GPU box's host.
 * The per-block integer sums are the same exact integers as the scalar oracle's
 * (dcqo_block_sums); only the fp32 summation order differs (8 lanes, then a horizontal sum).
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dcq_oracle.h"

#define QK8_0 32
#define QK_K 256

typedef struct {
    uint16_t d;
    int8_t qs[QK8_0];
} sq8_0;
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[QK_K / 2];
} sq4_K;
typedef struct {
    uint8_t ql[QK_K / 2];
    uint8_t qh[QK_K / 4];
    int8_t scales[QK_K / 16];
    uint16_t d;
} sq6_K;
typedef struct {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
} sq8_K;

enum { ISA_SCALAR = 0, ISA_AVX2 = 1, ISA_AVX512VNNI = 2 };

int dcqs_isa(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("fma"))
        return ISA_AVX512VNNI;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return ISA_AVX2;
    return ISA_SCALAR;
}

/* the 6-bit scale and min of sub-block j of a Q4_K superblock (GGUF packing) */
static inline void q4k_scale_min(const uint8_t* s, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* ------------------------------------------------------------------ AVX2 */
__attribute__((target("avx2,fma"))) static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,fma"))) static inline int hsum8i(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* sum over 32 byte pairs of w*a, as 8 int32 lanes: |w| (u8) times a with w's sign (s8) */
__attribute__((target("avx2,fma"))) static inline __m256i dot32_avx2(__m256i w, __m256i a) {
    const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(a, w));
    return _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
}

__attribute__((target("avx2,fma"))) static float dot_q8_0_avx2(int64_t k, const sq8_0* x, const sq8_0* y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK8_0; ++b) {
        const __m256i w = _mm256_loadu_si256((const __m256i*)x[b].qs);
        const __m256i a = _mm256_loadu_si256((const __m256i*)y[b].qs);
        const float d = dcqo_fp16_to_fp32(x[b].d) * dcqo_fp16_to_fp32(y[b].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(dot32_avx2(w, a)), acc);
    }
    return hsum8(acc);
}

__attribute__((target("avx2,fma"))) static float dot_q4_K_avx2(int64_t k, const sq4_K* x, const sq8_K* y) {
    __m256 acc = _mm256_setzero_ps();
    float mins = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    for (int64_t i = 0; i < k / QK_K; ++i) {
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) q4k_scale_min(x[i].scales, j, &sc[j], &mn[j]);
        int msum = 0;
        for (int j = 0; j < 8; ++j) msum += mn[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; ++c) {
            const __m256i q = _mm256_loadu_si256((const __m256i*)(x[i].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            const __m256i a0 = _mm256_loadu_si256((const __m256i*)(y[i].qs + 64 * c));
            const __m256i a1 = _mm256_loadu_si256((const __m256i*)(y[i].qs + 64 * c + 32));
            const __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, a0), _mm256_set1_epi16((short)sc[2 * c]));
            const __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, a1), _mm256_set1_epi16((short)sc[2 * c + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
        }
        const float d = dcqo_fp16_to_fp32(x[i].d) * y[i].d;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        mins += dcqo_fp16_to_fp32(x[i].dmin) * y[i].d * (float)msum;
    }
    return hsum8(acc) - mins;
}

__attribute__((target("avx2,fma"))) static float dot_q6_K_avx2(int64_t k, const sq6_K* x, const sq8_K* y) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i m4 = _mm256_set1_epi8(0xF), m3 = _mm256_set1_epi8(3);
    for (int64_t i = 0; i < k / QK_K; ++i) {
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; ++h) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i*)(x[i].ql + 64 * h));
            const __m256i l1 = _mm256_loadu_si256((const __m256i*)(x[i].ql + 64 * h + 32));
            const __m256i qh = _mm256_loadu_si256((const __m256i*)(x[i].qh + 32 * h));
            for (int t = 0; t < 4; ++t) {
                const __m256i lsrc = (t & 1) ? l1 : l0;
                const __m256i lo = t < 2 ? _mm256_and_si256(lsrc, m4) : _mm256_and_si256(_mm256_srli_epi16(lsrc, 4), m4);
                const __m256i hb = _mm256_and_si256(_mm256_srli_epi16(qh, 2 * t), m3);
                const __m256i q6 = _mm256_or_si256(lo, _mm256_slli_epi16(hb, 4)); /* 0..63, bytes stay in range */
                const __m256i a = _mm256_loadu_si256((const __m256i*)(y[i].qs + 128 * h + 32 * t));
                const int g = 8 * h + 2 * t;
                const __m256i scv = _mm256_setr_m128i(_mm_set1_epi16(x[i].scales[g]), _mm_set1_epi16(x[i].scales[g + 1]));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(q6, a), scv));
            }
        }
        int corr = 0; /* the -32 offset of every 6-bit value, over the Q8_K group sums */
        for (int g = 0; g < 16; ++g) corr += x[i].scales[g] * y[i].bsums[g];
        const float d = dcqo_fp16_to_fp32(x[i].d) * y[i].d;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d),
                              _mm256_cvtepi32_ps(_mm256_sub_epi32(sumi, _mm256_setr_epi32(32 * corr, 0, 0, 0, 0, 0, 0, 0))),
                              acc);
    }
    return hsum8(acc);
}

/* ------------------------------------------------------------------ AVX-512 VNNI (256-bit VL) */
__attribute__((target("avx2,fma,avx512f,avx512vl,avx512bw,avx512vnni"))) static float dot_q8_0_vnni(
    int64_t k, const sq8_0* x, const sq8_0* y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK8_0; ++b) {
        const __m256i w = _mm256_loadu_si256((const __m256i*)x[b].qs);
        const __m256i a = _mm256_loadu_si256((const __m256i*)y[b].qs);
        const __m256i s = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_abs_epi8(w), _mm256_sign_epi8(a, w));
        const float d = dcqo_fp16_to_fp32(x[b].d) * dcqo_fp16_to_fp32(y[b].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum8(acc);
}

/* ------------------------------------------------------------------ dispatch + driver */
typedef float (*dot_fn)(int64_t, const void*, const void*);

static float scalar_dot(int wtype, int64_t k, const void* w, const void* a) { return dcqo_vec_dot(wtype, k, w, a); }

static float dot_one(int isa, int wtype, int64_t k, const void* w, const void* a) {
    if (isa == ISA_SCALAR) return scalar_dot(wtype, k, w, a);
    switch (wtype) {
        case DCQO_TYPE_Q8_0:
            return isa == ISA_AVX512VNNI ? dot_q8_0_vnni(k, (const sq8_0*)w, (const sq8_0*)a)
                                         : dot_q8_0_avx2(k, (const sq8_0*)w, (const sq8_0*)a);
        case DCQO_TYPE_Q4_K: return dot_q4_K_avx2(k, (const sq4_K*)w, (const sq8_K*)a);
        case DCQO_TYPE_Q6_K: return dot_q6_K_avx2(k, (const sq6_K*)w, (const sq8_K*)a);
        default: return 0.0f;
    }
}

float dcqs_vec_dot(int isa, int wtype, int64_t k, const void* w, const void* xq) {
    return dot_one(isa, wtype, k, w, xq);
}

/* Logical CPUs of this process's affinity mask, one per physical core (the first sibling of each
 * (package, core) pair, from sysfs topology). Returns the count written to cpus (<= max); *logical
 * receives the number of logical CPUs in the mask. */
int dcqs_physical_cpus(int* cpus, int max, int* logical) {
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof(set), &set) != 0) return -1;
    int seen_pkg[4096], seen_core[4096], nseen = 0, n = 0, nlog = 0;
    for (int c = 0; c < CPU_SETSIZE; ++c) {
        if (!CPU_ISSET(c, &set)) continue;
        ++nlog;
        int pkg = -1, core = -1;
        char path[128];
        FILE* f;
        snprintf(path, sizeof(path), "/sys/devices/system/cpu/cpu%d/topology/physical_package_id", c);
        if ((f = fopen(path, "r"))) {
            if (fscanf(f, "%d", &pkg) != 1) pkg = -1;
            fclose(f);
        }
        snprintf(path, sizeof(path), "/sys/devices/system/cpu/cpu%d/topology/core_id", c);
        if ((f = fopen(path, "r"))) {
            if (fscanf(f, "%d", &core) != 1) core = -1;
            fclose(f);
        }
        int dup = 0;
        if (pkg >= 0 && core >= 0)
            for (int i = 0; i < nseen; ++i)
                if (seen_pkg[i] == pkg && seen_core[i] == core) dup = 1;
        if (dup) continue;
        if (nseen < 4096) {
            seen_pkg[nseen] = pkg;
            seen_core[nseen] = core;
            ++nseen;
        }
        if (n < max) cpus[n] = c;
        ++n;
    }
    if (logical) *logical = nlog;
    return n < max ? n : max;
}

/* A persistent pool of pinned workers, as the reference keeps its worker threads for the life of
 * the engine (core/src/worker.cpp:63-77). A call runs in two phases separated by a barrier: each
 * worker quantizes its share of the X rows, then computes its share of the W rows. */
typedef struct {
    int isa, wtype, vdt;
    const char* w;
    int64_t k;
    size_t wrb;
    const float* x;
    int64_t x_stride;
    char* xq;
    size_t xrb;
    int64_t m, n;
    float* y;
    int64_t ys;
} simd_call;

static struct {
    int n, alive;
    int cpus[256];
    pthread_t th[256];
    pthread_barrier_t start, mid, done;
    simd_call call;
} pool;

static void worker_run(int t) {
    const simd_call* c = &pool.call;
    const int nt = pool.n;
    const int64_t mper = (c->m + nt - 1) / nt;
    const int64_t m0 = t * mper, m1 = (t + 1) * mper < c->m ? (t + 1) * mper : c->m;
    if (m0 < m1) dcqo_quantize_rows(c->vdt, c->x + m0 * c->x_stride, m1 - m0, c->k, c->x_stride, c->xq + m0 * c->xrb,
                                    DCQO_Q8_0_X86);
    pthread_barrier_wait(&pool.mid);
    const int64_t per = (c->n + nt - 1) / nt; /* row partition of core/src/inference.cpp:896-902 */
    const int64_t n0 = t * per, n1 = (t + 1) * per < c->n ? (t + 1) * per : c->n;
    const int64_t TN = 16, TM = 64;
    for (int64_t nb = n0; nb < n1; nb += TN) {
        const int64_t ne = nb + TN < n1 ? nb + TN : n1;
        for (int64_t mt = 0; mt < c->m; mt += TM) {
            const int64_t me = mt + TM < c->m ? mt + TM : c->m;
            for (int64_t mi = mt; mi < me; ++mi) {
                const char* a = c->xq + mi * c->xrb;
                for (int64_t r = nb; r < ne; ++r) c->y[mi * c->ys + r] = dot_one(c->isa, c->wtype, c->k, c->w + r * c->wrb, a);
            }
        }
    }
}

static void* pool_worker(void* p) {
    const int t = (int)(intptr_t)p;
    if (pool.cpus[t] >= 0) {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(pool.cpus[t], &set);
        pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
    }
    for (;;) {
        pthread_barrier_wait(&pool.start);
        if (!pool.alive) break;
        worker_run(t);
        pthread_barrier_wait(&pool.done);
    }
    return NULL;
}

static void pool_stop(void) {
    if (!pool.n) return;
    pool.alive = 0;
    pthread_barrier_wait(&pool.start);
    for (int t = 0; t < pool.n; ++t) pthread_join(pool.th[t], NULL);
    pthread_barrier_destroy(&pool.start);
    pthread_barrier_destroy(&pool.mid);
    pthread_barrier_destroy(&pool.done);
    pool.n = 0;
}

/* (Re)start the pool with nt workers pinned to cpus[0 .. nt) (NULL: unpinned). */
static int pool_start(int nt, const int* cpus) {
    int same = pool.n == nt;
    for (int t = 0; same && t < nt; ++t) same = pool.cpus[t] == (cpus ? cpus[t] : -1);
    if (same) return 0;
    pool_stop();
    pool.n = nt;
    pool.alive = 1;
    for (int t = 0; t < nt; ++t) pool.cpus[t] = cpus ? cpus[t] : -1;
    pthread_barrier_init(&pool.start, NULL, (unsigned)nt + 1);
    pthread_barrier_init(&pool.mid, NULL, (unsigned)nt);
    pthread_barrier_init(&pool.done, NULL, (unsigned)nt + 1);
    for (int t = 0; t < nt; ++t)
        if (pthread_create(&pool.th[t], NULL, pool_worker, (void*)(intptr_t)t) != 0) return -1;
    return 0;
}

/*
 * Y[m][n] = vec_dot(W row n, quantize(X row m)) for m < M, n < N: the operator the reference's
 * CPU backend computes, as described at the top of this file. isa < 0 picks the best the CPU
 * supports. The workers (nthreads, pinned to cpus[0 .. nthreads) unless cpus is NULL) persist
 * between calls with the same nthreads and cpus; calls must not overlap. Returns 0, or a negative
 * value on bad arguments.
 */
int dcqs_mul_mat(int isa, int wtype, const void* w, int64_t n, int64_t k, size_t w_row_bytes, const float* x,
                 int64_t m, int64_t x_stride, float* y, int64_t y_stride, int nthreads, const int* cpus) {
    const int vdt = dcqo_vec_dot_type(wtype);
    if (vdt < 0 || dcqo_row_size(wtype, k) <= 0 || n <= 0 || m <= 0) return -1;
    if (isa < 0) isa = dcqs_isa();
    const size_t xrb = (size_t)dcqo_row_size(vdt, k);
    char* xq = (char*)malloc(xrb * (size_t)m);
    if (!xq) return -3;
    int nt = nthreads > 0 ? nthreads : 1;
    if (nt > 256) nt = 256;
    if (pool_start(nt, cpus) != 0) {
        free(xq);
        return -4;
    }
    pool.call = (simd_call){isa, wtype, vdt, (const char*)w, k, w_row_bytes, x, x_stride, xq, xrb, m, n, y, y_stride};
    pthread_barrier_wait(&pool.start);
    pthread_barrier_wait(&pool.done);
    free(xq);
    return 0;
}

/* Stops the worker pool (the next dcqs_mul_mat starts a new one). */
void dcqs_shutdown(void) { pool_stop(); }
