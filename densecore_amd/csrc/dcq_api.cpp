// dcq_api.cpp — the extern "C" boundary of libdcq (declared in include/dcq.h).
//
// Every entry point validates its arguments on the host before touching the
// device, so a bad call returns a status and launches nothing. Device work is
// stream-ordered on the caller's stream.
#include <hip/hip_runtime.h>

#include <array>
#include <mutex>
#include <stdlib.h>
#include <string.h>

#include "../../include/dcq.h"
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

size_t planar_bytes(int vdt, int64_t M, int64_t K, PlanarBuffers* pb, void* base) {
    const int64_t bs = vdt == kTypeQ8_0 ? QK8_0 : QK_K;  // the activation types: Q8_0 or Q8_K
    const int64_t m_ld = round_up(M, 128);  // >= every MFMA m-tile, so float4 scale loads stay in bounds
    const size_t qs_b = (size_t)round_up(M * K, 256);
    const size_t d_b = (size_t)round_up((K / bs) * m_ld * 4, 256);
    const size_t bs_b = vdt == kTypeQ8_K ? (size_t)round_up(M * (K / 16) * 2, 256) : 0;
    if (pb) {
        char* p = (char*)base;
        pb->qs = (int8_t*)p;
        pb->d = (float*)(p + qs_b);
        pb->bs = vdt == kTypeQ8_K ? (int16_t*)(p + qs_b + d_b) : nullptr;
        pb->m_ld = m_ld;
    }
    return qs_b + d_b + bs_b;
}

// Room for the split-K partial tiles of the MFMA kernels (used past the decode kernels' rows when
// the output tiles cannot give every CU a workgroup): one fp32 128 x 128 tile per CU of a 256-CU
// device, i.e. M * 128 KB up to M = 128 (16 MB).
size_t split_tail_bytes(int64_t M) { return M > 4 ? (size_t)(M < 128 ? M : 128) * 128 * 1024 : 0; }

// Activation rows up to which the decode (GEMV) kernels serve a product. Past four rows their
// per-row VALU work falls behind the batch MFMA kernels (8192 x 2048 at M = 8: Q8_0 23.3 ->
// 11.5 us, Q4_K 10.8 -> 9.4 us, Q6_K 17.7 -> 9.5 us). At three and four rows (steps, GEMV against
// batch kernel, one box): Q6_K keeps the GEMV from 10 to 16 superblocks per row and below 4096
// rows (4096 x 4096 9.6 against 12.7 us, 8192 x 4096 13.9 against 14.5 us, 2560 x 9728 21.1 against
// 22.1 us) and takes the batch kernel elsewhere (8192 x 2048 12.1 against 9.7 us, 5120 x 5120 14.8
// against 14.0 us, 4096 x 14336 33.6 against 28.4 us); Q4_0 keeps the GEMV up to K = 2048 (8192 x
// 2048 7.5 against 9.5 us) but not beyond (9728 x 2560 20.6 against 11.9 us). Tall Q6_K matrices
// (LM heads, 32768+ rows) keep their MFMA decode kernel up to eight rows (151936 x 2560 at M = 4:
// 68 us against 120 us on the batch kernel).
// fused: the activation quantization runs inside the GEMV kernel (the small-matrix extension to
// eight rows pays only there: on a pre-quantized activation, Q8_0 M = 5 3072 x 1024 took 8.2 us on
// the GEMV against 5.3 us on the batch kernel)
int gemv_rows(int wtype, int64_t N, int64_t K, bool fused) {
    if (wtype == kTypeQ6_K) {
        if (N >= 32768) return 8;
        const int64_t nsb = K / 256;
        return N < 4096 || (nsb >= 10 && nsb <= 16) ? 4 : 2;
    }
    // small matrices keep the GEMV up to eight rows, where the batch kernel has few tiles and too
    // little K to split (M = 5-8: Q8_0 3072 x 1024 4.6 against 7.6 us, Q4_K 2048 x 2048 5.1-5.4
    // against 6.7 us; not Q8_0 at K = 2048: 2048 x 2048 11.2 against 10.1 us), and Q8_0 rows of
    // 1024 elements at any height (151936 x 1024 at M = 6: 58.0 against 77.7 us)
    // (row-split Q8_0 rows as their Q8_0 originals, so both give the same bits)
    const bool q8 = wtype == kTypeQ8_0 || wtype == kTypeQ8_0_RS;
    if (fused && ((q8 && K <= 1024) || (wtype == kTypeQ4_0 && K <= 1024 && N <= 4096) ||
                  ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && N * K <= (int64_t)2048 * 2048)))
        return 8;
    // Q8_0 rows of 4096+ elements over 4096+ rows: the batch kernel from three rows (M = 3:
    // 32000 x 4096 86.3 against 47.1 us; M = 4: 4096 x 4096 16.6 against 14.6 us; but 2048 x 8192
    // 16.0 against 22.1 us on the GEMV)
    if (q8 && K >= 4096 && N >= 4096) return 2;
    // Q4_K / Q5_K: likewise for large matrices of 4096+ element rows (M = 3: 14336 x 4096 23.4
    // against 15.7 us, 4096 x 14336 47.6 against 18.7 us, 8192 x 8192 31.7 against 14.8 us; the
    // GEMV stays for 9728 x 2560, 4096 x 4096 and 151936 x 1024)
    if ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && K >= 4096 && N * K >= ((int64_t)1 << 25)) return 2;
    if (wtype == kTypeQ4_0) return K <= 2048 ? 4 : 2;
    return 4;
}

// the bytes of a workspace past its first `used` ones, as split-K scratch (none if too small)
SplitScratch tail_of(void* ws, size_t ws_bytes, size_t used) {
    SplitScratch sc;
    used = (size_t)round_up((int64_t)used, 256);
    if (ws && ws_bytes > used) {
        sc.p = reinterpret_cast<float*>(static_cast<char*>(ws) + used);
        sc.bytes = ws_bytes - used;
    }
    return sc;
}

#ifdef DCQ_TUNING
// Tuning build only: the overrides come from the environment, read once (thread-safe static
// initialisation), not per call. The default build uses the constant knob() in dcq_kernels.h.
int knob(Knob k) {
    static const char* const kNames[(int)Knob::kCount] = {
        "DCQ_Q4K_SHAPE",    "DCQ_Q4K_NW",  "DCQ_NO_FUSE",      "DCQ_Q6K_DECODE", "DCQ_Q6K_LDS_OFF",
        "DCQ_Q6K_NO_FUSE",  "DCQ_Q6K_FUSE_NW", "DCQ_Q8_SHAPE", "DCQ_GEMV_GENERIC", "DCQ_GEMV_LG",
        "DCQ_ATTN_NO_MFMA", "DCQ_Q6K_RPW", "DCQ_Q6K_MFMA",     "DCQ_SPLIT_K",    "DCQ_BATCH_MTI",
    };
    static const std::array<int, (int)Knob::kCount> values = [] {
        std::array<int, (int)Knob::kCount> v{};
        for (int i = 0; i < (int)Knob::kCount; ++i) {
            const char* s = getenv(kNames[i]);
            v[i] = (s && *s) ? atoi(s) : kKnobDefault[i];
        }
        return v;
    }();
    return values[(int)k];
}
#endif

}  // namespace dcq

using namespace dcq;

namespace {

bool is_weight_type(int t) {
    return t == kTypeQ8_0 || t == kTypeQ4_0 || t == kTypeQ4_K || t == kTypeQ5_K || t == kTypeQ6_K || t == kTypeQ8_0_RS;
}

// Row-split Q8_0 rows: K % 256 == 0 and 16-byte row strides (every 16-byte piece of the quants
// plane aligned). DCQ_OK or the status to return.
int check_rs_rows(int wtype, int64_t K, size_t w_row_bytes) {
    if (wtype != kTypeQ8_0_RS) return DCQ_OK;
    if (K % 256) return DCQ_ERR_BAD_SHAPE;
    if (w_row_bytes % 16) return DCQ_ERR_MISALIGNED;
    return DCQ_OK;
}

// The kernels are built for gfx950 only; refuse other devices loudly.
int check_device() {
    static std::mutex mu;
    static int ok_for[64] = {0};  // 0 unknown, 1 ok, -1 bad
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return DCQ_ERR_NO_DEVICE;
    if (dev < 0 || dev >= 64) return DCQ_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(mu);
    if (ok_for[dev] == 0) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return DCQ_ERR_NO_DEVICE;
        ok_for[dev] = strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    }
    return ok_for[dev] == 1 ? DCQ_OK : DCQ_ERR_NO_DEVICE;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int hip_status(hipError_t e) { return e == hipSuccess ? DCQ_OK : DCQ_ERR_HIP; }

// Validation of dcq_mul_mat-style arguments (no device calls).
int validate_mul_mat(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X, int64_t M,
                     size_t x_stride_bytes, const float* Y, size_t y_stride_bytes) {
    if (!is_weight_type(wtype)) return DCQ_ERR_UNSUPPORTED;
    if (!W || !X || !Y) return DCQ_ERR_INVALID_ARG;
    if (N <= 0 || M <= 0 || K <= 0) return DCQ_ERR_BAD_SHAPE;
    if (K % dcq_block_size(wtype)) return DCQ_ERR_BAD_SHAPE;
    if (K > (int64_t)1 << 30 || N > (int64_t)1 << 31 || M > (int64_t)1 << 31) return DCQ_ERR_BAD_SHAPE;
    if (w_row_bytes < dcq_row_size(wtype, K)) return DCQ_ERR_INVALID_ARG;
    if (x_stride_bytes < (size_t)K * 4 || y_stride_bytes < (size_t)N * 4) return DCQ_ERR_INVALID_ARG;
    if (!aligned(W, 16) || !aligned(X, 16) || !aligned(Y, 4)) return DCQ_ERR_MISALIGNED;
    if (x_stride_bytes % 16 || y_stride_bytes % 4) return DCQ_ERR_MISALIGNED;
    if (w_row_bytes % 2) return DCQ_ERR_MISALIGNED;
    if ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && w_row_bytes % 16) return DCQ_ERR_MISALIGNED;
    return check_rs_rows(wtype, K, w_row_bytes);
}

bool is_cache_type(int t) { return t == kTypeQ8_0 || t == kTypeF16 || t == kTypeF32; }

// Shared checks of the arena arguments (no device calls).
int validate_arena(int ct, const void* arena, int64_t n_blocks, int n_layer, int layer, int64_t row_elems) {
    if (!is_cache_type(ct)) return DCQ_ERR_UNSUPPORTED;
    if (!arena) return DCQ_ERR_INVALID_ARG;
    if (n_blocks <= 0 || n_blocks > INT32_MAX || n_layer <= 0 || layer < 0 || layer >= n_layer) return DCQ_ERR_BAD_SHAPE;
    if (row_elems <= 0 || row_elems % 32 || row_elems > ((int64_t)1 << 24)) return DCQ_ERR_BAD_SHAPE;
    if (!aligned(arena, 16)) return DCQ_ERR_MISALIGNED;
    return DCQ_OK;
}

}  // namespace

extern "C" {

const char* dcq_version(void) { return "dcq 0.1.0 gfx950"; }

const char* dcq_status_string(int s) {
    switch (s) {
        case DCQ_OK: return "ok";
        case DCQ_ERR_INVALID_ARG: return "invalid argument";
        case DCQ_ERR_UNSUPPORTED: return "unsupported type";
        case DCQ_ERR_BAD_SHAPE: return "bad shape (K must be a multiple of the block size; dims > 0)";
        case DCQ_ERR_MISALIGNED: return "misaligned pointer or stride";
        case DCQ_ERR_WORKSPACE: return "workspace too small";
        case DCQ_ERR_HIP: return "HIP runtime error";
        case DCQ_ERR_NO_DEVICE: return "no gfx950 device";
        case DCQ_ERR_FORMAT: return "malformed GGUF file";
        case DCQ_ERR_IO: return "file could not be opened or read";
        case DCQ_ERR_NOT_FOUND: return "key not found";
        case DCQ_ERR_SCRATCH_LIMIT: return "product needs more than the no-alloc scratch (DCQ_NOALLOC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

int64_t dcq_block_size(int type) {
    switch (type) {
        case DCQ_TYPE_F32:
        case DCQ_TYPE_F16: return 1;
        case DCQ_TYPE_Q4_0:
        case DCQ_TYPE_Q8_0:
        case DCQ_TYPE_Q8_0_RS: return QK8_0;
        case DCQ_TYPE_Q4_K:
        case DCQ_TYPE_Q5_K:
        case DCQ_TYPE_Q6_K:
        case DCQ_TYPE_Q8_K: return QK_K;
        default: return 0;
    }
}

int64_t dcq_type_size(int type) {
    switch (type) {
        case DCQ_TYPE_F32: return 4;
        case DCQ_TYPE_F16: return 2;
        case DCQ_TYPE_Q4_0: return (int64_t)sizeof(BlockQ4_0);
        case DCQ_TYPE_Q8_0:
        case DCQ_TYPE_Q8_0_RS: return (int64_t)sizeof(BlockQ8_0);
        case DCQ_TYPE_Q4_K: return (int64_t)sizeof(BlockQ4_K);
        case DCQ_TYPE_Q5_K: return (int64_t)sizeof(BlockQ5_K);
        case DCQ_TYPE_Q6_K: return (int64_t)sizeof(BlockQ6_K);
        case DCQ_TYPE_Q8_K: return (int64_t)sizeof(BlockQ8_K);
        default: return 0;
    }
}

size_t dcq_row_size(int type, int64_t k) {
    const int64_t bs = dcq_block_size(type);
    if (bs <= 0 || k < 0 || k % bs) return 0;
    return (size_t)((k / bs) * dcq_type_size(type));
}

int dcq_vec_dot_type(int wtype) {
    switch (wtype) {
        case DCQ_TYPE_Q4_0:
        case DCQ_TYPE_Q8_0:
        case DCQ_TYPE_Q8_0_RS: return DCQ_TYPE_Q8_0;
        case DCQ_TYPE_Q4_K:
        case DCQ_TYPE_Q5_K:
        case DCQ_TYPE_Q6_K: return DCQ_TYPE_Q8_K;
        default: return DCQ_ERR_UNSUPPORTED;
    }
}

int dcq_supports_mul_mat(int wtype, int xtype, int ytype) {
    return is_weight_type(wtype) && xtype == DCQ_TYPE_F32 && ytype == DCQ_TYPE_F32;
}

int64_t dcq_block_sums_per_row(int wtype, int64_t k) {
    if (!is_weight_type(wtype) || k <= 0 || k % dcq_block_size(wtype)) return 0;
    switch (wtype) {
        case DCQ_TYPE_Q4_0:
        case DCQ_TYPE_Q8_0:
        case DCQ_TYPE_Q8_0_RS: return k / QK8_0;
        case DCQ_TYPE_Q4_K:
        case DCQ_TYPE_Q5_K: return 2 * (k / QK_K);
        default: return k / QK_K;
    }
}

size_t dcq_mul_mat_workspace_size(int wtype, int64_t M, int64_t K) {
    const int vdt = dcq_vec_dot_type(wtype);
    if (vdt < 0 || M <= 0 || K <= 0 || K % dcq_block_size(wtype)) return 0;
    return planar_bytes(vdt, M, K, nullptr, nullptr) + split_tail_bytes(M);
}

int dcq_quantize_rows(int vdt, const float* X, int64_t M, int64_t K, size_t x_stride_bytes, void* Xq, void* stream) {
    if (vdt != DCQ_TYPE_Q8_0 && vdt != DCQ_TYPE_Q8_K) return DCQ_ERR_UNSUPPORTED;
    if (!X || !Xq) return DCQ_ERR_INVALID_ARG;
    if (M <= 0 || K <= 0 || K % dcq_block_size(vdt)) return DCQ_ERR_BAD_SHAPE;
    if (x_stride_bytes < (size_t)K * 4) return DCQ_ERR_INVALID_ARG;
    if (!aligned(X, 16) || x_stride_bytes % 16) return DCQ_ERR_MISALIGNED;
    if (!aligned(Xq, vdt == DCQ_TYPE_Q8_K ? 4 : 2)) return DCQ_ERR_MISALIGNED;
    int rc = check_device();
    if (rc) return rc;
    return hip_status(launch_quantize_ggml(vdt, X, (int64_t)(x_stride_bytes / 4), M, K, Xq,
                                           (int64_t)dcq_row_size(vdt, K), (hipStream_t)stream));
}

int dcq_mul_mat_ex(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X, int64_t M,
                   size_t x_stride_bytes, float* Y, size_t y_stride_bytes, void* workspace, size_t workspace_bytes,
                   int path, int32_t* block_sums, void* stream) {
    int rc = validate_mul_mat(wtype, W, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes);
    if (rc) return rc;
    if (path != DCQ_PATH_AUTO && path != DCQ_PATH_GEMV && path != DCQ_PATH_MMQ) return DCQ_ERR_INVALID_ARG;
    if (block_sums && !aligned(block_sums, 4)) return DCQ_ERR_MISALIGNED;
    const int vdt = dcq_vec_dot_type(wtype);
    const size_t need = planar_bytes(vdt, M, K, nullptr, nullptr);
    if (workspace) {
        if (workspace_bytes < need) return DCQ_ERR_WORKSPACE;
        if (!aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    }
    rc = check_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const bool use_gemv = path == DCQ_PATH_GEMV || (path == DCQ_PATH_AUTO && M <= gemv_rows(wtype, N, K, false));
    if (path == DCQ_PATH_GEMV || (path == DCQ_PATH_AUTO && M <= gemv_rows(wtype, N, K, true))) {
        // decode: the activation quantization runs inside the GEMV kernel where it can
        hipError_t e = launch_decode_fused(wtype, W, (int64_t)w_row_bytes, N, K, X, (int64_t)(x_stride_bytes / 4), M,
                                           Y, (int64_t)(y_stride_bytes / 4), block_sums, st);
        if (e != hipErrorNotSupported) return hip_status(e);
    }
    // the workspace past the quantized activation (when there is room) holds split-K partial sums
    void* ws = workspace;
    size_t ws_total = workspace_bytes;
    if (!ws) {
        ws_total = need + split_tail_bytes(M);
        if (hipMallocAsync(&ws, ws_total, st) != hipSuccess) return DCQ_ERR_HIP;
    }
    PlanarBuffers pb;
    planar_bytes(vdt, M, K, &pb, ws);
    hipError_t e = launch_quantize_planar(vdt, X, (int64_t)(x_stride_bytes / 4), M, K, pb, st);
    if (e == hipSuccess) {
        const int64_t y_stride = (int64_t)(y_stride_bytes / 4);
        if (use_gemv)
            e = launch_gemv(wtype, W, (int64_t)w_row_bytes, 0, N, K, pb, M, Y, y_stride, block_sums, N, st);
        else
            e = launch_mmq(wtype, W, (int64_t)w_row_bytes, N, K, pb, M, Y, y_stride, block_sums, st,
                           tail_of(ws, ws_total, need));
    }
    if (!workspace) {
        hipError_t e2 = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = e2;
    }
    return hip_status(e);
}

int dcq_mul_mat(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X, int64_t M,
                size_t x_stride_bytes, float* Y, size_t y_stride_bytes, void* workspace, size_t workspace_bytes,
                void* stream) {
    return dcq_mul_mat_ex(wtype, W, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes, workspace,
                          workspace_bytes, DCQ_PATH_AUTO, nullptr, stream);
}

int dcq_mul_mat_noalloc(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X,
                        int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes, void* stream) {
    int rc = validate_mul_mat(wtype, W, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes);
    if (rc) return rc;
    if (planar_bytes(dcq_vec_dot_type(wtype), M, K, nullptr, nullptr) > DCQ_NOALLOC_SCRATCH_BYTES)
        return DCQ_ERR_SCRATCH_LIMIT;
    if ((rc = check_device())) return rc;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    if ((rc = noalloc_scratch(&ws, &ws_bytes))) return rc;
    // a non-null workspace: dcq_mul_mat_ex allocates nothing
    return dcq_mul_mat_ex(wtype, W, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes, ws, ws_bytes,
                          DCQ_PATH_AUTO, nullptr, stream);
}

size_t dcq_mul_mat_add_workspace_size(int wtype, int64_t M, int64_t N, int64_t K) {
    const size_t a = dcq_mul_mat_workspace_size(wtype, M, K);
    if (!a || N <= 0) return 0;
    return a + (size_t)round_up(M * N * 4, 256);
}

int dcq_mul_mat_add(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const float* X, int64_t M,
                    size_t x_stride_bytes, const float* R, size_t r_stride_bytes, float* Y, size_t y_stride_bytes,
                    void* workspace, size_t workspace_bytes, void* stream) {
    int rc = validate_mul_mat(wtype, W, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes);
    if (rc) return rc;
    if (!R) return DCQ_ERR_INVALID_ARG;
    if (r_stride_bytes != 0 && r_stride_bytes < (size_t)N * 4) return DCQ_ERR_INVALID_ARG;
    if (!aligned(R, 4) || r_stride_bytes % 4) return DCQ_ERR_MISALIGNED;
    // R is either Y itself (same stride: each element is read, then written, by one lane) or
    // disjoint from Y's extent
    const bool in_place = (const void*)R == (const void*)Y;
    if (in_place && r_stride_bytes != y_stride_bytes) return DCQ_ERR_INVALID_ARG;
    if (!in_place) {
        const uintptr_t y0 = (uintptr_t)Y, y1 = y0 + (size_t)(M - 1) * y_stride_bytes + (size_t)N * 4;
        const uintptr_t r0 = (uintptr_t)R, r1 = r0 + (size_t)(M - 1) * r_stride_bytes + (size_t)N * 4;
        if (r0 < y1 && y0 < r1) return DCQ_ERR_INVALID_ARG;
    }
    // required: the activation and the [M][N] temporary; the split-K room after them is optional
    const size_t need = dcq_mul_mat_add_workspace_size(wtype, M, N, K);
    if (workspace) {
        if (workspace_bytes < need - split_tail_bytes(M)) return DCQ_ERR_WORKSPACE;
        if (!aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    }
    rc = check_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int64_t y_stride = (int64_t)(y_stride_bytes / 4), r_stride = (int64_t)(r_stride_bytes / 4);
    if (M <= gemv_rows(wtype, N, K, true)) {
        // decode: the add is the fused kernel's store epilogue
        hipError_t e = launch_decode_fused(wtype, W, (int64_t)w_row_bytes, N, K, X, (int64_t)(x_stride_bytes / 4), M,
                                           Y, y_stride, nullptr, st, R, r_stride);
        if (e != hipErrorNotSupported) return hip_status(e);
    }
    void* ws = workspace;
    if (!ws) {
        if (hipMallocAsync(&ws, need, st) != hipSuccess) return DCQ_ERR_HIP;
    }
    const int vdt = dcq_vec_dot_type(wtype);
    PlanarBuffers pb;
    const size_t act_bytes = planar_bytes(vdt, M, K, &pb, ws);
    // the product goes to Y when R is elsewhere, else to a workspace temporary [M][N]
    float* T = in_place ? reinterpret_cast<float*>(static_cast<char*>(ws) + act_bytes) : Y;
    const int64_t t_stride = in_place ? N : y_stride;
    // split-K partial sums after the temporary
    const SplitScratch sc = tail_of(ws, workspace ? workspace_bytes : need, act_bytes + (size_t)M * N * 4);
    hipError_t e = launch_quantize_planar(vdt, X, (int64_t)(x_stride_bytes / 4), M, K, pb, st);
    bool added = false;
    if (e == hipSuccess && M <= gemv_rows(wtype, N, K, false)) {
        // the LDS-staged decode kernels add R in their store
        e = launch_gemv(wtype, W, (int64_t)w_row_bytes, 0, N, K, pb, M, Y, y_stride, nullptr, N, st, R, r_stride);
        added = e != hipErrorNotSupported;
        if (!added) e = hipSuccess;
    }
    if (e == hipSuccess && !added) {
        e = M <= gemv_rows(wtype, N, K, false)
                ? launch_gemv(wtype, W, (int64_t)w_row_bytes, 0, N, K, pb, M, T, t_stride, nullptr, N, st)
                : launch_mmq(wtype, W, (int64_t)w_row_bytes, N, K, pb, M, T, t_stride, nullptr, st, sc);
        if (e == hipSuccess) e = launch_add_rows(Y, y_stride, T, t_stride, R, r_stride, M, N, st);
    }
    if (!workspace) {
        hipError_t e2 = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = e2;
    }
    return hip_status(e);
}

size_t dcq_ffn_gate_up_workspace_size(int wtype, int64_t M, int64_t N, int64_t K) {
    const size_t a = dcq_mul_mat_workspace_size(wtype, M, K);
    if (!a || N <= 0) return 0;
    return a + (size_t)round_up(M * N * 4, 256);
}

int dcq_ffn_gate_up(int wtype, const void* Wg, const void* Wu, int64_t N, int64_t K, size_t w_row_bytes,
                    const float* X, int64_t M, size_t x_stride_bytes, float* Y, size_t y_stride_bytes,
                    void* workspace, size_t workspace_bytes, void* stream) {
    int rc = validate_mul_mat(wtype, Wg, N, K, w_row_bytes, X, M, x_stride_bytes, Y, y_stride_bytes);
    if (rc) return rc;
    if (!Wu) return DCQ_ERR_INVALID_ARG;
    if (!aligned(Wu, 16)) return DCQ_ERR_MISALIGNED;
    // required: the activation and the [M][N] temporary; the split-K room after them is optional
    const size_t need = dcq_ffn_gate_up_workspace_size(wtype, M, N, K);
    if (workspace) {
        if (workspace_bytes < need - split_tail_bytes(M)) return DCQ_ERR_WORKSPACE;
        if (!aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    }
    rc = check_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int64_t y_stride = (int64_t)(y_stride_bytes / 4);
    if (M <= gemv_rows(wtype, N, K, true)) {
        // one launch: both weight rows per lane group, the activation quantized in the workgroup
        hipError_t e = launch_decode_fused_glu(wtype, Wg, Wu, (int64_t)w_row_bytes, N, K, X,
                                               (int64_t)(x_stride_bytes / 4), M, Y, y_stride, st);
        if (e != hipErrorNotSupported) return hip_status(e);
    }
    void* ws = workspace;
    if (!ws) {
        if (hipMallocAsync(&ws, need, st) != hipSuccess) return DCQ_ERR_HIP;
    }
    const int vdt = dcq_vec_dot_type(wtype);
    PlanarBuffers pb;
    const size_t act_bytes = planar_bytes(vdt, M, K, &pb, ws);
    float* U = reinterpret_cast<float*>(static_cast<char*>(ws) + act_bytes);  // [M][N]
    // split-K partial sums after U (the two products run one after the other on the stream)
    const SplitScratch sc = tail_of(ws, workspace ? workspace_bytes : need, act_bytes + (size_t)M * N * 4);
    hipError_t e = launch_quantize_planar(vdt, X, (int64_t)(x_stride_bytes / 4), M, K, pb, st);
    const bool use_gemv = M <= gemv_rows(wtype, N, K, false);
    if (e == hipSuccess)
        e = use_gemv ? launch_gemv(wtype, Wg, (int64_t)w_row_bytes, 0, N, K, pb, M, Y, y_stride, nullptr, N, st)
                     : launch_mmq(wtype, Wg, (int64_t)w_row_bytes, N, K, pb, M, Y, y_stride, nullptr, st, sc);
    if (e == hipSuccess)
        e = use_gemv ? launch_gemv(wtype, Wu, (int64_t)w_row_bytes, 0, N, K, pb, M, U, N, nullptr, N, st)
                     : launch_mmq(wtype, Wu, (int64_t)w_row_bytes, N, K, pb, M, U, N, nullptr, st, sc);
    if (e == hipSuccess) e = launch_silu_mul(Y, y_stride, U, N, M, N, st);
    if (!workspace) {
        hipError_t e2 = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = e2;
    }
    return hip_status(e);
}

int dcq_quantize_src1(int wtype, const float* X, int64_t M, int64_t K, size_t x_stride_bytes, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (!is_weight_type(wtype)) return DCQ_ERR_UNSUPPORTED;
    if (!X || !workspace) return DCQ_ERR_INVALID_ARG;
    if (M <= 0 || K <= 0 || K % dcq_block_size(wtype)) return DCQ_ERR_BAD_SHAPE;
    if (K > (int64_t)1 << 30 || M > (int64_t)1 << 31) return DCQ_ERR_BAD_SHAPE;
    if (x_stride_bytes < (size_t)K * 4) return DCQ_ERR_INVALID_ARG;
    if (!aligned(X, 16) || x_stride_bytes % 16 || !aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    const int vdt = dcq_vec_dot_type(wtype);
    if (workspace_bytes < planar_bytes(vdt, M, K, nullptr, nullptr)) return DCQ_ERR_WORKSPACE;
    int rc = check_device();
    if (rc) return rc;
    PlanarBuffers pb;
    planar_bytes(vdt, M, K, &pb, workspace);
    return hip_status(launch_quantize_planar(vdt, X, (int64_t)(x_stride_bytes / 4), M, K, pb, (hipStream_t)stream));
}

int dcq_mul_mat_q(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, const void* workspace,
                  size_t workspace_bytes, int64_t M, float* Y, size_t y_stride_bytes, int path, void* stream) {
    if (!workspace) return DCQ_ERR_INVALID_ARG;
    // X is already quantized: validate the rest with a stand-in X of the right alignment
    int rc = validate_mul_mat(wtype, W, N, K, w_row_bytes, (const float*)workspace, M, (size_t)K * 4 + 16, Y,
                              y_stride_bytes);
    if (rc) return rc;
    if (path != DCQ_PATH_AUTO && path != DCQ_PATH_GEMV && path != DCQ_PATH_MMQ) return DCQ_ERR_INVALID_ARG;
    const int vdt = dcq_vec_dot_type(wtype);
    if (workspace_bytes < planar_bytes(vdt, M, K, nullptr, nullptr)) return DCQ_ERR_WORKSPACE;
    if (!aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    rc = check_device();
    if (rc) return rc;
    PlanarBuffers pb;
    planar_bytes(vdt, M, K, &pb, (void*)workspace);
    hipStream_t st = (hipStream_t)stream;
    const int64_t y_stride = (int64_t)(y_stride_bytes / 4);
    const bool use_gemv = path == DCQ_PATH_GEMV || (path == DCQ_PATH_AUTO && M <= gemv_rows(wtype, N, K, false));
    // The workspace is read-only here: products that share one quantization may run on different
    // streams. So there is no split-K room (it would be written): the MFMA kernels run unsplit,
    // with the same result bits as dcq_mul_mat given an activation-only workspace.
    hipError_t e = use_gemv ? launch_gemv(wtype, W, (int64_t)w_row_bytes, 0, N, K, pb, M, Y, y_stride, nullptr, N, st)
                            : launch_mmq(wtype, W, (int64_t)w_row_bytes, N, K, pb, M, Y, y_stride, nullptr, st,
                                         SplitScratch{});
    return hip_status(e);
}

int dcq_dot_rows(int wtype, const void* W, size_t w_row_bytes, const void* Xq, int64_t K, float* Y, int64_t n0,
                 int64_t n1, void* stream) {
    if (!is_weight_type(wtype)) return DCQ_ERR_UNSUPPORTED;
    if (!W || !Xq || !Y) return DCQ_ERR_INVALID_ARG;
    if (K <= 0 || K % dcq_block_size(wtype) || n0 < 0 || n1 < n0) return DCQ_ERR_BAD_SHAPE;
    if (w_row_bytes < dcq_row_size(wtype, K)) return DCQ_ERR_INVALID_ARG;
    if (!aligned(W, 16) || !aligned(Y, 4)) return DCQ_ERR_MISALIGNED;
    if (w_row_bytes % 2) return DCQ_ERR_MISALIGNED;
    if ((wtype == kTypeQ4_K || wtype == kTypeQ5_K) && w_row_bytes % 16) return DCQ_ERR_MISALIGNED;
    if (int rs = check_rs_rows(wtype, K, w_row_bytes)) return rs;
    const int vdt = dcq_vec_dot_type(wtype);
    if (!aligned(Xq, vdt == kTypeQ8_K ? 4 : 2)) return DCQ_ERR_MISALIGNED;
    if (n1 == n0) return DCQ_OK;
    int rc = check_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const size_t need = planar_bytes(vdt, 1, K, nullptr, nullptr);
    void* ws = nullptr;
    if (hipMallocAsync(&ws, need, st) != hipSuccess) return DCQ_ERR_HIP;
    PlanarBuffers pb;
    planar_bytes(vdt, 1, K, &pb, ws);
    hipError_t e = launch_unpack_ggml_rows(vdt, Xq, (int64_t)dcq_row_size(vdt, K), 1, K, pb, st);
    if (e == hipSuccess)
        e = launch_gemv(wtype, (const uint8_t*)W, (int64_t)w_row_bytes, n0, n1, K, pb, 1, Y, n1 - n0, nullptr,
                        n1 - n0, st);
    hipError_t e2 = hipFreeAsync(ws, st);
    if (e == hipSuccess) e = e2;
    return hip_status(e);
}

int dcq_quantize_weights(int wtype, const float* W, int64_t N, int64_t K, void* Wq, void* stream) {
    if (!is_weight_type(wtype) || wtype == kTypeQ8_0_RS) return DCQ_ERR_UNSUPPORTED;
    if (!W || !Wq) return DCQ_ERR_INVALID_ARG;
    if (N <= 0 || K <= 0 || K % dcq_block_size(wtype)) return DCQ_ERR_BAD_SHAPE;
    if (!aligned(W, 4) || !aligned(Wq, 16)) return DCQ_ERR_MISALIGNED;
    int rc = check_device();
    if (rc) return rc;
    return hip_status(launch_quantize_weights(wtype, W, N, K, Wq, (hipStream_t)stream));
}

int dcq_repack_weights(int wtype, const void* W, int64_t N, int64_t K, size_t w_row_bytes, int out_type, void* Wr,
                       size_t wr_row_bytes, void* stream) {
    if (wtype != DCQ_TYPE_Q8_0 || out_type != DCQ_TYPE_Q8_0_RS) return DCQ_ERR_UNSUPPORTED;
    if (!W || !Wr) return DCQ_ERR_INVALID_ARG;
    if (N <= 0 || K <= 0 || K % 256 || K > (int64_t)1 << 30 || N > (int64_t)1 << 31) return DCQ_ERR_BAD_SHAPE;
    if (w_row_bytes < dcq_row_size(wtype, K) || wr_row_bytes < dcq_row_size(out_type, K)) return DCQ_ERR_INVALID_ARG;
    if (!aligned(W, 2) || w_row_bytes % 2 || !aligned(Wr, 16) || wr_row_bytes % 16) return DCQ_ERR_MISALIGNED;
    // the source and destination must not overlap (rows are rearranged, not moved in place)
    const uintptr_t a0 = (uintptr_t)W, a1 = a0 + (uintptr_t)((N - 1) * (int64_t)w_row_bytes + dcq_row_size(wtype, K));
    const uintptr_t b0 = (uintptr_t)Wr, b1 = b0 + (uintptr_t)((N - 1) * (int64_t)wr_row_bytes + dcq_row_size(out_type, K));
    if (a0 < b1 && b0 < a1) return DCQ_ERR_INVALID_ARG;
    int rc = check_device();
    if (rc) return rc;
    return hip_status(launch_repack_q8_0_rs(W, (int64_t)w_row_bytes, N, K, Wr, (int64_t)wr_row_bytes,
                                            (hipStream_t)stream));
}

int dcq_dequantize_rows(int type, const void* Wq, int64_t N, int64_t K, size_t w_row_bytes, float* Y, void* stream) {
    if (!is_weight_type(type) && type != DCQ_TYPE_Q8_K) return DCQ_ERR_UNSUPPORTED;
    if (!Wq || !Y) return DCQ_ERR_INVALID_ARG;
    if (N <= 0 || K <= 0 || K % dcq_block_size(type)) return DCQ_ERR_BAD_SHAPE;
    if (w_row_bytes < dcq_row_size(type, K)) return DCQ_ERR_INVALID_ARG;
    if (!aligned(Y, 4) || w_row_bytes % 2 || !aligned(Wq, 4)) return DCQ_ERR_MISALIGNED;
    int rc = check_device();
    if (rc) return rc;
    return hip_status(launch_dequantize(type, Wq, N, K, (int64_t)w_row_bytes, Y, (hipStream_t)stream));
}

size_t dcq_kv_slot_bytes(int cache_type, int64_t row_elems) {
    if (!is_cache_type(cache_type) || row_elems <= 0 || row_elems % 32) return 0;
    return dcq_row_size(cache_type, row_elems);
}

int dcq_kv_write(int cache_type, void* arena, int64_t n_blocks, int n_layer, int layer, int64_t row_elems,
                 const int32_t* block_table, int64_t n_table, int64_t pos0, const float* src,
                 size_t src_stride_bytes, int64_t n_tokens, void* stream) {
    int rc = validate_arena(cache_type, arena, n_blocks, n_layer, layer, row_elems);
    if (rc) return rc;
    if (n_tokens < 0 || pos0 < 0 || n_tokens > INT32_MAX || pos0 + n_tokens > INT32_MAX) return DCQ_ERR_BAD_SHAPE;
    if (n_tokens == 0) return DCQ_OK;
    if (!block_table || !src) return DCQ_ERR_INVALID_ARG;
    if ((pos0 + n_tokens - 1) / DCQ_KV_BLOCK_SIZE >= n_table) return DCQ_ERR_INVALID_ARG;
    if (src_stride_bytes < (size_t)row_elems * 4) return DCQ_ERR_INVALID_ARG;
    if (!aligned(src, 16) || src_stride_bytes % 16 || !aligned(block_table, 4)) return DCQ_ERR_MISALIGNED;
    if ((rc = check_device())) return rc;
    return hip_status(launch_kv_write(cache_type, arena, (int)n_blocks, n_layer, layer, row_elems,
                                      (int64_t)dcq_kv_slot_bytes(cache_type, row_elems), block_table, (int)pos0, src,
                                      (int64_t)(src_stride_bytes / 4), (int)n_tokens, (hipStream_t)stream));
}

int dcq_kv_gather(int cache_type, const void* arena, int64_t n_blocks, int n_layer, int layer, int64_t row_elems,
                  const int32_t* block_table, int64_t n_table, int64_t n_past, const float* cur,
                  size_t cur_stride_bytes, int64_t n_tokens, float* dst, size_t dst_stride_bytes, void* stream) {
    int rc = validate_arena(cache_type, arena, n_blocks, n_layer, layer, row_elems);
    if (rc) return rc;
    if (n_tokens < 0 || n_past < 0 || n_table < 0 || n_past + n_tokens > INT32_MAX) return DCQ_ERR_BAD_SHAPE;
    if (n_past + n_tokens == 0) return DCQ_OK;
    if (!dst || (n_tokens > 0 && !cur) || (n_past > 0 && n_table > 0 && !block_table)) return DCQ_ERR_INVALID_ARG;
    if (dst_stride_bytes < (size_t)row_elems * 4 || (n_tokens > 0 && cur_stride_bytes < (size_t)row_elems * 4))
        return DCQ_ERR_INVALID_ARG;
    if (!aligned(dst, 16) || dst_stride_bytes % 16 || !aligned(block_table, 4)) return DCQ_ERR_MISALIGNED;
    if (n_tokens > 0 && (!aligned(cur, 16) || cur_stride_bytes % 16)) return DCQ_ERR_MISALIGNED;
    if ((rc = check_device())) return rc;
    const int nt = n_table > INT32_MAX ? INT32_MAX : (int)n_table;
    return hip_status(launch_kv_gather(cache_type, arena, (int)n_blocks, n_layer, layer, row_elems,
                                       (int64_t)dcq_kv_slot_bytes(cache_type, row_elems), block_table, nt,
                                       (int)n_past, cur, (int64_t)(cur_stride_bytes / 4), (int)n_tokens, dst,
                                       (int64_t)(dst_stride_bytes / 4), (hipStream_t)stream));
}

static int validate_attention_shape(int n_head, int n_head_kv, int head_dim, int64_t n_tokens, int64_t n_past) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return DCQ_ERR_UNSUPPORTED;
    if (n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv || n_head > 4096) return DCQ_ERR_BAD_SHAPE;
    if (n_tokens <= 0 || n_tokens > 65535 || n_past < 0 || n_past > ((int64_t)1 << 24)) return DCQ_ERR_BAD_SHAPE;
    return DCQ_OK;
}

size_t dcq_kv_attention_workspace_size(int n_head, int n_head_kv, int head_dim, int64_t n_tokens, int64_t n_past) {
    if (validate_attention_shape(n_head, n_head_kv, head_dim, n_tokens, n_past)) return 0;
    return attn_workspace_bytes(head_dim, n_head, n_head_kv, (int)n_tokens, (int)n_past);
}

int dcq_kv_attention(int cache_type, const void* k_arena, const void* v_arena, int64_t n_blocks, int n_layer,
                     int layer, const int32_t* block_table, int64_t n_table, int n_head, int n_head_kv,
                     int head_dim, const float* q, size_t q_stride_bytes, const float* k_cur, const float* v_cur,
                     size_t kv_stride_bytes, int64_t n_tokens, int64_t n_past, float scale, float* out,
                     size_t out_stride_bytes, void* workspace, size_t workspace_bytes, void* stream) {
    const int64_t row_elems = (int64_t)n_head_kv * head_dim;
    int rc = validate_attention_shape(n_head, n_head_kv, head_dim, n_tokens, n_past);
    if (rc) return rc;
    if ((rc = validate_arena(cache_type, k_arena, n_blocks, n_layer, layer, row_elems))) return rc;
    if ((rc = validate_arena(cache_type, v_arena, n_blocks, n_layer, layer, row_elems))) return rc;
    if (!q || !k_cur || !v_cur || !out || (n_past > 0 && n_table > 0 && !block_table) || n_table < 0)
        return DCQ_ERR_INVALID_ARG;
    if (!(scale == scale) || scale == INFINITY || scale == -INFINITY) return DCQ_ERR_INVALID_ARG;
    const size_t q_row = (size_t)n_head * head_dim * 4, kv_row = (size_t)row_elems * 4;
    if (q_stride_bytes < q_row || kv_stride_bytes < kv_row || out_stride_bytes < q_row) return DCQ_ERR_INVALID_ARG;
    if (!aligned(q, 16) || !aligned(k_cur, 16) || !aligned(v_cur, 16) || !aligned(out, 4) ||
        !aligned(block_table, 4))
        return DCQ_ERR_MISALIGNED;
    if (q_stride_bytes % 16 || kv_stride_bytes % 16 || out_stride_bytes % 4) return DCQ_ERR_MISALIGNED;
    const size_t need = attn_workspace_bytes(head_dim, n_head, n_head_kv, (int)n_tokens, (int)n_past);
    if (need) {
        if (!workspace || workspace_bytes < need) return DCQ_ERR_WORKSPACE;
        if (!aligned(workspace, 256)) return DCQ_ERR_MISALIGNED;
    }
    if ((rc = check_device())) return rc;
    const int nt = n_table > INT32_MAX ? INT32_MAX : (int)n_table;
    return hip_status(launch_kv_attention(
        cache_type, k_arena, v_arena, (int)n_blocks, n_layer, layer, (int64_t)dcq_kv_slot_bytes(cache_type, row_elems),
        block_table, nt, n_head, n_head_kv, head_dim, q, (int64_t)(q_stride_bytes / 4), k_cur, v_cur,
        (int64_t)(kv_stride_bytes / 4), (int)n_tokens, (int)n_past, scale, out, (int64_t)(out_stride_bytes / 4),
        workspace, workspace_bytes, (hipStream_t)stream));
}

}  // extern "C"
