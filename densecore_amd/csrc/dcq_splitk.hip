// dcq_splitk.hip — split-K for the 128 x 128-tile int8-MFMA prefill kernels.
//
// ggml's CPU MUL_MAT at M > 1 (core/src/inference.cpp:1049-1063, executed at
// core/src/worker.cpp:544) runs every projection of a batch. With few output tiles (a 2048-row
// weight at M <= 256 has 16-32 tiles of 128 x 128) the tiled kernels leave most of the 256 CUs
// idle while each workgroup walks the whole K. Here the K stages are cut into ranges; each range
// of each tile is a workgroup that stores its partial tile (fp32) in a plane of the caller's
// workspace, and a second kernel adds the planes in range order. The order is fixed, so a given
// shape, device and workspace always give the same bits.
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

namespace {

// one thread per output (V4: four consecutive outputs): Y[m][n] = sum_s P[s][m][n], s ascending
template <bool V4>
__global__ void __launch_bounds__(256) sum_splits_kernel(const float* __restrict__ P, int splits, int64_t plane,
                                                         int64_t N, int64_t n_items, float* __restrict__ Y,
                                                         int64_t y_stride) {
    constexpr int V = V4 ? 4 : 1;
    const int64_t nv = N / V;  // items per row
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n_items; i += (int64_t)gridDim.x * 256) {
        const int64_t m = i / nv, n = (i - m * nv) * V;
        const int64_t e = m * N + n;
        if constexpr (V4) {
            float4 a = *reinterpret_cast<const float4*>(P + e);
            for (int s = 1; s < splits; ++s) {
                const float4 b = *reinterpret_cast<const float4*>(P + s * plane + e);
                a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
            }
            *reinterpret_cast<float4*>(Y + m * y_stride + n) = a;
        } else {
            float a = P[e];
            for (int s = 1; s < splits; ++s) a += P[s * plane + e];
            Y[m * y_stride + n] = a;
        }
    }
}

}  // namespace

// Splits while the tiles cannot give every CU a workgroup: at most one workgroup per CU, at least
// two stages per range (a range's first stage is not overlapped with loads) and no more planes
// than the scratch holds. Among those counts the one with the least estimated time: a lone
// workgroup per CU takes about us_per_stage per stage (2 us for the 128 x 128-tile kernels:
// measured 1.9 - 2.6 us on 2048 x 8192 and 8192 x 2048 at M = 64 - 256), and splitting adds about 2 us for the sum launch plus the partial planes
// written and read back at about 5 TB/s. DCQ_SPLIT_K forces the count (tuning).
SplitPlan plan_split_k(int64_t tiles, int nstages, int align, int64_t M, int64_t N, const SplitScratch& sc,
                       double us_per_stage) {
    const SplitPlan none{1, nstages};
    const int64_t plane_bytes = M * N * (int64_t)sizeof(float);
    const int min_stps = align > 2 ? align : 2;
    if (!sc.p || plane_bytes <= 0 || nstages < 2 * min_stps) return none;
    const int64_t max_by_scratch = (int64_t)(sc.bytes / (size_t)plane_bytes);
    int64_t smax = nstages / min_stps;
    if (smax > max_by_scratch) smax = max_by_scratch;
    auto plan_of = [&](int64_t s) {
        int stps = (int)((nstages + s - 1) / s);
        stps = (stps + align - 1) / align * align;
        return SplitPlan{(nstages + stps - 1) / stps, stps};
    };
    const int forced = knob(Knob::SplitK);
    if (forced >= 1) {
        const int64_t s = forced < smax ? forced : smax;
        return s < 2 ? none : plan_of(s);
    }
    const int64_t cus = cu_count();
    if (tiles >= cus) return none;
    if (smax > cus / tiles) smax = cus / tiles;
    SplitPlan best = none;
    double best_us = us_per_stage * nstages;  // no split
    for (int64_t s = 2; s <= smax; ++s) {
        const SplitPlan p = plan_of(s);
        if (p.splits < 2) continue;
        const double us = us_per_stage * p.stps + 2.0 + 2.0 * (double)p.splits * (double)plane_bytes / 5.0e6;
        if (us < best_us) {
            best_us = us;
            best = p;
        }
    }
    return best;
}

hipError_t launch_sum_splits(const float* P, int splits, int64_t M, int64_t N, float* Y, int64_t y_stride,
                             hipStream_t st) {
    const bool v4 = N % 4 == 0 && y_stride % 4 == 0 && (uintptr_t)Y % 16 == 0 && (uintptr_t)P % 16 == 0;
    const int64_t items = M * N / (v4 ? 4 : 1);
    int64_t grid = (items + 255) / 256;
    const int64_t cap = 4 * (int64_t)cu_count();
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    if (v4)
        hipLaunchKernelGGL(sum_splits_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, P, splits, M * N, N, items,
                           Y, y_stride);
    else
        hipLaunchKernelGGL(sum_splits_kernel<false>, dim3((unsigned)grid), dim3(256), 0, st, P, splits, M * N, N,
                           items, Y, y_stride);
    return hipGetLastError();
}

}  // namespace dcq
