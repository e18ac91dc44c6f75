// dcq_probe.hip — measurement aid: the fastest this GPU reads a given number of bytes.
//
// A decode GEMV must stream every weight byte once, so its best possible time at a given
// weight size is the time a kernel that does nothing but read those bytes takes. At the
// BASELINE decode sizes (3 - 20 MB) that time is dominated by launch, ramp-up and tail, not
// by the 8 TB/s peak, so the bench reports each decode kernel against this measured ceiling
// beside the peak. The kernel reads `bytes` with 16-byte loads, `per_lane` loads in flight
// per lane (all issued before any is used), 256 threads per workgroup, and folds the words
// into an XOR that is stored only if it equals a constant, so no load can be dropped.
#include <hip/hip_runtime.h>

#include "../../include/dcq_probe.h"

namespace {

template <int U>
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
    const int64_t per_wg = (int64_t)256 * U;
    uint32_t acc = 0;
    for (int64_t base = (int64_t)blockIdx.x * per_wg; base < n16; base += (int64_t)gridDim.x * per_wg) {
        uint4 v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t i = base + (int64_t)j * 256 + threadIdx.x;
            v[j] = i < n16 ? src[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

extern "C" int dcq_probe_stream_read(const void* src, size_t bytes, int per_lane, int max_workgroups, uint32_t* sink,
                                     void* stream) {
    if (!src || !sink || bytes == 0) return -1;
    if (bytes % 16 || (uintptr_t)src % 16 || (uintptr_t)sink % 4) return -4;
    if (per_lane != 1 && per_lane != 2 && per_lane != 4 && per_lane != 8 && per_lane != 16) return -1;
    const int64_t n16 = (int64_t)(bytes / 16);
    int64_t grid = (n16 + 256 * per_lane - 1) / (256 * per_lane);
    if (max_workgroups > 0 && grid > max_workgroups) grid = max_workgroups;
    if (grid > INT32_MAX) return -3;
    hipStream_t st = (hipStream_t)stream;
    const uint4* s = (const uint4*)src;
    switch (per_lane) {
        case 1: hipLaunchKernelGGL(stream_read_kernel<1>, dim3((unsigned)grid), dim3(256), 0, st, s, n16, sink); break;
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3((unsigned)grid), dim3(256), 0, st, s, n16, sink); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3((unsigned)grid), dim3(256), 0, st, s, n16, sink); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3((unsigned)grid), dim3(256), 0, st, s, n16, sink); break;
        default: hipLaunchKernelGGL(stream_read_kernel<16>, dim3((unsigned)grid), dim3(256), 0, st, s, n16, sink); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -6;
}
