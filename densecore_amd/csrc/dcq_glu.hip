// dcq_glu.hip — elementwise epilogues of the projections when no fused decode kernel covers the
// shape: the SwiGLU product Y = silu(Y) * U, and the residual / bias add Y = T + R.
//
// The reference FFN multiplies silu(w1 x) by (w3 x) elementwise (core/src/inference.cpp:1796,
// ggml_mul of ggml_silu). When the fused gate/up decode kernels do not cover a shape, the two
// projections run as mul_mat launches into Y and a workspace U, and this kernel applies the
// product in place. HBM-bound: 12 bytes per element.
#include "dcq_common.h"
#include "dcq_kernels.h"

namespace dcq {

__global__ void __launch_bounds__(256) silu_mul_kernel(float* __restrict__ Y, int64_t y_stride,
                                                       const float* __restrict__ U, int64_t u_stride, int64_t M,
                                                       int64_t N) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= N || m >= M) return;
    float* y = Y + m * y_stride + n;
    *y = silu(*y) * U[m * u_stride + n];
}

hipError_t launch_silu_mul(float* Y, int64_t y_stride, const float* U, int64_t u_stride, int64_t M, int64_t N,
                           hipStream_t st) {
    if (M > 65535) {  // one grid row per activation row
        for (int64_t m0 = 0; m0 < M; m0 += 65535) {
            const int64_t mc = M - m0 < 65535 ? M - m0 : 65535;
            const hipError_t e = launch_silu_mul(Y + m0 * y_stride, y_stride, U + m0 * u_stride, u_stride, mc, N, st);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
    hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, st, Y, y_stride, U, u_stride, M, N);
    return hipGetLastError();
}

// Y = T + R, one fp32 add per element (the reference's ggml_add of a projection and its residual
// or bias, core/src/inference.cpp:1135-1151, 1761-1764, 1800). r_stride 0 broadcasts one bias row.
// T may be Y itself; each element is read and written by the same lane. HBM-bound: 12 bytes per
// element.
__global__ void __launch_bounds__(256) add_rows_kernel(float* Y, int64_t y_stride, const float* T, int64_t t_stride,
                                                       const float* R, int64_t r_stride, int64_t M, int64_t N) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= N || m >= M) return;
    Y[m * y_stride + n] = T[m * t_stride + n] + R[m * r_stride + n];
}

hipError_t launch_add_rows(float* Y, int64_t y_stride, const float* T, int64_t t_stride, const float* R,
                           int64_t r_stride, int64_t M, int64_t N, hipStream_t st) {
    for (int64_t m0 = 0; m0 < M; m0 += 65535) {  // one grid row per activation row
        const int64_t mc = M - m0 < 65535 ? M - m0 : 65535;
        dim3 grid((unsigned)((N + 255) / 256), (unsigned)mc);
        hipLaunchKernelGGL(add_rows_kernel, grid, dim3(256), 0, st, Y + m0 * y_stride, y_stride, T + m0 * t_stride,
                           t_stride, R + m0 * r_stride, r_stride, mc, N);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace dcq
