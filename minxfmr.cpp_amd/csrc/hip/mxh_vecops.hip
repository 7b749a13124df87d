// mxh_vecops.hip — small F32 vector ops behind the per-op backend interface.
//
// Reference semantics (src/backend/cpu/cpu_backend.cpp:325-393): dot products
// and column sums accumulate in double and round to float once; these kernels
// keep that (fp64 is cheap at these sizes and removes an accuracy gap).
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {
namespace {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// one wave per output row; ring addressing (head + j) % seq_max
__global__ void vec_dot_rows_kernel(const float* __restrict__ vec, const float* __restrict__ rows,
                                    float* __restrict__ out, int64_t K, int64_t nrows, int64_t stride, int64_t head,
                                    int64_t seq_max) {
    const int lane = threadIdx.x & 63;
    const int64_t j = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (j >= nrows) return;
    const float* r = rows + ((head + j) % seq_max) * stride;
    double acc = 0.0;
    for (int64_t k = lane; k < K; k += 64) acc += (double)vec[k] * (double)r[k];
    acc = wave_sum_d(acc);
    if (lane == 0) out[j] = (float)acc;
}

__global__ void vec_mul_rows_cols_kernel(const float* __restrict__ vec, const float* __restrict__ rows,
                                         float* __restrict__ out, int64_t nrows, int64_t ncols, int64_t stride) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= ncols) return;
    double acc = 0.0;
    for (int64_t r = 0; r < nrows; ++r) acc += (double)vec[r] * (double)rows[r * stride + c];
    out[c] = (float)acc;
}

__global__ void matmul_f32_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                                  int64_t m, int64_t k, int64_t n) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t i = blockIdx.y;
    if (j >= n || i >= m) return;
    float acc = 0.f;
    for (int64_t t = 0; t < k; ++t) acc = fmaf(a[i * k + t], b[t * n + j], acc);
    out[i * n + j] = acc;
}

}  // namespace

int vec_dot_rows_launch(const float* vec, const float* rows, float* out, int64_t K, int64_t nrows, int64_t stride,
                        int64_t head, int64_t seq_max, hipStream_t st) {
    if (K <= 0 || nrows <= 0 || seq_max <= 0) return MXH_ERR_ARG;
    const unsigned grid = (unsigned)((nrows + 3) / 4);
    hipLaunchKernelGGL(vec_dot_rows_kernel, dim3(grid), dim3(256), 0, st, vec, rows, out, K, nrows, stride, head,
                       seq_max);
    return MXH_OK;
}

int vec_mul_rows_cols_launch(const float* vec, const float* rows, float* out, int64_t nrows, int64_t ncols,
                             int64_t stride, hipStream_t st) {
    if (nrows <= 0 || ncols <= 0) return MXH_ERR_ARG;
    hipLaunchKernelGGL(vec_mul_rows_cols_kernel, dim3((unsigned)((ncols + 255) / 256)), dim3(256), 0, st, vec, rows,
                       out, nrows, ncols, stride);
    return MXH_OK;
}

int matmul_f32_launch(const float* a, const float* b, float* out, int64_t m, int64_t k, int64_t n, hipStream_t st) {
    if (m <= 0 || k <= 0 || n <= 0 || m > 65535) return MXH_ERR_ARG;
    hipLaunchKernelGGL(matmul_f32_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)m), dim3(256), 0, st, a, b,
                       out, m, k, n);
    return MXH_OK;
}

}  // namespace mxh
