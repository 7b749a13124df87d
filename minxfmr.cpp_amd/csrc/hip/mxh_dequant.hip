// mxh_dequant.hip — GGUF block -> fp32 decode on the device, bit-exact with
// the reference CPU decoders (src/tensor/tensor.cpp:405-457) and with its
// load-time F16 / Q6_K conversions (third_party/gguf/gguf_reader.cpp:759-785,
// :905-1008; see mxh_quant.h).  One thread writes one run of 32 consecutive outputs.
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"
#include "mxh_quant.h"

namespace mxh {
namespace {

template <int TYPE>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out, int64_t rows, int64_t cols,
                               int form) {
    const int64_t runs_per_row = cols / 32;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * runs_per_row) return;
    const int64_t row = t / runs_per_row, run = t % runs_per_row;
    float y[32];
    dequant_run32<TYPE>(w + (size_t)row * row_bytes(TYPE, cols), run, form, y);
    float* o = out + row * cols + run * 32;
#pragma unroll
    for (int i = 0; i < 32; ++i) o[i] = y[i];
}

template <int TYPE>
void launch(const void* w, float* out, int64_t rows, int64_t cols, int form, hipStream_t st) {
    const int64_t threads = rows * (cols / 32);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(dequant_kernel<TYPE>, dim3(grid), dim3(256), 0, st, (const uint8_t*)w, out, rows, cols, form);
}

}  // namespace

int dequant_launch(int type, const void* w, float* out, int64_t rows, int64_t cols, int form, hipStream_t st) {
    if (rows <= 0 || cols <= 0 || cols % 32 || row_bytes(type, cols) == 0) return MXH_ERR_ARG;
    switch (type) {
    case MXH_Q4_K: launch<MXH_Q4_K>(w, out, rows, cols, form, st); break;
    case MXH_Q5_K: launch<MXH_Q5_K>(w, out, rows, cols, form, st); break;
    case MXH_Q8_0: launch<MXH_Q8_0>(w, out, rows, cols, form, st); break;
    case MXH_Q5_0: launch<MXH_Q5_0>(w, out, rows, cols, form, st); break;
    case MXH_Q6_K: launch<MXH_Q6_K>(w, out, rows, cols, form, st); break;
    case MXH_F16: launch<MXH_F16>(w, out, rows, cols, form, st); break;
    case MXH_F32: launch<MXH_F32>(w, out, rows, cols, form, st); break;
    default: return MXH_ERR_UNSUPPORTED;
    }
    return MXH_OK;
}

}  // namespace mxh
