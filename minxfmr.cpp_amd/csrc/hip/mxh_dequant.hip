// mxh_dequant.hip — GGUF block -> fp32 decode on the device.
//
// Bit-exact with the reference CPU decoders (src/tensor/tensor.cpp:405-457):
// every product is exact in fp32 (fp16 d x 6-bit scale x 4/5-bit code needs at
// most 22 significant bits), so only the final subtraction rounds and fused
// or separate multiply-add give the same bits.  One thread writes one run of
// 32 consecutive outputs.
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {
namespace {

__device__ __forceinline__ uint32_t rd_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

template <int TYPE>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out, int64_t rows, int64_t cols,
                               int form) {
    const int64_t runs_per_row = cols / 32;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * runs_per_row) return;
    const int64_t row = t / runs_per_row, run = t % runs_per_row;
    float* y = out + row * cols + run * 32;
    const size_t rb = row_bytes(TYPE, cols);
    const uint8_t* rp = w + (size_t)row * rb;
    if constexpr (TYPE == MXH_Q4_K || TYPE == MXH_Q5_K) {
        constexpr int BB = TYPE == MXH_Q4_K ? 144 : 176;
        const int64_t b = run >> 3;
        const int j = (int)(run & 7);  // sub-block: elements 32j..32j+31
        const uint8_t* blk = rp + (size_t)b * BB;
        const float d = half_bits_to_float(rd_u16(blk));
        const float dm = half_bits_to_float(rd_u16(blk + 2));
        const uint32_t s0 = rd_u16(blk + 4) | (rd_u16(blk + 6) << 16);
        const uint32_t s1 = rd_u16(blk + 8) | (rd_u16(blk + 10) << 16);
        const uint32_t s2 = rd_u16(blk + 12) | (rd_u16(blk + 14) << 16);
        uint32_t sc, mn;
        k4_scale_min(s0, s1, s2, j, form, sc, mn);
        const float ds = d * (float)sc, ms = dm * (float)mn;
        const int g = j >> 1, hi = j & 1;
        const uint8_t* qs = blk + (TYPE == MXH_Q4_K ? 16 : 48) + 32 * g;
        for (int i = 0; i < 32; ++i) {
            uint32_t q = rd_u8(qs + i);
            q = hi ? (q >> 4) : (q & 15u);
            if constexpr (TYPE == MXH_Q5_K) q |= ((rd_u8(blk + 16 + i) >> j) & 1u) << 4;
            y[i] = ds * (float)q - ms;
        }
    } else if constexpr (TYPE == MXH_Q8_0) {
        const uint8_t* blk = rp + (size_t)run * 34;
        const float d = half_bits_to_float(rd_u16(blk));
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int)(int8_t)blk[2 + i];
    } else if constexpr (TYPE == MXH_Q5_0) {
        const uint8_t* blk = rp + (size_t)run * 22;
        const float d = half_bits_to_float(rd_u16(blk));
        const uint32_t qh = rd_u16(blk + 2) | (rd_u16(blk + 4) << 16);
        for (int i = 0; i < 16; ++i) {
            const uint32_t ql = blk[6 + i];
            const int a = (int)((ql & 15u) | (((qh >> i) & 1u) << 4));
            const int c = (int)((ql >> 4) | (((qh >> (i + 16)) & 1u) << 4));
            y[i] = d * (float)(a - 16);
            y[i + 16] = d * (float)(c - 16);
        }
    } else if constexpr (TYPE == MXH_F16) {
        for (int i = 0; i < 32; ++i) y[i] = half_bits_to_float(rd_u16(rp + 2 * (run * 32 + i)));
    } else {
        const float* src = reinterpret_cast<const float*>(rp) + run * 32;
        for (int i = 0; i < 32; ++i) y[i] = src[i];
    }
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
    case MXH_F16: launch<MXH_F16>(w, out, rows, cols, form, st); break;
    case MXH_F32: launch<MXH_F32>(w, out, rows, cols, form, st); break;
    default: return MXH_ERR_UNSUPPORTED;
    }
    return MXH_OK;
}

}  // namespace mxh
