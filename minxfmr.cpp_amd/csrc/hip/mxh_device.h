// mxh_device.h — device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxh_types.h"

namespace mxh {

// binary16 -> binary32 on integer ALUs so NaN payloads and subnormals give the
// same bits as the host decoder the weights are checked against
// (reference: src/tensor/tensor.cpp:366-393).
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t s = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    uint32_t f = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = s | 0x7f800000u | (f << 13);
    } else if (e != 0u) {
        bits = s | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0u) {
        bits = s;
    } else {
        // f * 2^-24 with f in [1, 1023]: leading one at bit (31 - clz)
        const int lead = 31 - __clz((int)f);
        const uint32_t mant = (f << (10 - lead)) & 1023u;
        bits = s | ((uint32_t)(103 + lead) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

// byte `j` (0..11) of the 12-byte K-quant scale field held in three dwords
__device__ __forceinline__ uint32_t scale_byte(uint32_t s0, uint32_t s1, uint32_t s2, int j) {
    const uint32_t w = j < 4 ? s0 : (j < 8 ? s1 : s2);
    return (w >> (8 * (j & 3))) & 0xffu;
}

// 6-bit (scale, min) of sub-block j (0..7).  form 0: reference CPU decoder
// (tensor.cpp:395-403, top bits of both from byte j); form 1: ggml decoder
// (scale's top bits from byte j-4).
__device__ __forceinline__ void k4_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int form,
                                             uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = scale_byte(s0, s1, s2, j) & 63u;
        mn = scale_byte(s0, s1, s2, j + 4) & 63u;
    } else {
        const uint32_t lo = scale_byte(s0, s1, s2, j + 4);
        const uint32_t hm = scale_byte(s0, s1, s2, j) >> 6;
        const uint32_t hs = form ? (scale_byte(s0, s1, s2, j - 4) >> 6) : hm;
        sc = (lo & 15u) | (hs << 4);
        mn = (lo >> 4) | (hm << 4);
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

}  // namespace mxh
