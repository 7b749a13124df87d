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

// 6-bit (scale, min) of sub-blocks 2g and 2g+1 as byte pairs, without
// branches (tensor.cpp:395-403 reference form; ggml form for form != 0)
__device__ __forceinline__ void k4_pair(uint32_t s0, uint32_t s1, uint32_t s2, int g, int form, uint32_t& sc,
                                        uint32_t& mn) {
    const int sh = (g & 1) * 16;
    const uint32_t A = s0 >> sh, B = s1 >> sh, C = s2 >> sh;
    if (g >= 2) {
        sc = (C & 0x0f0fu) | (((form ? A : B) >> 2) & 0x3030u);
        mn = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    } else {
        sc = A & 0x3f3fu;
        mn = B & 0x3f3fu;
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

// Wave64 sum with DPP row operations; the total lands in lane 63
// (quad swaps, half-row and row mirrors, then row broadcasts 15 and 31).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp_f<0xb1>(v);        // quad_perm [1,0,3,2]
    v += dpp_f<0x4e>(v);        // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);       // row_half_mirror
    v += dpp_f<0x140>(v);       // row_mirror
    v += dpp_f<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// DPP reductions inside groups of 4 / 8 lanes and across the wave (double).
__device__ __forceinline__ float max8_dpp(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4e>(v));   // quad_perm [2,3,0,1]
    return fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror: the other quad of the 8
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

__device__ __forceinline__ int sum4_dpp(int v) {
    v += dpp_i<0xb1>(v);
    return v + dpp_i<0x4e>(v);
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROW_MASK, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// wave sum of doubles; the total lands in lane 63
__device__ __forceinline__ double wave_sum_d_lane63(double v) {
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    v += dpp_d<0x142, 0xa>(v);
    v += dpp_d<0x143, 0xc>(v);
    return v;
}

// sum over a 16-lane row (quad swaps, half-row and row mirrors); every lane
// of the row ends with the row sum
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xb1>(v);
    v += dpp_f<0x4e>(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

// wave-wide sum / max broadcast to every lane
// v of lane (lane ^ OFF) within the wave, OFF in {4, 8, 16, 32}: VALU lane
// swaps for 16 and 32 (v_permlane16/32_swap: the first result holds, for the
// odd rows / upper half, the swapped-in values, the second for the others),
// a row rotation for 8
template <int OFF>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (OFF == 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((threadIdx.x & 32) ? p[0] : p[1]);
    } else if constexpr (OFF == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((threadIdx.x & 16) ? p[0] : p[1]);
    } else if constexpr (OFF == 8) {
        return dpp_f<0x128>(v);  // row_ror:8 (i + 8 mod 16 == i ^ 8)
    } else {
        return __shfl_xor(v, OFF, 64);
    }
}

__device__ __forceinline__ float wave_sum_all(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_lane63(v)), 63));
}

__device__ __forceinline__ float wave_max_all(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));
    v = fmaxf(v, dpp_f<0x4e>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    // rows: broadcast lane 15 / 31 maxima upward, then read lane 63
    const float b15 = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), 0x142, 0xa, 0xf, false));
    v = fmaxf(v, b15);
    const float b31 = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), 0x143, 0xc, 0xf, false));
    v = fmaxf(v, b31);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ double wave_sum_d_all(double v) {
    v = wave_sum_d_lane63(v);
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, 63), hi = __builtin_amdgcn_readlane((int)(b >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// 16-byte load through a buffer descriptor over [base, base + bytes) with
// the default cache policy; offsets at or past `bytes` read 0 without a
// branch, so a run of such loads keeps a fixed count for s_waitcnt
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld_buf16(__amdgpu_buffer_rsrc_t r, int byte_off) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace mxh
