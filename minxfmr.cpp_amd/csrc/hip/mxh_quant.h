// mxh_quant.h — device decode of one 32-element run of a GGUF row.
//
// Bit-exact with the reference CPU decoders (src/tensor/tensor.cpp:405-457):
// every product is exact in fp32 (fp16 d x 6-bit scale x 4/5-bit code needs at
// most 22 significant bits), so only the final subtraction rounds and fused
// or separate multiply-add give the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxh_device.h"
#include "mxh_types.h"

namespace mxh {

__device__ __forceinline__ uint32_t rd_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// y[0..31] = elements 32*run .. 32*run+31 of the row starting at rp; the
// tiled layouts also need the row's block count
template <int TYPE>
__device__ __forceinline__ void dequant_run32(const uint8_t* __restrict__ rp, int64_t run, int form, float* y,
                                              int64_t row_blocks = 0) {
    if constexpr (TYPE == MXH_Q4_K_TILED) {
        const int j = (int)(run & 7);
        const Q4KTileOffs o = q4k_tile_offsets((run >> 3) * 4 + (j >> 1), row_blocks);
        const uint8_t* hd = rp + o.hd;
        uint32_t sc, mn;
        k4_scale_min(rd_u16(hd + 4) | (rd_u16(hd + 6) << 16), rd_u16(hd + 8) | (rd_u16(hd + 10) << 16),
                     rd_u16(hd + 12) | (rd_u16(hd + 14) << 16), j, form, sc, mn);
        const float ds = half_bits_to_float(rd_u16(hd)) * (float)sc, ms = half_bits_to_float(rd_u16(hd + 2)) * (float)mn;
        const int hi = j & 1;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            uint32_t q = rd_u8(rp + (i < 16 ? o.qa + i : o.qb + i - 16));
            q = hi ? (q >> 4) : (q & 15u);
            y[i] = ds * (float)q - ms;
        }
    } else if constexpr (TYPE == MXH_Q5_K_TILED) {
        const int j = (int)(run & 7);  // sub-block: the low (even j) or high nibbles of 64-group j/2
        const Q5KTileOffs o = q5k_tile_offsets((run >> 3) * 8 + 2 * (j >> 1), row_blocks);
        const uint8_t* hd = rp + o.hd;
        uint32_t sc, mn;
        k4_scale_min(rd_u16(hd + 4) | (rd_u16(hd + 6) << 16), rd_u16(hd + 8) | (rd_u16(hd + 10) << 16),
                     rd_u16(hd + 12) | (rd_u16(hd + 14) << 16), j, form, sc, mn);
        const float ds = half_bits_to_float(rd_u16(hd)) * (float)sc, ms = half_bits_to_float(rd_u16(hd + 2)) * (float)mn;
        const int hi = j & 1;
        const uint8_t* qs = rp + o.qs;  // the group's 32 qs bytes: chunks 2g and 2g+1, adjacent
        const uint8_t* qh = rp + o.qh;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            uint32_t q = rd_u8(qs + i);
            q = hi ? (q >> 4) : (q & 15u);
            q |= ((rd_u8(qh + i) >> j) & 1u) << 4;
            y[i] = ds * (float)q - ms;
        }
    } else if constexpr (TYPE == MXH_Q6_K || TYPE == MXH_Q6_K_TILED) {
        // run r of block b: elements 128 h + 32 g + i (i < 32) with h = r / 4,
        // g = r % 4; the code of i comes from ql byte 64 h + 32 (g & 1) + i
        // (low nibble for g < 2) and the 2-bit field g of qh byte 32 h + i,
        // minus 32; value (d * sc) * q with sc = scales[8 h + 2 g + i / 16]
        // (gguf_reader.cpp:905-1008, the reference's load-time conversion)
        const int64_t b = run >> 3;
        const int r = (int)(run & 7), h = r >> 2, g = r & 3;
        const uint8_t *ql0, *ql1, *qh0, *qh1, *sc;
        float d;
        if constexpr (TYPE == MXH_Q6_K) {
            const uint8_t* blk = rp + (size_t)b * 210;
            ql0 = blk + 64 * h + 32 * (g & 1);
            ql1 = ql0 + 16;
            qh0 = blk + 128 + 32 * h;
            qh1 = qh0 + 16;
            sc = blk + 192;
            d = half_bits_to_float(rd_u16(blk + 208));
        } else {
            // elements i < 16 lie in chunk 4 b + 2 h, the rest in chunk + 1
            const Q6KTileOffs o0 = q6k_tile_offsets(4 * b + 2 * h, row_blocks);
            const Q6KTileOffs o1 = q6k_tile_offsets(4 * b + 2 * h + 1, row_blocks);
            ql0 = rp + ((g & 1) ? o0.qb : o0.qa);
            ql1 = rp + ((g & 1) ? o1.qb : o1.qa);
            qh0 = rp + o0.qh;
            qh1 = rp + o1.qh;
            sc = rp + o0.sc;
            d = half_bits_to_float(rd_u16(rp + o0.d));
        }
        const int nib = (g >> 1) * 4, hs = 2 * g;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            const uint32_t lq = rd_u8(i < 16 ? ql0 + i : ql1 + i - 16);
            const uint32_t hq = rd_u8(i < 16 ? qh0 + i : qh1 + i - 16);
            const int q = (int)(((lq >> nib) & 15u) | (((hq >> hs) & 3u) << 4)) - 32;
            y[i] = d * (float)(int)(int8_t)sc[8 * h + 2 * g + (i >> 4)] * (float)q;
        }
    } else if constexpr (TYPE == MXH_Q8_0_TILED) {
        const Q80TileOffs o = q80_tile_offsets(run, row_blocks);
        const float d = half_bits_to_float(rd_u16(rp + o.d));
#pragma unroll 8
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int)(int8_t)rp[i < 16 ? o.lo + i : o.hi + i - 16];
    } else if constexpr (TYPE == MXH_Q4_K || TYPE == MXH_Q5_K) {
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
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            uint32_t q = rd_u8(qs + i);
            q = hi ? (q >> 4) : (q & 15u);
            if constexpr (TYPE == MXH_Q5_K) q |= ((rd_u8(blk + 16 + i) >> j) & 1u) << 4;
            y[i] = ds * (float)q - ms;
        }
    } else if constexpr (TYPE == MXH_Q8_0) {
        const uint8_t* blk = rp + (size_t)run * 34;
        const float d = half_bits_to_float(rd_u16(blk));
#pragma unroll 8
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int)(int8_t)blk[2 + i];
    } else if constexpr (TYPE == MXH_Q5_0) {
        const uint8_t* blk = rp + (size_t)run * 22;
        const float d = half_bits_to_float(rd_u16(blk));
        const uint32_t qh = rd_u16(blk + 2) | (rd_u16(blk + 4) << 16);
#pragma unroll 8
        for (int i = 0; i < 16; ++i) {
            const uint32_t ql = blk[6 + i];
            const int a = (int)((ql & 15u) | (((qh >> i) & 1u) << 4));
            const int c = (int)((ql >> 4) | (((qh >> (i + 16)) & 1u) << 4));
            y[i] = d * (float)(a - 16);
            y[i + 16] = d * (float)(c - 16);
        }
    } else if constexpr (TYPE == MXH_F16) {
#pragma unroll 8
        for (int i = 0; i < 32; ++i) y[i] = half_bits_to_float(rd_u16(rp + 2 * (run * 32 + i)));
    } else {
        const float* src = reinterpret_cast<const float*>(rp) + run * 32;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) y[i] = src[i];
    }
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const __bf16 b = (__bf16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

}  // namespace mxh
