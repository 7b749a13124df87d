// mxh_repack.hip — in-place regrouping of device weight rows into the tiled
// layouts of mxh_types.h (q4k_tile_offsets, q5k_tile_offsets, q6k_tile_offsets,
// q80_tile_offsets).
//
// A GGUF Q4_K row interleaves 16 header bytes and 128 quant bytes per block,
// so the 16-byte loads of one wave instruction (one 64-element chunk per
// lane) touch every cache line of the row three times over.  The tiled row
// holds the same bytes grouped so that each such instruction reads whole,
// contiguous lines.  Only device copies the model owns are tiled; the
// arithmetic on the bytes is unchanged, so results are identical.
#include <hip/hip_runtime.h>

#include "mxh_internal.h"
#include "mxh_types.h"

namespace mxh {

namespace {

__device__ __forceinline__ uint4 lds_u16x8(const uint8_t* p) {  // 2-aligned 16 bytes
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16), h[4] | ((uint32_t)h[5] << 16),
                      h[6] | ((uint32_t)h[7] << 16));
}

// Workgroup r' takes rows r', r' + grid, ...: the row is copied to LDS, then
// written back in tiled order.
template <int TYPE>
__global__ __launch_bounds__(256) void tile_rows_kernel(uint8_t* __restrict__ w, int64_t rows, int nblocks) {
    extern __shared__ __align__(16) uint8_t row_buf[];
    constexpr int BB = TYPE == MXH_Q4_K ? 144 : TYPE == MXH_Q5_K ? 176 : TYPE == MXH_Q6_K ? 210 : 34;
    const size_t rb = (size_t)nblocks * BB;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        uint8_t* rp = w + (size_t)r * rb;
        for (size_t i = threadIdx.x; i < rb / 16; i += blockDim.x)
            reinterpret_cast<uint4*>(row_buf)[i] = reinterpret_cast<const uint4*>(rp)[i];
        __syncthreads();
        if constexpr (TYPE == MXH_Q4_K) {
            for (int c = threadIdx.x; c < 4 * nblocks; c += blockDim.x) {
                const Q4KTileOffs o = q4k_tile_offsets(c, nblocks);
                const uint8_t* src = row_buf + (size_t)(c >> 2) * 144;
                const int g = c & 3;
                if (g == 0) *reinterpret_cast<uint4*>(rp + o.hd) = *reinterpret_cast<const uint4*>(src);
                *reinterpret_cast<uint4*>(rp + o.qa) = *reinterpret_cast<const uint4*>(src + 16 + 32 * g);
                *reinterpret_cast<uint4*>(rp + o.qb) = *reinterpret_cast<const uint4*>(src + 32 + 32 * g);
            }
        } else if constexpr (TYPE == MXH_Q5_K) {
            for (int c = threadIdx.x; c < 8 * nblocks; c += blockDim.x) {
                const Q5KTileOffs o = q5k_tile_offsets(c, nblocks);
                const uint8_t* src = row_buf + (size_t)(c >> 3) * 176;
                const int p = c & 7;
                if (p == 0) {
                    *reinterpret_cast<uint4*>(rp + o.hd) = *reinterpret_cast<const uint4*>(src);
                    *reinterpret_cast<uint4*>(rp + o.qh) = *reinterpret_cast<const uint4*>(src + 16);
                    *reinterpret_cast<uint4*>(rp + o.qh + 16) = *reinterpret_cast<const uint4*>(src + 32);
                }
                *reinterpret_cast<uint4*>(rp + o.qs) = *reinterpret_cast<const uint4*>(src + 48 + 16 * p);
            }
        } else if constexpr (TYPE == MXH_Q6_K) {
            // 210-byte blocks are 2-aligned in the LDS copy: 16-bit reads
            for (int c = threadIdx.x; c < 4 * nblocks; c += blockDim.x) {
                const Q6KTileOffs o = q6k_tile_offsets(c, nblocks);
                const uint8_t* src = row_buf + (size_t)(c >> 2) * 210;
                const int h = (c >> 1) & 1, p = c & 1;
                *reinterpret_cast<uint4*>(rp + o.qa) = lds_u16x8(src + 64 * h + 16 * p);
                *reinterpret_cast<uint4*>(rp + o.qb) = lds_u16x8(src + 64 * h + 32 + 16 * p);
                *reinterpret_cast<uint4*>(rp + o.qh) = lds_u16x8(src + 128 + 32 * h + 16 * p);
                if ((c & 3) == 0) {
                    *reinterpret_cast<uint4*>(rp + o.sc) = lds_u16x8(src + 192);
                    *reinterpret_cast<uint16_t*>(rp + o.d) = *reinterpret_cast<const uint16_t*>(src + 208);
                }
            }
        } else {
            for (int b = threadIdx.x; b < nblocks; b += blockDim.x) {
                const Q80TileOffs o = q80_tile_offsets(b, nblocks);
                const uint8_t* src = row_buf + (size_t)b * 34;
                *reinterpret_cast<uint4*>(rp + o.lo) = lds_u16x8(src + 2);
                *reinterpret_cast<uint4*>(rp + o.hi) = lds_u16x8(src + 18);
                *reinterpret_cast<uint16_t*>(rp + o.d) = *reinterpret_cast<const uint16_t*>(src);
            }
        }
        __syncthreads();
    }
}

}  // namespace

int tiled_type(int type, int64_t cols) {
    // rows up to the GEMV's largest K (one row is staged in LDS); Q8_0 rows
    // are 16-byte aligned, as the tiled loads need, when K is a multiple of 256
    if (type == MXH_Q4_K && cols % 256 == 0 && cols <= 15360) return MXH_Q4_K_TILED;
    if (type == MXH_Q8_0 && cols % 256 == 0 && cols <= 15360) return MXH_Q8_0_TILED;
    if (type == MXH_Q5_K && cols % 256 == 0 && cols <= 15360) return MXH_Q5_K_TILED;
    // 210-byte blocks: rows stay 16-byte aligned when K is a multiple of 2048
    if (type == MXH_Q6_K && cols % 2048 == 0 && cols <= 15360) return MXH_Q6_K_TILED;
    return type;
}

int tile_rows_launch(int type, void* w, int64_t rows, int64_t cols, hipStream_t st) {
    if (tiled_type(type, cols) == type || rows <= 0 || ((uintptr_t)w & 15)) return MXH_ERR_ARG;
    const int nblocks = (int)(cols / block_geom(type).elems);
    const size_t lds = row_bytes(type, cols);
    const unsigned grid = (unsigned)(rows < 4096 ? rows : 4096);
    if (type == MXH_Q4_K)
        hipLaunchKernelGGL(tile_rows_kernel<MXH_Q4_K>, dim3(grid), dim3(256), lds, st, (uint8_t*)w, rows, nblocks);
    else if (type == MXH_Q5_K)
        hipLaunchKernelGGL(tile_rows_kernel<MXH_Q5_K>, dim3(grid), dim3(256), lds, st, (uint8_t*)w, rows, nblocks);
    else if (type == MXH_Q6_K)
        hipLaunchKernelGGL(tile_rows_kernel<MXH_Q6_K>, dim3(grid), dim3(256), lds, st, (uint8_t*)w, rows, nblocks);
    else
        hipLaunchKernelGGL(tile_rows_kernel<MXH_Q8_0>, dim3(grid), dim3(256), lds, st, (uint8_t*)w, rows, nblocks);
    return hipGetLastError() == hipSuccess ? MXH_OK : MXH_ERR_HIP;
}

}  // namespace mxh
