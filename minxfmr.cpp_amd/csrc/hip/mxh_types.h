// mxh_types.h — tensor element types and block geometry (host + device).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "minxfmr_hip.h"

namespace mxh {

// Block geometry of the GGUF formats (reference: src/tensor/tensor.h:61-73;
// Q5_K is the published ggml layout, absent from the reference).
struct BlockGeom {
    int elems;
    int bytes;
};

// Device-resident layouts that no GGUF file holds: the blocks of each row
// regrouped in tiles so that the 16-byte loads of one wave instruction read
// whole cache lines (see q4k_tile_offsets / q80_tile_offsets).  A row keeps
// the byte count of its GGUF type.  The C ABI takes these ids only in
// mxh_gemv, for rows that mxh_tile_rows regrouped (MXH_TILED_FLAG == kTiledFlag).
constexpr int kTiledFlag = 0x100;
constexpr int MXH_Q4_K_TILED = kTiledFlag | MXH_Q4_K;
constexpr int MXH_Q8_0_TILED = kTiledFlag | MXH_Q8_0;
constexpr int MXH_Q5_K_TILED = kTiledFlag | MXH_Q5_K;
constexpr int MXH_Q6_K_TILED = kTiledFlag | MXH_Q6_K;

__host__ __device__ constexpr int storage_type(int type) { return type & (kTiledFlag - 1); }

__host__ __device__ constexpr BlockGeom block_geom(int t) {
    const int type =
        t == MXH_Q4_K_TILED || t == MXH_Q8_0_TILED || t == MXH_Q5_K_TILED || t == MXH_Q6_K_TILED ? storage_type(t) : t;
    return type == MXH_Q4_K   ? BlockGeom{256, 144}
           : type == MXH_Q5_K ? BlockGeom{256, 176}
           : type == MXH_Q6_K ? BlockGeom{256, 210}
           : type == MXH_Q8_0 ? BlockGeom{32, 34}
           : type == MXH_Q5_0 ? BlockGeom{32, 22}
           : type == MXH_F16  ? BlockGeom{1, 2}
           : type == MXH_F32  ? BlockGeom{1, 4}
                              : BlockGeom{0, 0};
}

__host__ __device__ constexpr size_t row_bytes(int type, int64_t cols) {
    return block_geom(type).elems == 0 || cols % block_geom(type).elems
               ? 0
               : (size_t)(cols / block_geom(type).elems) * (size_t)block_geom(type).bytes;
}

// Q4_K tiles of 16 blocks (4096 elements, 2304 bytes; the last tile of a row
// may hold fewer, nb): the nb 16-byte block headers (d, dmin, scales), then
// for each 64-element chunk l = 4 b + g of the tile (block b, group g) the
// first 16 qs bytes of the group, then for each chunk the last 16.  Lane l
// of a wave reading chunk l thus reads line-contiguous 16-byte pieces.
struct Q4KTileOffs {
    uint32_t hd, qa, qb;
};
__host__ __device__ constexpr Q4KTileOffs q4k_tile_offsets(int64_t chunk, int64_t nblocks) {
    const int64_t j = chunk >> 6, l = chunk & 63;
    const int64_t nb = nblocks - 16 * j < 16 ? nblocks - 16 * j : 16;
    const uint32_t base = (uint32_t)(j * 2304);
    return Q4KTileOffs{base + 16u * (uint32_t)(l >> 2), base + 16u * (uint32_t)(nb + l),
                       base + 16u * (uint32_t)(5 * nb + l)};
}

// Q5_K tiles of 8 blocks (64 chunks of 32 elements, 1408 bytes; the last may
// hold fewer, nb): the nb 16-byte headers, the nb 32-byte high-bit planes
// (qh), then for each 32-element chunk l = 8 b + p the 16 qs bytes it reads
// (qs bytes 16p..16p+15 of block b).
struct Q5KTileOffs {
    uint32_t hd, qh, qs;
};
__host__ __device__ constexpr Q5KTileOffs q5k_tile_offsets(int64_t chunk, int64_t nblocks) {
    const int64_t j = chunk >> 6, l = chunk & 63;
    const int64_t nb = nblocks - 8 * j < 8 ? nblocks - 8 * j : 8;
    const uint32_t base = (uint32_t)(j * 1408);
    return Q5KTileOffs{base + 16u * (uint32_t)(l >> 3), base + 16u * (uint32_t)nb + 32u * (uint32_t)(l >> 3),
                       base + 16u * (uint32_t)(3 * nb + l)};
}

// Q8_0 tiles of 64 blocks (2176 bytes; the last may hold fewer, nb): the
// first 16 quant bytes of each block, then the last 16, then the nb fp16
// scales.
struct Q80TileOffs {
    uint32_t lo, hi, d;
};
__host__ __device__ constexpr Q80TileOffs q80_tile_offsets(int64_t block, int64_t nblocks) {
    const int64_t j = block >> 6, l = block & 63;
    const int64_t nb = nblocks - 64 * j < 64 ? nblocks - 64 * j : 64;
    const uint32_t base = (uint32_t)(j * 2176);
    return Q80TileOffs{base + 16u * (uint32_t)l, base + 16u * (uint32_t)(nb + l), base + (uint32_t)(32 * nb + 2 * l)};
}

// Q6_K (ql[128], qh[64], int8 scales[16], fp16 d; 210 bytes per 256
// elements).  The GEMV takes a block in four 64-element chunks
// c = 4 b + 2 h + p (half h, run p): for l in [16 p, 16 p + 16) the elements
// 128 h + l + 32 g, g = 0..3, whose 6-bit codes come from the 16 ql bytes
// 64 h + 16 p.. (g = 0: low nibbles, g = 2: high), the 16 ql bytes
// 64 h + 32 + 16 p.. (g = 1, 3) and the 16 qh bytes 32 h + 16 p.. (2-bit
// field g).  Tiles of 16 blocks (3360 bytes; the last may hold fewer, nb):
// for each chunk l of the tile its first 16 ql bytes, then for each chunk its
// second 16, then for each chunk its 16 qh bytes, then the nb 16-byte scale
// fields, then the nb fp16 d.  A row is 16-byte aligned when its block count
// is a multiple of 8.
struct Q6KTileOffs {
    uint32_t qa, qb, qh, sc, d;
};
__host__ __device__ constexpr Q6KTileOffs q6k_tile_offsets(int64_t chunk, int64_t nblocks) {
    const int64_t j = chunk >> 6, l = chunk & 63;
    const int64_t nb = nblocks - 16 * j < 16 ? nblocks - 16 * j : 16;
    const uint32_t base = (uint32_t)(j * 3360), nc = (uint32_t)(4 * nb);
    return Q6KTileOffs{base + 16u * (uint32_t)l, base + 16u * (nc + (uint32_t)l), base + 16u * (2u * nc + (uint32_t)l),
                       base + 48u * nc + 16u * (uint32_t)(l >> 2), base + 48u * nc + 16u * (uint32_t)nb + 2u * (uint32_t)(l >> 2)};
}

}  // namespace mxh
