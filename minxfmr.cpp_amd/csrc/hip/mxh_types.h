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

__host__ __device__ constexpr BlockGeom block_geom(int type) {
    return type == MXH_Q4_K   ? BlockGeom{256, 144}
           : type == MXH_Q5_K ? BlockGeom{256, 176}
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

}  // namespace mxh
