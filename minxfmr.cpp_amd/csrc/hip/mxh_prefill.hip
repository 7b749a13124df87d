// mxh_prefill.hip — batched prefill for gfx950: a dequant-to-bf16, LDS-tiled
// MFMA GEMM over raw GGUF weights, and the row-batched layer ops around it.
//
// GEMM.  out[M x N] = A[M x K] . W[N x K]^T (+ res), A in bf16 (the layer's
// normed activations), W raw GGUF blocks decoded to bf16 tile by tile in LDS
// (reference op: backend_matmul_rhs_transposed with m > 1,
// src/backend/backend_runtime.cpp:302-319).  A workgroup of 4 waves owns a
// 128 x 128 output tile; each wave a 64 x 64 quarter as 2 x 2 blocks of
// v_mfma_f32_32x32x16_bf16 (fp32 accumulation).  Per K step of 64, the 256
// threads each stage 32 consecutive A values and decode one 32-element run
// of one W row (bit-exact fp32 dequant, then round-to-nearest-even bf16).
//
// Split mode (SPLIT = true, used by the model's prefill): every operand is
// carried as a pair of bf16 values, v = hi + lo with hi = bf16(v) and
// lo = bf16(v - hi), and each block product is hi*hi + hi*lo + lo*hi (three
// MFMAs).  That keeps about 16 significant bits of both operands (relative
// error near 2^-17 per product instead of 2^-8), so a prompt fed this way
// leaves the same greedy ids as the fp32 token-by-token path.
//
// Operand layout of v_mfma_f32_32x32x16_bf16 (checked on the device): lane l
// supplies row (A) / column (B) l % 32 at k = 8 (l / 32) .. +8; accumulator
// register i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"
#include "mxh_quant.h"

namespace mxh {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdk = kBK + 8;  // LDS row stride in bf16 elements (144 bytes)

__device__ __forceinline__ uint4 pack8(const float* y) {
    return make_uint4(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                      pack_bf16x2(y[6], y[7]));
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) { return __uint_as_float(b << 16); }

// v - bf16(v), the low half of a split operand
__device__ __forceinline__ float bf16_residual(float v) { return v - bf16_bits_to_float(f32_to_bf16_bits(v)); }

__device__ __forceinline__ uint4 pack8_lo(const float* y) {
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = bf16_residual(y[i]);
    return pack8(r);
}

// Weight tile staging, split in two so the next K step's global loads are
// in flight while the current step runs on the matrix cores: fetch() reads
// thread t's part of W rows [n0, n0 + 128) x columns [k0, k0 + 64) (run
// k0 / 32 + t % 2 of row n0 + t / 2; rows past n repeat the last) into
// registers, store() decodes it (bit-exact fp32, then bf16 hi / lo) into
// the LDS tiles.
template <int TYPE>
struct WStage {
    float y[32];  // generic types decode at fetch time
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int h, int form) {
        dequant_run32<TYPE>(w + (size_t)row * rb, (k0 >> 5) + h, form, y, (int64_t)(rb / block_geom(TYPE).bytes));
    }
    __device__ __forceinline__ void decode(int, int, float* out) const {
#pragma unroll
        for (int i = 0; i < 32; ++i) out[i] = y[i];
    }
};

template <>
struct WStage<MXH_Q4_K> {
    uint4 hd, qa, qb;  // header and the 32 qs bytes of 64-group g
    int form;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int, int f) {
        const uint8_t* blk = w + (size_t)row * rb + (size_t)(k0 >> 8) * 144;
        const int g = (k0 & 255) >> 6;
        hd = *reinterpret_cast<const uint4*>(blk);
        qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g);
        qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * g);
        form = f;
    }
    __device__ __forceinline__ void decode(int k0, int h, float* y) const {
        const int j = 2 * ((k0 & 255) >> 6) + h;
        uint32_t sc, mn;
        k4_scale_min(hd.y, hd.z, hd.w, j, form, sc, mn);
        const float ds = half_bits_to_float(hd.x & 0xffffu) * (float)sc;
        const float ms = half_bits_to_float(hd.x >> 16) * (float)mn;
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const int sh = 4 * h;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b) y[4 * i + b] = ds * (float)((q[i] >> (8 * b + sh)) & 15u) - ms;
    }
};

// tiled device layout: the same three 16-byte pieces (q4k_tile_offsets)
template <>
struct WStage<MXH_Q4_K_TILED> : WStage<MXH_Q4_K> {
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int, int f) {
        const Q4KTileOffs o = q4k_tile_offsets(k0 >> 6, (int64_t)(rb / 144));
        const uint8_t* rp = w + (size_t)row * rb;
        hd = *reinterpret_cast<const uint4*>(rp + o.hd);
        qa = *reinterpret_cast<const uint4*>(rp + o.qa);
        qb = *reinterpret_cast<const uint4*>(rp + o.qb);
        form = f;
    }
};

template <int TYPE>
__device__ __forceinline__ void store_w_tile(const WStage<TYPE>& ws, int k0, uint16_t* Ws, uint16_t* Ws_lo) {
    const int t = threadIdx.x, r = t >> 1, h = t & 1;
    float y[32];
    ws.decode(k0, h, y);
    uint4* dst = reinterpret_cast<uint4*>(Ws + r * kLdk + h * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = pack8(y + 8 * q);
    if (Ws_lo) {
        uint4* dlo = reinterpret_cast<uint4*>(Ws_lo + r * kLdk + h * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) dlo[q] = pack8_lo(y + 8 * q);
    }
}

// A rows [m0, m0 + 128) x columns [k0, k0 + 64): 32 bf16 of row m0 + t / 2
// per thread (zeros past m)
__device__ __forceinline__ void fetch_a(const uint16_t* __restrict__ a, int lda, int m, int m0, int k0, uint4 (&v)[4]) {
    const int t = threadIdx.x, r = t >> 1, h = t & 1;
    if (m0 + r < m) {
        const uint4* src = reinterpret_cast<const uint4*>(a + (size_t)(m0 + r) * lda + k0 + h * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = src[q];
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = make_uint4(0, 0, 0, 0);
    }
}

__device__ __forceinline__ void store_a(const uint4 (&v)[4], uint16_t* As) {
    const int t = threadIdx.x, r = t >> 1, h = t & 1;
    uint4* dst = reinterpret_cast<uint4*>(As + r * kLdk + h * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = v[q];
}

constexpr size_t kTileBytes = (size_t)kBM * kLdk * sizeof(uint16_t);  // one [128][72] bf16 tile

// Split K: workgroup z of gridDim.z takes K steps [z * ksteps, (z+1) * ksteps)
// and, with more than one split, writes its fp32 partial tile to
// part[z][m][n] for gemm_reduce_kernel.
template <int TYPE, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ a_lo,
                                                        int lda, const uint8_t* __restrict__ w, float* out, int ldo,
                                                        const float* res, int m, int n, int k, int form, int ksteps,
                                                        float* __restrict__ part) {
    // tiles: A, W, and (split) A lo, W lo
    extern __shared__ __align__(16) uint16_t smem[];
    uint16_t* As = smem;
    uint16_t* Ws = smem + kBM * kLdk;
    uint16_t* As_lo = SPLIT ? smem + 2 * kBM * kLdk : nullptr;
    uint16_t* Ws_lo = SPLIT ? smem + 3 * kBM * kLdk : nullptr;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const int kb = blockIdx.z * ksteps * kBK, ke = min(k, kb + ksteps * kBK);
    const size_t rb = row_bytes(TYPE, k);
    const int wrow = min(n0 + (int)(threadIdx.x >> 1), n - 1), wh = threadIdx.x & 1;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    const int lr = lane & 31, lk = 8 * (lane >> 5);
    uint4 av_g[4], al_g[4];
    WStage<TYPE> ws;
    fetch_a(a, lda, m, m0, kb, av_g);
    if (SPLIT) fetch_a(a_lo, lda, m, m0, kb, al_g);
    ws.fetch(w, rb, wrow, kb, wh, form);
    for (int k0 = kb; k0 < ke; k0 += kBK) {
        store_a(av_g, As);
        if (SPLIT) store_a(al_g, As_lo);
        store_w_tile<TYPE>(ws, k0, Ws, Ws_lo);
        __syncthreads();
        // next step's loads fly while this one runs on the matrix cores
        if (k0 + kBK < ke) {
            fetch_a(a, lda, m, m0, k0 + kBK, av_g);
            if (SPLIT) fetch_a(a_lo, lda, m, m0, k0 + kBK, al_g);
            ws.fetch(w, rb, wrow, k0 + kBK, wh, form);
        }
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 16) {
            bf16x8 av[2], bv[2], al[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ao = (wr * 64 + i * 32 + lr) * kLdk + ks + lk;
                const int bo = (wc * 64 + i * 32 + lr) * kLdk + ks + lk;
                av[i] = *reinterpret_cast<const bf16x8*>(As + ao);
                bv[i] = *reinterpret_cast<const bf16x8*>(Ws + bo);
                if (SPLIT) {
                    al[i] = *reinterpret_cast<const bf16x8*>(As_lo + ao);
                    bl[i] = *reinterpret_cast<const bf16x8*>(Ws_lo + bo);
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (SPLIT) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bv[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bl[j], acc[i][j], 0, 0, 0);
                    }
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
    }
    const bool partial = gridDim.z > 1;
    float* dst = partial ? part + (size_t)blockIdx.z * m * n : out;
    const int ld = partial ? n : ldo;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wc * 64 + j * 32 + lr;
            if (col >= n) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wr * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < m) {
                    const size_t o = (size_t)row * ld + col;
                    if (partial) dst[o] = acc[i][j][e];
                    else dst[o] = res ? acc[i][j][e] + res[o] : acc[i][j][e];
                }
            }
        }
}

// out = sum over splits of part (in split order) (+ res)
__global__ void gemm_reduce_kernel(const float* __restrict__ part, int splits, float* out, int ldo, const float* res,
                                   int m, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * n) return;
    const int r = i / n, c = i % n;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += part[(size_t)s * m * n + i];
    const size_t o = (size_t)r * ldo + c;
    out[o] = res ? v + res[o] : v;
}

// bf16 copy of rows of x, optionally replaced by the reference rmsnorm
// x / sqrt(mean(x^2) + eps) * w (rmsnorm.cpp:5-26; sum of squares in double).
// One workgroup per row.
__global__ __launch_bounds__(256) void rows_to_bf16_kernel(const float* __restrict__ x, int ldx,
                                                           const float* __restrict__ nw, float eps, int k,
                                                           uint16_t* __restrict__ a, uint16_t* __restrict__ a_lo,
                                                           int lda) {
    __shared__ double red[4];
    const float* xr = x + (size_t)blockIdx.x * ldx;
    uint16_t* ar = a + (size_t)blockIdx.x * lda;
    uint16_t* al = a_lo ? a_lo + (size_t)blockIdx.x * lda : nullptr;
    float inv = 1.f;
    if (nw) {
        double ss = 0.0;
        for (int e = threadIdx.x; e < k; e += 256) ss += (double)xr[e] * xr[e];
        ss = wave_sum_d_lane63(ss);
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        inv = (float)(1.0 / sqrt(((red[0] + red[1]) + (red[2] + red[3])) / (double)k + (double)eps));
    }
    for (int e = threadIdx.x; e < k; e += 256) {
        const float v = nw ? xr[e] * inv * nw[e] : xr[e];
        ar[e] = (uint16_t)f32_to_bf16_bits(v);
        if (al) al[e] = (uint16_t)f32_to_bf16_bits(bf16_residual(v));
    }
}

// h = silu(gate) * up as bf16 (and its low half) (transformer.cpp:183-185);
// gu rows are [gate | up]
__global__ void silu_mul_bf16_kernel(const float* __restrict__ gu, int f, uint16_t* __restrict__ h,
                                     uint16_t* __restrict__ h_lo, int total) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int r = i / f, c = i % f;
    const float g = gu[(size_t)r * 2 * f + c], u = gu[(size_t)r * 2 * f + f + c];
    const float v = g / (1.0f + expf(-g)) * u;
    h[i] = (uint16_t)f32_to_bf16_bits(v);
    if (h_lo) h_lo[i] = (uint16_t)f32_to_bf16_bits(bf16_residual(v));
}

// x rows z = 0..m-1: embedding rows of tokens[p0 + z] (one thread per run)
template <int TYPE>
__global__ void embed_rows_kernel(const uint8_t* __restrict__ w, const int* __restrict__ tokens, int p0, int m,
                                  float* __restrict__ x, int cols, int form) {
    const int runs = cols / 32;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= m * runs) return;
    const int z = t / runs, run = t % runs;
    float y[32];
    dequant_run32<TYPE>(w + (size_t)tokens[p0 + z] * row_bytes(TYPE, cols), run, form, y);
    float* o = x + (size_t)z * cols + run * 32;
#pragma unroll
    for (int i = 0; i < 32; ++i) o[i] = y[i];
}

}  // namespace

// ---- host launchers ---------------------------------------------------------

namespace {

template <int TYPE, bool SPLIT>
int gemm_launch(const uint16_t* a, const uint16_t* a_lo, int lda, const uint8_t* w, float* out, int ldo,
                const float* res, int m, int n, int k, int form, float* part, size_t part_floats, hipStream_t st) {
    const size_t lds = (SPLIT ? 4 : 2) * kTileBytes;
    static bool attr_set = false;  // above 64 KiB of LDS needs the opt-in, once per kernel
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)gemm_bf16_kernel<TYPE, SPLIT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return MXH_ERR_HIP;
        attr_set = true;
    }
    const int tn = (n + kBN - 1) / kBN, tm = (m + kBM - 1) / kBM, steps = k / kBK;
    // split K while the tile grid leaves CUs idle (at most 4 ways, partials
    // in `part`, reduced in split order)
    int splits = 1;
    while (splits < 4 && tn * tm * splits * 2 <= 512 && steps % (splits * 2) == 0 &&
           (size_t)(splits * 2) * m * n <= part_floats)
        splits *= 2;
    const dim3 grid(tn, tm, splits);
    hipLaunchKernelGGL((gemm_bf16_kernel<TYPE, SPLIT>), grid, dim3(256), lds, st, a, a_lo, lda, w, out, ldo, res, m, n,
                       k, form, steps / splits, part);
    if (splits > 1)
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((m * n + 255) / 256), dim3(256), 0, st, part, splits, out, ldo,
                           res, m, n);
    return MXH_OK;
}

template <bool SPLIT>
int gemm_dispatch(int type, const uint16_t* a, const uint16_t* a_lo, int lda, const uint8_t* w, float* out, int ldo,
                  const float* res, int m, int n, int k, int form, float* part, size_t pf, hipStream_t st) {
    switch (type) {
    case MXH_Q4_K: return gemm_launch<MXH_Q4_K, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q4_K_TILED:
        return gemm_launch<MXH_Q4_K_TILED, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q8_0_TILED:
        return gemm_launch<MXH_Q8_0_TILED, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q5_K_TILED:
        return gemm_launch<MXH_Q5_K_TILED, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q5_K: return gemm_launch<MXH_Q5_K, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q8_0: return gemm_launch<MXH_Q8_0, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q5_0: return gemm_launch<MXH_Q5_0, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q6_K: return gemm_launch<MXH_Q6_K, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_Q6_K_TILED:
        return gemm_launch<MXH_Q6_K_TILED, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_F16: return gemm_launch<MXH_F16, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    case MXH_F32: return gemm_launch<MXH_F32, SPLIT>(a, a_lo, lda, w, out, ldo, res, m, n, k, form, part, pf, st);
    }
    return MXH_ERR_UNSUPPORTED;
}

}  // namespace

int gemm_bf16_run(int type, const uint16_t* a, const uint16_t* a_lo, int lda, const void* w, float* out, int ldo,
                  const float* res, int m, int n, int k, int form, float* part, size_t part_floats, hipStream_t st) {
    if (m <= 0 || n <= 0 || k <= 0 || k % kBK || lda < k || ldo < n || row_bytes(type, k) == 0) return MXH_ERR_ARG;
    const uint8_t* wb = (const uint8_t*)w;
    if (!part) part_floats = 0;
    return a_lo ? gemm_dispatch<true>(type, a, a_lo, lda, wb, out, ldo, res, m, n, k, form, part, part_floats, st)
                : gemm_dispatch<false>(type, a, nullptr, lda, wb, out, ldo, res, m, n, k, form, part, part_floats, st);
}

int rows_to_bf16_launch(const float* x, int ldx, const float* nw, float eps, int k, uint16_t* a, uint16_t* a_lo,
                        int lda, int m, hipStream_t st) {
    if (m <= 0) return MXH_ERR_ARG;
    hipLaunchKernelGGL(rows_to_bf16_kernel, dim3(m), dim3(256), 0, st, x, ldx, nw, eps, k, a, a_lo, lda);
    return MXH_OK;
}

int silu_mul_bf16_launch(const float* gu, int f, uint16_t* h, uint16_t* h_lo, int m, hipStream_t st) {
    const int total = m * f;
    hipLaunchKernelGGL(silu_mul_bf16_kernel, dim3((total + 255) / 256), dim3(256), 0, st, gu, f, h, h_lo, total);
    return MXH_OK;
}

int embed_rows_launch(int type, const void* w, const int* tokens, int p0, int m, float* x, int cols, int form,
                      hipStream_t st) {
    const int threads = m * (cols / 32);
    const dim3 grid((threads + 255) / 256), block(256);
    const uint8_t* wb = (const uint8_t*)w;
    switch (type) {
    case MXH_Q4_K: hipLaunchKernelGGL(embed_rows_kernel<MXH_Q4_K>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_Q5_K: hipLaunchKernelGGL(embed_rows_kernel<MXH_Q5_K>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_Q8_0: hipLaunchKernelGGL(embed_rows_kernel<MXH_Q8_0>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_Q5_0: hipLaunchKernelGGL(embed_rows_kernel<MXH_Q5_0>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_Q6_K: hipLaunchKernelGGL(embed_rows_kernel<MXH_Q6_K>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_F16: hipLaunchKernelGGL(embed_rows_kernel<MXH_F16>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    case MXH_F32: hipLaunchKernelGGL(embed_rows_kernel<MXH_F32>, grid, block, 0, st, wb, tokens, p0, m, x, cols, form); break;
    default: return MXH_ERR_UNSUPPORTED;
    }
    return MXH_OK;
}

}  // namespace mxh
