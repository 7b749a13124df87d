// mxh_gemv.hip — raw-GGUF dequant-GEMV for gfx950 (decode hot path).
//
// y[n] = sum_k x[k] * dequant(W[n, k]), W row-major [N x K] of raw GGUF blocks
// (reference op: backend_matmul_rhs_transposed with m == 1,
// src/backend/backend_runtime.cpp:266-376).
//
// Work decomposition.  A row of W is cut into 16-byte "chunks" of packed
// codes (Q4_K: 16 qs bytes = 32 elements of two sub-blocks; Q8_0/Q5_0: one
// 32-element block; Q5_K: 16 qs bytes plus their 16 qh bytes).  Lane l of a
// wave64 owns chunks l, l+64, ... of every row, so the same x values serve
// all R rows the wave handles; x sits in LDS (padded so the eight 64-byte
// x runs a wave reads at once land in distinct banks).  Every load of W is a
// coalesced 128-bit (or dword) load of the raw block bytes; decoding happens
// in registers.  Per sub-block the inner product is factored as
//   sum_i x_i * (d*sc*q_i - dmin*m) = d*sc * sum_i x_i q_i - dmin*m * sum_i x_i
// with sum_i x_i computed once per chunk and shared across rows.  A row's
// 64 lane partials are reduced with cross-lane shuffles.
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kThreads = 64 * kWaves;

// x index -> padded LDS index (4 floats of padding after every 64)
__device__ __forceinline__ int xpad(int e) { return e + ((e >> 6) << 2); }

__device__ __forceinline__ float4 lds4(const float* xs, int e) {
    return *reinterpret_cast<const float4*>(xs + xpad(e));
}

// dot of 4 x values with the 4 bytes of `b` (each 0..255) as unsigned ints
__device__ __forceinline__ float dot4_ubyte(float4 x, uint32_t b, float acc) {
    acc = fmaf(x.x, (float)(b & 0xffu), acc);
    acc = fmaf(x.y, (float)((b >> 8) & 0xffu), acc);
    acc = fmaf(x.z, (float)((b >> 16) & 0xffu), acc);
    acc = fmaf(x.w, (float)(b >> 24), acc);
    return acc;
}

__device__ __forceinline__ float dot4_sbyte(float4 x, uint32_t b, float acc) {
    acc = fmaf(x.x, (float)(int)(int8_t)(b & 0xffu), acc);
    acc = fmaf(x.y, (float)(int)(int8_t)((b >> 8) & 0xffu), acc);
    acc = fmaf(x.z, (float)(int)(int8_t)((b >> 16) & 0xffu), acc);
    acc = fmaf(x.w, (float)(int)(int8_t)(b >> 24), acc);
    return acc;
}

__device__ __forceinline__ float sum4(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// Load a B-byte block (B = 4n+2) starting at the 2-aligned byte offset `o` of
// a 4-aligned base, into ceil(B/4) dwords, without touching bytes outside
// [o, o+B): n dwords from the aligned window plus two 16-bit tail loads.
template <int B>
__device__ __forceinline__ void load_block_2aligned(const uint8_t* base, size_t o, uint32_t (&bd)[(B + 2) / 4]) {
    constexpr int n = (B - 2) / 4;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(base + (o & ~(size_t)3));
    uint32_t dw[n];
#pragma unroll
    for (int i = 0; i < n; ++i) dw[i] = __builtin_nontemporal_load(wp + i);
    const uint32_t ua = *reinterpret_cast<const uint16_t*>(base + o + B - 4);
    const uint32_t ub = *reinterpret_cast<const uint16_t*>(base + o + B - 2);
    if ((o & 3) == 0) {
#pragma unroll
        for (int i = 0; i < n; ++i) bd[i] = dw[i];
    } else {
#pragma unroll
        for (int i = 0; i < n - 1; ++i) bd[i] = (dw[i] >> 16) | (dw[i + 1] << 16);
        bd[n - 1] = (dw[n - 1] >> 16) | (ua << 16);
    }
    bd[n] = ub;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load (weights are read once per call)
__device__ __forceinline__ uint4 ldg16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- per-type chunk kernels ------------------------------------------------
// Each accumulates, for R rows, the contribution of chunk c into acc[r].

template <int R>
struct Q4K {
    static constexpr int kType = MXH_Q4_K;
    static __device__ __forceinline__ void run(const uint8_t* w, size_t rb, const int (&rows)[R], int c,
                                               const float* xs, int form, float (&acc)[R]) {
        const int b = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
        const int e0 = 256 * b + 64 * g + 16 * h;
        uint4 hd[R], qs[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* blk = w + (size_t)rows[r] * rb + (size_t)b * 144;
            hd[r] = ldg16(blk);
            qs[r] = ldg16(blk + 16 + 16 * p);
        }
        const float4 xl0 = lds4(xs, e0), xl1 = lds4(xs, e0 + 4), xl2 = lds4(xs, e0 + 8), xl3 = lds4(xs, e0 + 12);
        const float4 xh0 = lds4(xs, e0 + 32), xh1 = lds4(xs, e0 + 36), xh2 = lds4(xs, e0 + 40),
                     xh3 = lds4(xs, e0 + 44);
        const float sl = (sum4(xl0) + sum4(xl1)) + (sum4(xl2) + sum4(xl3));
        const float sh = (sum4(xh0) + sum4(xh1)) + (sum4(xh2) + sum4(xh3));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = half_bits_to_float(hd[r].x & 0xffffu);
            const float dm = half_bits_to_float(hd[r].x >> 16);
            uint32_t sa, ma, sb, mb;
            k4_scale_min(hd[r].y, hd[r].z, hd[r].w, 2 * g, form, sa, ma);
            k4_scale_min(hd[r].y, hd[r].z, hd[r].w, 2 * g + 1, form, sb, mb);
            const uint32_t q0 = qs[r].x, q1 = qs[r].y, q2 = qs[r].z, q3 = qs[r].w;
            float dl = 0.f, dh = 0.f;
            dl = dot4_ubyte(xl0, q0 & 0x0f0f0f0fu, dl);
            dl = dot4_ubyte(xl1, q1 & 0x0f0f0f0fu, dl);
            dl = dot4_ubyte(xl2, q2 & 0x0f0f0f0fu, dl);
            dl = dot4_ubyte(xl3, q3 & 0x0f0f0f0fu, dl);
            dh = dot4_ubyte(xh0, (q0 >> 4) & 0x0f0f0f0fu, dh);
            dh = dot4_ubyte(xh1, (q1 >> 4) & 0x0f0f0f0fu, dh);
            dh = dot4_ubyte(xh2, (q2 >> 4) & 0x0f0f0f0fu, dh);
            dh = dot4_ubyte(xh3, (q3 >> 4) & 0x0f0f0f0fu, dh);
            float a = acc[r];
            a = fmaf(d * (float)sa, dl, a);
            a = fmaf(-(dm * (float)ma), sl, a);
            a = fmaf(d * (float)sb, dh, a);
            a = fmaf(-(dm * (float)mb), sh, a);
            acc[r] = a;
        }
    }
};

template <int R>
struct Q5K {
    static constexpr int kType = MXH_Q5_K;
    static __device__ __forceinline__ void run(const uint8_t* w, size_t rb, const int (&rows)[R], int c,
                                               const float* xs, int form, float (&acc)[R]) {
        const int b = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
        const int e0 = 256 * b + 64 * g + 16 * h;
        uint4 hd[R], qh[R], qs[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* blk = w + (size_t)rows[r] * rb + (size_t)b * 176;
            hd[r] = ldg16(blk);
            qh[r] = ldg16(blk + 16 + 16 * h);
            qs[r] = ldg16(blk + 48 + 16 * p);
        }
        const float4 xl0 = lds4(xs, e0), xl1 = lds4(xs, e0 + 4), xl2 = lds4(xs, e0 + 8), xl3 = lds4(xs, e0 + 12);
        const float4 xh0 = lds4(xs, e0 + 32), xh1 = lds4(xs, e0 + 36), xh2 = lds4(xs, e0 + 40),
                     xh3 = lds4(xs, e0 + 44);
        const float sl = (sum4(xl0) + sum4(xl1)) + (sum4(xl2) + sum4(xl3));
        const float sh = (sum4(xh0) + sum4(xh1)) + (sum4(xh2) + sum4(xh3));
        const int sl_bit = 2 * g, sh_bit = 2 * g + 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = half_bits_to_float(hd[r].x & 0xffffu);
            const float dm = half_bits_to_float(hd[r].x >> 16);
            uint32_t sa, ma, sb, mb;
            k4_scale_min(hd[r].y, hd[r].z, hd[r].w, 2 * g, form, sa, ma);
            k4_scale_min(hd[r].y, hd[r].z, hd[r].w, 2 * g + 1, form, sb, mb);
            const uint32_t q[4] = {qs[r].x, qs[r].y, qs[r].z, qs[r].w};
            const uint32_t hb[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
            const float4 xl[4] = {xl0, xl1, xl2, xl3};
            const float4 xh[4] = {xh0, xh1, xh2, xh3};
            float dl = 0.f, dh = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = (q[i] & 0x0f0f0f0fu) | (((hb[i] >> sl_bit) & 0x01010101u) << 4);
                const uint32_t hi = ((q[i] >> 4) & 0x0f0f0f0fu) | (((hb[i] >> sh_bit) & 0x01010101u) << 4);
                dl = dot4_ubyte(xl[i], lo, dl);
                dh = dot4_ubyte(xh[i], hi, dh);
            }
            float a = acc[r];
            a = fmaf(d * (float)sa, dl, a);
            a = fmaf(-(dm * (float)ma), sl, a);
            a = fmaf(d * (float)sb, dh, a);
            a = fmaf(-(dm * (float)mb), sh, a);
            acc[r] = a;
        }
    }
};

template <int R>
struct Q80 {
    static constexpr int kType = MXH_Q8_0;
    static __device__ __forceinline__ void run(const uint8_t* w, size_t rb, const int (&rows)[R], int c,
                                               const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        uint32_t bd[R][9];
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<34>(w, (size_t)rows[r] * rb + (size_t)c * 34, bd[r]);
        float4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = lds4(xs, e0 + 4 * i);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // block bytes: d = bytes 0-1, q = bytes 2..33
            const float d = half_bits_to_float(bd[r][0] & 0xffffu);
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qd = (bd[r][i] >> 16) | (bd[r][i + 1] << 16);
                s = dot4_sbyte(x[i], qd, s);
            }
            acc[r] = fmaf(d, s, acc[r]);
        }
    }
};

template <int R>
struct Q50 {
    static constexpr int kType = MXH_Q5_0;
    static __device__ __forceinline__ void run(const uint8_t* w, size_t rb, const int (&rows)[R], int c,
                                               const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        uint32_t bd[R][6];
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<22>(w, (size_t)rows[r] * rb + (size_t)c * 22, bd[r]);
        float4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = lds4(xs, e0 + 4 * i);
        const float sx = ((sum4(x[0]) + sum4(x[1])) + (sum4(x[2]) + sum4(x[3]))) +
                         ((sum4(x[4]) + sum4(x[5])) + (sum4(x[6]) + sum4(x[7])));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // bytes: d 0-1, qh 2-5, qs 6-21
            const float d = half_bits_to_float(bd[r][0] & 0xffffu);
            const uint32_t qh = (bd[r][0] >> 16) | (bd[r][1] << 16);
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t qd = (bd[r][1 + i] >> 16) | (bd[r][2 + i] << 16);  // qs bytes 4i..4i+3
                const uint32_t hlo = (qh >> (4 * i)) & 15u, hhi = (qh >> (16 + 4 * i)) & 15u;
                const uint32_t spread_lo = (hlo & 1u) | ((hlo & 2u) << 7) | ((hlo & 4u) << 14) | ((hlo & 8u) << 21);
                const uint32_t spread_hi = (hhi & 1u) | ((hhi & 2u) << 7) | ((hhi & 4u) << 14) | ((hhi & 8u) << 21);
                const uint32_t lo = (qd & 0x0f0f0f0fu) | (spread_lo << 4);
                const uint32_t hi = ((qd >> 4) & 0x0f0f0f0fu) | (spread_hi << 4);
                s = dot4_ubyte(x[i], lo, s);
                s = dot4_ubyte(x[4 + i], hi, s);
            }
            // d * (q - 16) summed: d * (sum x q - 16 sum x)
            acc[r] = fmaf(d, fmaf(-16.f, sx, s), acc[r]);
        }
    }
};

template <int R>
struct F32W {
    static constexpr int kType = MXH_F32;  // chunk = 32 floats
    static __device__ __forceinline__ void run(const uint8_t* w, size_t rb, const int (&rows)[R], int c,
                                               const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        float4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = lds4(xs, e0 + 4 * i);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const f32x4* p = reinterpret_cast<const f32x4*>(w + (size_t)rows[r] * rb + (size_t)c * 128);
            float s = acc[r];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const f32x4 v = __builtin_nontemporal_load(p + i);
                s = fmaf(x[i].x, v.x, s);
                s = fmaf(x[i].y, v.y, s);
                s = fmaf(x[i].z, v.z, s);
                s = fmaf(x[i].w, v.w, s);
            }
            acc[r] = s;
        }
    }
};

template <template <int> class T, int R>
// y[row] = W[row] . x (+ res[row] when res is given; res may alias y)
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                        float* y, const float* res, int n, int k, int form) {
    extern __shared__ float xs[];
    // stage x (all K values) into padded LDS
    for (int e = threadIdx.x * 4; e < k; e += kThreads * 4)
        *reinterpret_cast<float4*>(xs + xpad(e)) = *reinterpret_cast<const float4*>(x + e);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kWaves + wave) * R;
    if (row0 >= n) return;
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = min(row0 + r, n - 1);  // clamp loads in bounds
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    const size_t rbytes = row_bytes(T<R>::kType, k);
    const int nchunks = k >> 5;  // every chunk covers 32 elements
    for (int c = lane; c < nchunks; c += 64) T<R>::run(w, rbytes, rows, c, xs, form, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float s = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n) y[row0 + r] = res ? s + res[row0 + r] : s;
    }
}

template <template <int> class T, int R>
void launch_gemv(const void* w, const float* x, float* y, const float* res, int64_t n, int64_t k, int form,
                 hipStream_t st) {
    const int rows_per_block = kWaves * R;
    const unsigned grid = (unsigned)((n + rows_per_block - 1) / rows_per_block);
    const size_t lds = (size_t)(k + (k >> 4)) * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<T, R>), dim3(grid), dim3(kThreads), lds, st, (const uint8_t*)w, x, y, res,
                       (int)n, (int)k, form);
}

}  // namespace

// max K whose padded x fits the 64 KiB of LDS one workgroup may use
constexpr int64_t kGemvMaxK = 15360;

int gemv_launch(int type, const void* w, const float* x, float* y, const float* res, int64_t n, int64_t k, int form,
                hipStream_t st) {
    if (k % 32 || k > kGemvMaxK || n <= 0 || n > INT32_MAX) return MXH_ERR_ARG;
    switch (type) {
    case MXH_Q4_K: launch_gemv<Q4K, 2>(w, x, y, res, n, k, form, st); break;
    case MXH_Q5_K: launch_gemv<Q5K, 2>(w, x, y, res, n, k, form, st); break;
    case MXH_Q8_0: launch_gemv<Q80, 2>(w, x, y, res, n, k, form, st); break;
    case MXH_Q5_0: launch_gemv<Q50, 2>(w, x, y, res, n, k, form, st); break;
    case MXH_F32: launch_gemv<F32W, 2>(w, x, y, res, n, k, form, st); break;
    default: return MXH_ERR_UNSUPPORTED;
    }
    return MXH_OK;
}

}  // namespace mxh
