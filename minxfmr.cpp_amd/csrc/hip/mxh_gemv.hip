// mxh_gemv.hip — raw-GGUF dequant-GEMV for gfx950 (decode hot path).
//
// y[n] = sum_k x[k] * dequant(W[n, k]), W row-major [N x K] of raw GGUF blocks
// (reference op: backend_matmul_rhs_transposed with m == 1,
// src/backend/backend_runtime.cpp:266-376).
//
// Work decomposition.  A row of W is cut into "chunks" of 32 elements (Q4_K:
// 16 qs bytes covering half of two sub-blocks; Q5_K: the same plus their 16
// qh bytes; Q8_0/Q5_0: one block; F32: 128 bytes).  Lane l of a wave64 owns
// chunks l, l+64, ... of every row, so one x slice serves all R rows the
// wave handles at a time.  x sits in LDS, staged once per workgroup (padded
// so the 64-byte x runs read together land in distinct banks); workgroups
// are persistent over row groups so that staging, and the optional fused
// rmsnorm, are paid once per workgroup rather than once per few rows.  Each
// wave walks its (row group, chunk) sequence with the next step's weight
// loads issued before the current step's arithmetic (register double
// buffer), so 128-bit loads of raw block bytes stay in flight while decoding
// happens in registers.  Per sub-block the inner product is factored as
//   sum_i x_i (d*sc*q_i - dmin*m) = d*sc * sum_i x_i q_i - dmin*m * sum_i x_i.
// A row's 64 lane partials are reduced with cross-lane shuffles.
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = 64 * kWaves;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// x index -> padded LDS index (4 floats of padding after every 64)
__device__ __forceinline__ int xpad(int e) { return e + ((e >> 6) << 2); }

__device__ __forceinline__ float4 lds4(const float* xs, int e) {
    return *reinterpret_cast<const float4*>(xs + xpad(e));
}

// 128-bit streaming load (weights are read once per call)
__device__ __forceinline__ uint4 ldg16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// dot of 4 x values with the 4 bytes of `b` as unsigned / signed integers
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
// a 4-aligned base into ceil(B/4) dwords without touching bytes outside
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

// ---- per-type chunk load / compute ---------------------------------------
// load(): raw bytes of chunk c of R rows into a register buffer.
// compute(): add the chunk's contribution to acc[r].

template <int R>
struct Q4K {
    static constexpr int kType = MXH_Q4_K;
    struct Buf {
        uint4 hd[R], qs[R];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const int blk = c >> 3, p = c & 7;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* bp = w + (size_t)rows[r] * rb + (size_t)blk * 144;
            b.hd[r] = ldg16(bp);
            b.qs[r] = ldg16(bp + 16 + 16 * p);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int form, float (&acc)[R]) {
        const int blk = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
        const int e0 = 256 * blk + 64 * g + 16 * h;
        const float4 xl0 = lds4(xs, e0), xl1 = lds4(xs, e0 + 4), xl2 = lds4(xs, e0 + 8), xl3 = lds4(xs, e0 + 12);
        const float4 xh0 = lds4(xs, e0 + 32), xh1 = lds4(xs, e0 + 36), xh2 = lds4(xs, e0 + 40),
                     xh3 = lds4(xs, e0 + 44);
        const float sl = (sum4(xl0) + sum4(xl1)) + (sum4(xl2) + sum4(xl3));
        const float sh = (sum4(xh0) + sum4(xh1)) + (sum4(xh2) + sum4(xh3));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = half_bits_to_float(b.hd[r].x & 0xffffu);
            const float dm = half_bits_to_float(b.hd[r].x >> 16);
            uint32_t sa, ma, sb, mb;
            k4_scale_min(b.hd[r].y, b.hd[r].z, b.hd[r].w, 2 * g, form, sa, ma);
            k4_scale_min(b.hd[r].y, b.hd[r].z, b.hd[r].w, 2 * g + 1, form, sb, mb);
            const uint32_t q0 = b.qs[r].x, q1 = b.qs[r].y, q2 = b.qs[r].z, q3 = b.qs[r].w;
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
    struct Buf {
        uint4 hd[R], qh[R], qs[R];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const int blk = c >> 3, p = c & 7, h = p & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* bp = w + (size_t)rows[r] * rb + (size_t)blk * 176;
            b.hd[r] = ldg16(bp);
            b.qh[r] = ldg16(bp + 16 + 16 * h);
            b.qs[r] = ldg16(bp + 48 + 16 * p);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int form, float (&acc)[R]) {
        const int blk = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
        const int e0 = 256 * blk + 64 * g + 16 * h;
        const float4 xl[4] = {lds4(xs, e0), lds4(xs, e0 + 4), lds4(xs, e0 + 8), lds4(xs, e0 + 12)};
        const float4 xh[4] = {lds4(xs, e0 + 32), lds4(xs, e0 + 36), lds4(xs, e0 + 40), lds4(xs, e0 + 44)};
        const float sl = (sum4(xl[0]) + sum4(xl[1])) + (sum4(xl[2]) + sum4(xl[3]));
        const float sh = (sum4(xh[0]) + sum4(xh[1])) + (sum4(xh[2]) + sum4(xh[3]));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = half_bits_to_float(b.hd[r].x & 0xffffu);
            const float dm = half_bits_to_float(b.hd[r].x >> 16);
            uint32_t sa, ma, sb, mb;
            k4_scale_min(b.hd[r].y, b.hd[r].z, b.hd[r].w, 2 * g, form, sa, ma);
            k4_scale_min(b.hd[r].y, b.hd[r].z, b.hd[r].w, 2 * g + 1, form, sb, mb);
            const uint32_t q[4] = {b.qs[r].x, b.qs[r].y, b.qs[r].z, b.qs[r].w};
            const uint32_t hb[4] = {b.qh[r].x, b.qh[r].y, b.qh[r].z, b.qh[r].w};
            float dl = 0.f, dh = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = (q[i] & 0x0f0f0f0fu) | (((hb[i] >> (2 * g)) & 0x01010101u) << 4);
                const uint32_t hi = ((q[i] >> 4) & 0x0f0f0f0fu) | (((hb[i] >> (2 * g + 1)) & 0x01010101u) << 4);
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
    struct Buf {
        uint32_t bd[R][9];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<34>(w, (size_t)rows[r] * rb + (size_t)c * 34, b.bd[r]);
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        float4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = lds4(xs, e0 + 4 * i);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // block bytes: d = bytes 0-1, q = bytes 2..33
            const float d = half_bits_to_float(b.bd[r][0] & 0xffffu);
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = dot4_sbyte(x[i], (b.bd[r][i] >> 16) | (b.bd[r][i + 1] << 16), s);
            acc[r] = fmaf(d, s, acc[r]);
        }
    }
};

template <int R>
struct Q50 {
    static constexpr int kType = MXH_Q5_0;
    struct Buf {
        uint32_t bd[R][6];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<22>(w, (size_t)rows[r] * rb + (size_t)c * 22, b.bd[r]);
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        float4 x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = lds4(xs, e0 + 4 * i);
        const float sx = ((sum4(x[0]) + sum4(x[1])) + (sum4(x[2]) + sum4(x[3]))) +
                         ((sum4(x[4]) + sum4(x[5])) + (sum4(x[6]) + sum4(x[7])));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // bytes: d 0-1, qh 2-5, qs 6-21
            const float d = half_bits_to_float(b.bd[r][0] & 0xffffu);
            const uint32_t qh = (b.bd[r][0] >> 16) | (b.bd[r][1] << 16);
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t qd = (b.bd[r][1 + i] >> 16) | (b.bd[r][2 + i] << 16);  // qs bytes 4i..4i+3
                const uint32_t hlo = (qh >> (4 * i)) & 15u, hhi = (qh >> (16 + 4 * i)) & 15u;
                const uint32_t spread_lo = (hlo & 1u) | ((hlo & 2u) << 7) | ((hlo & 4u) << 14) | ((hlo & 8u) << 21);
                const uint32_t spread_hi = (hhi & 1u) | ((hhi & 2u) << 7) | ((hhi & 4u) << 14) | ((hhi & 8u) << 21);
                s = dot4_ubyte(x[i], (qd & 0x0f0f0f0fu) | (spread_lo << 4), s);
                s = dot4_ubyte(x[4 + i], ((qd >> 4) & 0x0f0f0f0fu) | (spread_hi << 4), s);
            }
            // d * (q - 16) summed: d * (sum x q - 16 sum x)
            acc[r] = fmaf(d, fmaf(-16.f, sx, s), acc[r]);
        }
    }
};

template <int R>
struct F32W {
    static constexpr int kType = MXH_F32;
    struct Buf {
        f32x4 v[R][8];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const f32x4* p = reinterpret_cast<const f32x4*>(w + (size_t)rows[r] * rb + (size_t)c * 128);
#pragma unroll
            for (int i = 0; i < 8; ++i) b.v[r][i] = __builtin_nontemporal_load(p + i);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 x = lds4(xs, e0 + 4 * i);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                acc[r] = fmaf(x.x, b.v[r][i].x, acc[r]);
                acc[r] = fmaf(x.y, b.v[r][i].y, acc[r]);
                acc[r] = fmaf(x.z, b.v[r][i].z, acc[r]);
                acc[r] = fmaf(x.w, b.v[r][i].w, acc[r]);
            }
        }
    }
};

// Stage x into padded LDS.  With a norm weight, x is replaced by the
// reference rmsnorm float(x / sqrt(mean(x^2) + eps)) * w (rmsnorm.cpp:5-26,
// transformer.cpp:189-214); the sum of squares is a double block reduction
// in a fixed order, so every workgroup computes identical inputs.
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, const float* __restrict__ nw,
                                        int k, float eps, double* red) {
    if (!nw) {
        for (int e = threadIdx.x * 4; e < k; e += kThreads * 4)
            *reinterpret_cast<float4*>(xs + xpad(e)) = *reinterpret_cast<const float4*>(x + e);
        __syncthreads();
        return;
    }
    double ss = 0.0;
    for (int e = threadIdx.x * 4; e < k; e += kThreads * 4) {
        const float4 v = *reinterpret_cast<const float4*>(x + e);
        *reinterpret_cast<float4*>(xs + xpad(e)) = v;
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double inv = 1.0 / sqrt((((red[0] + red[1]) + (red[2] + red[3]))) / (double)k + (double)eps);
    // each thread rescales the elements it staged
    for (int e = threadIdx.x * 4; e < k; e += kThreads * 4) {
        float4 v = *reinterpret_cast<const float4*>(xs + xpad(e));
        const float4 g = *reinterpret_cast<const float4*>(nw + e);
        v.x = (float)((double)v.x * inv) * g.x;
        v.y = (float)((double)v.y * inv) * g.y;
        v.z = (float)((double)v.z * inv) * g.z;
        v.w = (float)((double)v.w * inv) * g.w;
        *reinterpret_cast<float4*>(xs + xpad(e)) = v;
    }
    __syncthreads();
}

// Output modes (epilogues) of one GEMV launch.
//  GEMV_PLAIN : y[r] = W[r].x (+ res[r])
//  GEMV_SILU  : W = [gate; up] with n = 2F rows; y[i] = silu(gate_i) * up_i
//               (transformer.cpp:183-185, 696-704) for i < F
//  GEMV_ARGMAX: y = logits; each workgroup also leaves its (largest logit,
//               lowest index) in red_val/red_idx[blockIdx] for argmax_finish
template <template <int> class T, int R, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    using Ty = T<R>;
    using Buf = typename Ty::Buf;
    extern __shared__ float xs[];
    __shared__ double red[kWaves];
    __shared__ float wmax[kWaves];
    __shared__ int widx[kWaves];
    stage_x(xs, a.x, a.norm_w, a.k, a.eps, red);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // rows a wave accumulates at once; in SILU mode rows [j] and [R/2 + j]
    // are the gate and up rows of output i0 + j
    constexpr int kOut = MODE == GEMV_SILU ? R / 2 : R;
    const int n_out = MODE == GEMV_SILU ? a.n / 2 : a.n;
    const int n_groups = (n_out + kOut - 1) / kOut;
    const int nchunks = a.k >> 5;                // every chunk covers 32 elements
    const int cpl = (nchunks + 63) >> 6;         // chunk steps per lane per row group
    const size_t rbytes = row_bytes(Ty::kType, a.k);
    const int wave_id = blockIdx.x * kWaves + wave, n_waves = gridDim.x * kWaves;
    const int my_groups = wave_id < n_groups ? (n_groups - 1 - wave_id) / n_waves + 1 : 0;
    const int total = my_groups * cpl;           // (row group, chunk step) pairs of this wave
    float best = -INFINITY;
    int best_i = 0x7fffffff;

    auto rows_of = [&](int it, int (&rows)[R]) {
        const int grp = wave_id + (it / cpl) * n_waves;
#pragma unroll
        for (int r = 0; r < kOut; ++r) {
            const int o = min(grp * kOut + r, n_out - 1);  // clamp loads in bounds
            rows[r] = o;
            if (MODE == GEMV_SILU) rows[kOut + r] = o + n_out;
        }
    };
    auto chunk_of = [&](int it) { return lane + 64 * (it % cpl); };

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    Buf cur, nxt;
    if (total > 0) {
        int rows[R];
        rows_of(0, rows);
        const int c0 = chunk_of(0);
        if (c0 < nchunks) Ty::load(a.w, rbytes, rows, c0, cur);
    }
    for (int it = 0; it < total; ++it) {
        const int c = chunk_of(it);
        if (it + 1 < total) {
            int rows[R];
            rows_of(it + 1, rows);
            const int cn = chunk_of(it + 1);
            if (cn < nchunks) Ty::load(a.w, rbytes, rows, cn, nxt);
        }
        if (c < nchunks) Ty::compute(cur, c, xs, a.form, acc);
        cur = nxt;
        if (it % cpl == cpl - 1) {
            // row group complete: reduce across lanes and write
            const int grp = wave_id + (it / cpl) * n_waves;
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < kOut; ++r) {
                    const int o = grp * kOut + r;
                    if (o < n_out) {
                        float v;
                        if (MODE == GEMV_SILU) {
                            const float gt = acc[r];
                            v = gt / (1.0f + expf(-gt)) * acc[kOut + r];
                        } else {
                            v = a.res ? acc[r] + a.res[o] : acc[r];
                        }
                        a.y[o] = v;
                        if (MODE == GEMV_ARGMAX && (v > best || (v == best && o < best_i))) {
                            best = v;
                            best_i = o;
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = 0.f;
        }
    }
    if constexpr (MODE == GEMV_ARGMAX) {
        if (lane == 0) {
            wmax[wave] = best;
            widx[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w2 = 1; w2 < kWaves; ++w2)
                if (wmax[w2] > best || (wmax[w2] == best && widx[w2] < best_i)) {
                    best = wmax[w2];
                    best_i = widx[w2];
                }
            a.red_val[blockIdx.x] = best;
            a.red_idx[blockIdx.x] = best_i;
        }
    }
}

// Greedy id from the per-workgroup winners (minxfmr.cpp:2091-2115: the
// largest logit, lowest index on ties); it becomes tokens[*pos + 1] and the
// position advances.
__global__ __launch_bounds__(1024) void argmax_finish_kernel(const float* __restrict__ val, const int* __restrict__ idx,
                                                             int n, int* __restrict__ tokens, int* __restrict__ pos) {
    __shared__ float bv_s[16];
    __shared__ int bi_s[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = threadIdx.x; b < n; b += blockDim.x) {
        const float v = val[b];
        const int i = idx[b];
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { bv_s[wave] = bv; bi_s[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
            if (bv_s[w] > bv || (bv_s[w] == bv && bi_s[w] < bi)) { bv = bv_s[w]; bi = bi_s[w]; }
        if (bi == 0x7fffffff) bi = 0;  // all-NaN logits
        const int p = *pos;
        tokens[p + 1] = bi;
        *pos = p + 1;
    }
}

// Persistent grid: enough workgroups to fill the chip, never more than there
// are row groups.
int gemv_grid(int64_t wgs_needed) {
    const int64_t cap = 1024;  // 4 workgroups (16 waves) per CU on 256 CUs
    return (int)(wgs_needed < cap ? wgs_needed : cap);
}

template <template <int> class T, int R>
int launch_gemv(const GemvArgs& a, int mode, hipStream_t st) {
    const int kout = mode == GEMV_SILU ? R / 2 : R;
    const int64_t n_out = mode == GEMV_SILU ? a.n / 2 : a.n;
    const int64_t n_groups = (n_out + kout - 1) / kout;
    const unsigned grid = (unsigned)gemv_grid((n_groups + kWaves - 1) / kWaves);
    const size_t lds = (size_t)(a.k + (a.k >> 4)) * sizeof(float);
    if (mode == GEMV_PLAIN) hipLaunchKernelGGL((gemv_kernel<T, R, GEMV_PLAIN>), dim3(grid), dim3(kThreads), lds, st, a);
    else if (mode == GEMV_SILU) hipLaunchKernelGGL((gemv_kernel<T, R, GEMV_SILU>), dim3(grid), dim3(kThreads), lds, st, a);
    else {
        if ((int)grid > a.red_cap) return MXH_ERR_ARG;
        hipLaunchKernelGGL((gemv_kernel<T, R, GEMV_ARGMAX>), dim3(grid), dim3(kThreads), lds, st, a);
        hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1024), 0, st, a.red_val, a.red_idx, (int)grid, a.tokens,
                           a.pos);
    }
    return MXH_OK;
}

}  // namespace

// max K whose padded x fits the 64 KiB of LDS one workgroup may use
constexpr int64_t kGemvMaxK = 15360;

int gemv_run(int type, const GemvArgs& a, int mode, hipStream_t st) {
    if (a.k % 32 || a.k > kGemvMaxK || a.n <= 0 || (mode == GEMV_SILU && a.n % 2)) return MXH_ERR_ARG;
    if (mode == GEMV_ARGMAX && (!a.red_val || !a.red_idx || !a.tokens || !a.pos)) return MXH_ERR_ARG;
    switch (type) {
    case MXH_Q4_K: return launch_gemv<Q4K, 2>(a, mode, st);
    case MXH_Q5_K: return launch_gemv<Q5K, 2>(a, mode, st);
    case MXH_Q8_0: return launch_gemv<Q80, 2>(a, mode, st);
    case MXH_Q5_0: return launch_gemv<Q50, 2>(a, mode, st);
    case MXH_F32: return launch_gemv<F32W, 2>(a, mode, st);
    }
    return MXH_ERR_UNSUPPORTED;
}

int gemv_launch(int type, const void* w, const float* x, float* y, const float* res, int64_t n, int64_t k, int form,
                hipStream_t st) {
    if (n <= 0 || n > INT32_MAX) return MXH_ERR_ARG;
    GemvArgs a{};
    a.w = (const uint8_t*)w;
    a.x = x;
    a.y = y;
    a.res = res;
    a.n = (int)n;
    a.k = (int)k;
    a.form = form;
    return gemv_run(type, a, GEMV_PLAIN, st);
}

}  // namespace mxh
