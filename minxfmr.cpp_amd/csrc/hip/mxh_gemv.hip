// mxh_gemv.hip — raw-GGUF dequant-GEMV for gfx950 (decode hot path).
//
// y[n] = sum_k x[k] * dequant(W[n, k]), W row-major [N x K] of raw GGUF blocks
// (reference op: backend_matmul_rhs_transposed with m == 1,
// src/backend/backend_runtime.cpp:266-376).
//
// Work decomposition.  A row of W is cut into "chunks" (Q4_K: a 64-element
// group of a super-block, its 32 qs bytes covering two whole sub-blocks;
// Q5_K: 32 elements, 16 qs bytes covering half of two sub-blocks plus their
// 16 qh bytes; Q8_0/Q5_0: one block; F32: 128 bytes).  Lane l of a wave64 owns
// chunks l, l+64, ... of every row, so one x slice serves all R rows the
// wave handles at a time.  x is staged in LDS once per workgroup;
// workgroups are persistent over row groups so that staging, and the
// optional fused rmsnorm, are paid once per workgroup rather than once per
// few rows.  Each wave walks its (row group, chunk) sequence with the next
// step's weight loads issued before the current step's arithmetic (register
// double buffer), so 128-bit loads of raw block bytes stay in flight while
// decoding happens in registers.  A row's 64 lane partials are reduced with
// cross-lane shuffles.
//
// Integer inner products.  For the quantized formats x is staged as 24-bit
// block fixed point: per 32-element sub-block j, X_i = rint(x_i / s_j) with
// s_j = max|x| / kXMax (kXMax = 8355000, so |X| < 0x7f7f7f), split into three
// signed bytes X = 65536 hi + 256 mid + lo.  The codes q are small integers,
// so each limb's sum_i L_i q_i is exact in int32 at three v_dot4_i32_i8 per
// four elements (no per-element conversion), and 256 hi-sum + mid-sum is
// still exact in int32.  With
//   sum_i x_i (d*sc*q_i - dmin*m) = d*sc*s_j * sum_i X_i q_i - dmin*m * s_j * sum_i X_i
// the approximations are x's rounding to 24 bits (half a unit of 2^-23 of
// the sub-block maximum, the size of a float rounding of that maximum) and
// float roundings of the per-sub-block sums: errors of the order of an fp32
// dot product's, while the weights are used exactly.  A NaN in x makes its
// sub-block scale NaN, so it reaches the outputs as in fp32 arithmetic.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kShortSteps = 3;  // steps per wave of the short form
// the SwiGLU (gate|up) short form: 768 workgroups of four waves (three per
// CU) take the Qwen3-8B gate|up rows in one round (3, 5, 6, 12 steps:
// 598.6, 586.0, 599-605, 578.0 against 599-602 tok/s; 6 was 1-2% slower on
// the smaller models)
constexpr int kSiluShortSteps = 4;

constexpr int kThreads = 64 * kWaves;

// sum of the per-wave partials in a fixed order
// 1 / sqrt(v) in double, v > 0: the hardware estimate and two Newton steps
// (each squares the relative error), so the float rounding the callers take
// is that of the exact quotient
__device__ __forceinline__ double rsqrt_d(double v) {
    double r = __builtin_amdgcn_rsq(v);
    r = r * (1.5 - 0.5 * v * r * r);
    return r * (1.5 - 0.5 * v * r * r);
}

template <int W>
__device__ __forceinline__ double block_sum(const double* red) {
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < W; w += 2) s += red[w] + red[w + 1];
    return s;
}

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

// ---- staged x in LDS ------------------------------------------------------
// Quantized formats: lo/mid/hi limb bytes (K each, 4 per dword, with 4
// dwords of padding after every 16 so that lanes reading consecutive
// 64-element runs hit distinct banks), per-32 scales (K/32) and per-16 scaled
// sums s_j * sum X_i (K/16).
struct XQ {
    const uint32_t* lo;
    const uint32_t* mid;
    const uint32_t* hi;
    const float* scale;
    const float* sum16;
};

// 24-bit fixed point: X = rint(x * kXMax / max|x|) stays within
// [-0x7f7f7f, 0x7f7f7f] (kXMax leaves room for the reciprocal's error), the
// range in which X + 0x808080 has three bytes that are the limbs plus 128
constexpr float kXMax = 8355000.0f;

// dword index of limb dword d (elements 4d..4d+3) in the padded arrays
__device__ __forceinline__ int limb(int d) { return d + ((d >> 4) << 2); }
__host__ __device__ constexpr int limb_dwords(int k) { return k / 4 + k / 16; }
// The arrays are sized for K rounded up to whole staging passes (1024
// elements: 4 per thread), so a pass past K writes zeros into padding
// instead of needing a per-lane guard.
// (W waves per workgroup: one pass is 256 W elements)
template <int W>
__host__ __device__ constexpr int xq_cap(int k) { return (k + 256 * W - 1) / (256 * W) * (256 * W); }
template <int W>
__host__ __device__ constexpr int xq_dwords(int k) {
    return 3 * limb_dwords(xq_cap<W>(k)) + xq_cap<W>(k) / 32 + xq_cap<W>(k) / 16;
}

template <int W>
__device__ __forceinline__ XQ xq_view(const float* smem, int k) {
    const uint32_t* lo = reinterpret_cast<const uint32_t*>(smem);
    const int n = limb_dwords(xq_cap<W>(k));
    return XQ{lo, lo + n, lo + 2 * n, reinterpret_cast<const float*>(lo + 3 * n),
              reinterpret_cast<const float*>(lo + 3 * n) + xq_cap<W>(k) / 32};
}

__device__ __forceinline__ uint4 lds16(const uint32_t* p) { return *reinterpret_cast<const uint4*>(p); }

// the three limbs of 16 staged elements (limb dwords d .. d+3)
struct XP {
    uint4 l, m, h;
};
__device__ __forceinline__ XP xp_load(const XQ& x, int d) {
    return XP{lds16(x.lo + limb(d)), lds16(x.mid + limb(d)), lds16(x.hi + limb(d))};
}

// s_waitcnt vmcnt(N): wait until at most N vector memory operations of this
// wave are outstanding (they complete in issue order for loads); expcnt and
// lgkmcnt are left alone.  Explicit waits with exact counts keep the weight
// loads of later steps in flight where the compiler's own analysis would wait
// for them too.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// per-limb integer sums of X_i q_i
struct LimbSum {
    int l, m, h;
};
__device__ __forceinline__ LimbSum limb_zero() { return LimbSum{0, 0, 0}; }
// add 16 elements: the limbs of x against the code bytes q0..q3
__device__ __forceinline__ void limb_acc(LimbSum& a, const XP& x, uint32_t q0, uint32_t q1, uint32_t q2,
                                         uint32_t q3) {
    a.l = sdot4(x.l.x, q0, a.l);
    a.m = sdot4(x.m.x, q0, a.m);
    a.h = sdot4(x.h.x, q0, a.h);
    a.l = sdot4(x.l.y, q1, a.l);
    a.m = sdot4(x.m.y, q1, a.m);
    a.h = sdot4(x.h.y, q1, a.h);
    a.l = sdot4(x.l.z, q2, a.l);
    a.m = sdot4(x.m.z, q2, a.m);
    a.h = sdot4(x.h.z, q2, a.h);
    a.l = sdot4(x.l.w, q3, a.l);
    a.m = sdot4(x.m.w, q3, a.m);
    a.h = sdot4(x.h.w, q3, a.h);
}
// sum_i X_i q_i = 65536 h + 256 m + l.  Over at most 32 elements with
// |q| <= 128 each limb sum is at most 2^19 in magnitude, so 256 h + m is exact
// in int32; the float result takes one rounding (two for codes above 16)
__device__ __forceinline__ float limb_total(const LimbSum& a) {
    return fmaf((float)(a.h * 256 + a.m), 256.0f, (float)a.l);
}
// sum over 16 elements of X_i q_i
__device__ __forceinline__ float dot16(const XP& x, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3) {
    LimbSum a = limb_zero();
    limb_acc(a, x, q0, q1, q2, q3);
    return limb_total(a);
}

__device__ __forceinline__ float2 h2f2(uint32_t v) {
    __half2 h;
    __builtin_memcpy(&h, &v, 4);
    return __half22float2(h);
}

__device__ __forceinline__ float h2f(uint32_t v) {
    __half h;
    const uint16_t b = (uint16_t)v;
    __builtin_memcpy(&h, &b, 2);
    return __half2float(h);
}

// ---- per-type chunk load / compute -----------------------------------------
// load(): raw bytes of chunk c of R rows into a register buffer.
// compute(): add the chunk's contribution to acc[r].

// Q4_K, 64-element chunks: chunk c is 64-group g = c & 3 of super-block
// c >> 2 (32 qs bytes: low nibbles = sub-block 2g, high nibbles = 2g+1).
// Lane l always sees the same g (= l & 3), so the 6-bit scale/min unpack
// reduces to lane-constant masks.
template <int R>
struct Q4K {
    static constexpr int kType = MXH_Q4_K;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 6;
    static constexpr int kLoads = 3;  // vector loads per row per chunk
    struct Buf {
        uint4 hd[R], qa[R], qb[R];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const int blk = c >> 2, g = c & 3;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* bp = w + (size_t)rows[r] * rb + (size_t)blk * 144;
            b.hd[r] = ldg16(bp);
            b.qa[r] = ldg16(bp + 16 + 32 * g);
            b.qb[r] = ldg16(bp + 32 + 32 * g);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int form, float (&acc)[R]) {
        const int blk = c >> 2, g = c & 3;
        const int d0 = 64 * blk + 16 * g;  // limb dword of element e0 = 256 blk + 64 g
        const XP x0 = xp_load(x, d0), x1 = xp_load(x, d0 + 4), x2 = xp_load(x, d0 + 8), x3 = xp_load(x, d0 + 12);
        const int j0 = d0 >> 3;  // sub-block 2g of the row
        const float sa = x.scale[j0], sb = x.scale[j0 + 1];
        const float ta = x.sum16[2 * j0] + x.sum16[2 * j0 + 1], tb = x.sum16[2 * j0 + 2] + x.sum16[2 * j0 + 3];
        // scale/min bytes of sub-blocks (2g, 2g+1) (tensor.cpp:395-403; ggml
        // form for form != 0): g < 2 reads bytes 2g.. of the first two dwords,
        // g >= 2 combines low nibbles of the third dword with top bits
        const int sh = (g & 1) * 16;
        const bool up = g >= 2;
        const uint32_t mA = up ? 0u : 0x3f3fu, mC = up ? 0x0f0fu : 0u, mT = up ? 0x3030u : 0u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float2 dd = h2f2(b.hd[r].x);  // d, dmin
            const uint32_t A = b.hd[r].y >> sh, B = b.hd[r].z >> sh, C = b.hd[r].w >> sh;
            const uint32_t scp = (A & mA) | (C & mC) | (((form ? A : B) >> 2) & mT);
            const uint32_t mnp = (B & mA) | ((C >> 4) & mC) | ((B >> 2) & mT);
            const uint4 qa = b.qa[r], qb = b.qb[r];
            // low nibbles: elements e0..e0+31; high nibbles: e0+32..e0+63
            constexpr uint32_t kN = 0x0f0f0f0fu;
            LimbSum la = limb_zero(), lb = limb_zero();
            limb_acc(la, x0, qa.x & kN, qa.y & kN, qa.z & kN, qa.w & kN);
            limb_acc(la, x1, qb.x & kN, qb.y & kN, qb.z & kN, qb.w & kN);
            limb_acc(lb, x2, (qa.x >> 4) & kN, (qa.y >> 4) & kN, (qa.z >> 4) & kN, (qa.w >> 4) & kN);
            limb_acc(lb, x3, (qb.x >> 4) & kN, (qb.y >> 4) & kN, (qb.z >> 4) & kN, (qb.w >> 4) & kN);
            const float da = limb_total(la), db = limb_total(lb);
            float a = acc[r];
            a = fmaf(dd.x * (float)(scp & 0xffu) * sa, da, a);
            a = fmaf(-(dd.y * (float)(mnp & 0xffu)), ta, a);
            a = fmaf(dd.x * (float)((scp >> 8) & 0xffu) * sb, db, a);
            a = fmaf(-(dd.y * (float)((mnp >> 8) & 0xffu)), tb, a);
            acc[r] = a;
        }
    }
};

// Q4_K in the tiled device layout: the same bytes per chunk, read from
// line-contiguous 16-byte pieces (q4k_tile_offsets)
template <int R>
struct Q4KT : Q4K<R> {
    static constexpr int kType = MXH_Q4_K_TILED;
    using Buf = typename Q4K<R>::Buf;
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const Q4KTileOffs o = q4k_tile_offsets(c, (int64_t)(rb / 144));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* rp = w + (size_t)rows[r] * rb;
            b.hd[r] = ldg16(rp + o.hd);
            b.qa[r] = ldg16(rp + o.qa);
            b.qb[r] = ldg16(rp + o.qb);
        }
    }
};

template <int R>
struct Q5K {
    static constexpr int kType = MXH_Q5_K;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 3;
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
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int form, float (&acc)[R]) {
        const int blk = c >> 3, p = c & 7, g = p >> 1, h = p & 1;
        const int e0 = 256 * blk + 64 * g + 16 * h;
        const XP xa = xp_load(x, e0 / 4), xb = xp_load(x, e0 / 4 + 8);
        const float sa = x.scale[e0 >> 5], sb = x.scale[(e0 >> 5) + 1];
        const float ta = x.sum16[e0 >> 4], tb = x.sum16[(e0 >> 4) + 2];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float2 dd = h2f2(b.hd[r].x);
            uint32_t scp, mnp;
            k4_pair(b.hd[r].y, b.hd[r].z, b.hd[r].w, g, form, scp, mnp);
            const uint32_t q[4] = {b.qs[r].x, b.qs[r].y, b.qs[r].z, b.qs[r].w};
            const uint32_t hb[4] = {b.qh[r].x, b.qh[r].y, b.qh[r].z, b.qh[r].w};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] = (q[i] & 0x0f0f0f0fu) | (((hb[i] >> (2 * g)) & 0x01010101u) << 4);
                hi[i] = ((q[i] >> 4) & 0x0f0f0f0fu) | (((hb[i] >> (2 * g + 1)) & 0x01010101u) << 4);
            }
            const float da = dot16(xa, lo[0], lo[1], lo[2], lo[3]);
            const float db = dot16(xb, hi[0], hi[1], hi[2], hi[3]);
            float a = acc[r];
            a = fmaf(dd.x * (float)(scp & 0xffu) * sa, da, a);
            a = fmaf(-(dd.y * (float)(mnp & 0xffu)), ta, a);
            a = fmaf(dd.x * (float)((scp >> 8) & 0xffu) * sb, db, a);
            a = fmaf(-(dd.y * (float)((mnp >> 8) & 0xffu)), tb, a);
            acc[r] = a;
        }
    }
};

// Q5_K in the tiled device layout (q5k_tile_offsets)
template <int R>
struct Q5KT : Q5K<R> {
    static constexpr int kType = MXH_Q5_K_TILED;
    using Buf = typename Q5K<R>::Buf;
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const Q5KTileOffs o = q5k_tile_offsets(c, (int64_t)(rb / 176));
        const int h = c & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* rp = w + (size_t)rows[r] * rb;
            b.hd[r] = ldg16(rp + o.hd);
            b.qh[r] = ldg16(rp + o.qh + 16 * h);
            b.qs[r] = ldg16(rp + o.qs);
        }
    }
};

template <int R>
struct Q80 {
    static constexpr int kType = MXH_Q8_0;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 10;
    struct Buf {
        uint32_t bd[R][9];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<34>(w, (size_t)rows[r] * rb + (size_t)c * 34, b.bd[r]);
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        const XP x0 = xp_load(x, e0 / 4), x1 = xp_load(x, e0 / 4 + 4);
        const float s = x.scale[c];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // block bytes: d = bytes 0-1, q = bytes 2..33 (signed)
            const float d = h2f(b.bd[r][0]);
            uint32_t q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = (b.bd[r][i] >> 16) | (b.bd[r][i + 1] << 16);
            LimbSum ls = limb_zero();
            limb_acc(ls, x0, q[0], q[1], q[2], q[3]);
            limb_acc(ls, x1, q[4], q[5], q[6], q[7]);
            acc[r] = fmaf(d * s, limb_total(ls), acc[r]);
        }
    }
};

// Q8_0 in the tiled device layout (q80_tile_offsets): two aligned 16-byte
// quant loads and the scale per block instead of ten 2-aligned pieces
template <int R>
struct Q80T {
    static constexpr int kType = MXH_Q8_0_TILED;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 3;
    struct Buf {
        uint4 lo[R], hi[R];
        uint32_t d[R];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const Q80TileOffs o = q80_tile_offsets(c, (int64_t)(rb / 34));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* rp = w + (size_t)rows[r] * rb;
            b.lo[r] = ldg16(rp + o.lo);
            b.hi[r] = ldg16(rp + o.hi);
            b.d[r] = *reinterpret_cast<const uint16_t*>(rp + o.d);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        const XP x0 = xp_load(x, e0 / 4), x1 = xp_load(x, e0 / 4 + 4);
        const float s = x.scale[c];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            LimbSum ls = limb_zero();
            limb_acc(ls, x0, b.lo[r].x, b.lo[r].y, b.lo[r].z, b.lo[r].w);
            limb_acc(ls, x1, b.hi[r].x, b.hi[r].y, b.hi[r].z, b.hi[r].w);
            acc[r] = fmaf(h2f(b.d[r]) * s, limb_total(ls), acc[r]);
        }
    }
};

template <int R>
struct Q50 {
    static constexpr int kType = MXH_Q5_0;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 7;
    struct Buf {
        uint32_t bd[R][6];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) load_block_2aligned<22>(w, (size_t)rows[r] * rb + (size_t)c * 22, b.bd[r]);
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int, float (&acc)[R]) {
        const int e0 = 32 * c;
        const XP x0 = xp_load(x, e0 / 4), x1 = xp_load(x, e0 / 4 + 4);
        const float s = x.scale[c];
        const float t = x.sum16[2 * c] + x.sum16[2 * c + 1];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // bytes: d 0-1, qh 2-5, qs 6-21; code q = nibble | bit << 4, value d*(q-16)
            const float d = h2f(b.bd[r][0]);
            const uint32_t qh = (b.bd[r][0] >> 16) | (b.bd[r][1] << 16);
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t qd = (b.bd[r][1 + i] >> 16) | (b.bd[r][2 + i] << 16);  // qs bytes 4i..4i+3
                const uint32_t hlo = (qh >> (4 * i)) & 15u, hhi = (qh >> (16 + 4 * i)) & 15u;
                const uint32_t spread_lo = (hlo & 1u) | ((hlo & 2u) << 7) | ((hlo & 4u) << 14) | ((hlo & 8u) << 21);
                const uint32_t spread_hi = (hhi & 1u) | ((hhi & 2u) << 7) | ((hhi & 4u) << 14) | ((hhi & 8u) << 21);
                lo[i] = (qd & 0x0f0f0f0fu) | (spread_lo << 4);
                hi[i] = ((qd >> 4) & 0x0f0f0f0fu) | (spread_hi << 4);
            }
            // elements 0..15 are the low nibbles, 16..31 the high nibbles
            LimbSum ls = limb_zero();
            limb_acc(ls, x0, lo[0], lo[1], lo[2], lo[3]);
            limb_acc(ls, x1, hi[0], hi[1], hi[2], hi[3]);
            acc[r] = fmaf(d, fmaf(s, limb_total(ls), -16.f * t), acc[r]);
        }
    }
};

// Q6_K, 64-element chunks c = 4 b + 2 h + p (mxh_types.h): for l in
// [16 p, 16 p + 16) the elements 128 h + l + 32 g of block b, g = 0..3, with
// codes from the 16 ql bytes 64 h + 16 p (qa: g = 0 low, g = 2 high
// nibbles), the 16 ql bytes 64 h + 32 + 16 p (qb: g = 1, 3) and the 16 qh
// bytes 32 h + 16 p (2-bit field g), and the int8 scale 8 h + p + 2 g.  The
// code minus 32 is formed as a signed byte (the 6-bit value with bit 5
// flipped, sign-extended), so each 16-element sum of X_i (q_i - 32) is an
// exact int32 v_dot4 sum and the weights, (d * sc) * (q - 32), are exact.
struct Q6KPieces {
    uint4 qa, qb, qh;
    uint2 sc;  // scales 8 h .. 8 h + 7 of the block
    float d;
};
// q - 32 of four bytes as signed bytes from 4-bit parts lo (bits 0-3 of each
// byte) and 2-bit parts hi (bits 0-1): (hi ^ 2) is the signed top field
__device__ __forceinline__ uint32_t q6_signed(uint32_t lo, uint32_t hi) {
    const uint32_t f = (hi & 0x03030303u) ^ 0x02020202u;
    return (lo & 0x0f0f0f0fu) | (f << 4) | ((f & 0x02020202u) * 0x60u);
}
template <int R>
__device__ __forceinline__ void q6k_accum(const Q6KPieces (&pc)[R], int c, const XQ& x, float (&acc)[R]) {
    const int blk = c >> 2, h = (c >> 1) & 1, p = c & 1;
    const int e0 = 256 * blk + 128 * h + 16 * p;
    XP xg[4];
    float sg[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        xg[g] = xp_load(x, (e0 + 32 * g) >> 2);
        sg[g] = x.scale[(e0 + 32 * g) >> 5];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t A[4] = {pc[r].qa.x, pc[r].qa.y, pc[r].qa.z, pc[r].qa.w};
        const uint32_t B[4] = {pc[r].qb.x, pc[r].qb.y, pc[r].qb.z, pc[r].qb.w};
        const uint32_t H[4] = {pc[r].qh.x, pc[r].qh.y, pc[r].qh.z, pc[r].qh.w};
        LimbSum ls[4] = {limb_zero(), limb_zero(), limb_zero(), limb_zero()};
        uint32_t q0[4], q1[4], q2[4], q3[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q0[i] = q6_signed(A[i], H[i]);
            q1[i] = q6_signed(B[i], H[i] >> 2);
            q2[i] = q6_signed(A[i] >> 4, H[i] >> 4);
            q3[i] = q6_signed(B[i] >> 4, H[i] >> 6);
        }
        limb_acc(ls[0], xg[0], q0[0], q0[1], q0[2], q0[3]);
        limb_acc(ls[1], xg[1], q1[0], q1[1], q1[2], q1[3]);
        limb_acc(ls[2], xg[2], q2[0], q2[1], q2[2], q2[3]);
        limb_acc(ls[3], xg[3], q3[0], q3[1], q3[2], q3[3]);
        const uint32_t scw = p ? (pc[r].sc.x >> 8) | (pc[r].sc.y << 24) : pc[r].sc.x;  // bytes p, p+1, ...
        const uint32_t scw2 = p ? (pc[r].sc.y >> 8) : pc[r].sc.y;                     // bytes p+4, ...
        const float d = pc[r].d;
        float a = acc[r];
        a = fmaf(d * (float)(int)(int8_t)(scw & 0xffu) * sg[0], limb_total(ls[0]), a);
        a = fmaf(d * (float)(int)(int8_t)((scw >> 16) & 0xffu) * sg[1], limb_total(ls[1]), a);
        a = fmaf(d * (float)(int)(int8_t)(scw2 & 0xffu) * sg[2], limb_total(ls[2]), a);
        a = fmaf(d * (float)(int)(int8_t)((scw2 >> 16) & 0xffu) * sg[3], limb_total(ls[3]), a);
        acc[r] = a;
    }
}

// Q6_K in the tiled device layout (q6k_tile_offsets): three 16-byte code
// pieces, the block's 8 scales of half h and d
template <int R>
struct Q6KT {
    static constexpr int kType = MXH_Q6_K_TILED;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 6;
    static constexpr int kLoads = 5;
    struct Buf {
        uint4 qa[R], qb[R], qh[R];
        uint2 sc[R];
        uint32_t d[R];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const Q6KTileOffs o = q6k_tile_offsets(c, (int64_t)(rb / 210));
        const int h = (c >> 1) & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* rp = w + (size_t)rows[r] * rb;
            b.qa[r] = ldg16(rp + o.qa);
            b.qb[r] = ldg16(rp + o.qb);
            b.qh[r] = ldg16(rp + o.qh);
            b.sc[r] = *reinterpret_cast<const uint2*>(rp + o.sc + 8 * h);
            b.d[r] = *reinterpret_cast<const uint16_t*>(rp + o.d);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int, float (&acc)[R]) {
        Q6KPieces pc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) pc[r] = Q6KPieces{b.qa[r], b.qb[r], b.qh[r], b.sc[r], h2f(b.d[r])};
        q6k_accum<R>(pc, c, x, acc);
    }
};

// Q6_K in the GGUF block order, whose 210-byte blocks are only 2-aligned:
// each piece is read as the dwords of its aligned window (one dword before
// the piece when the block starts at 2 mod 4) plus the piece's last 16 bits,
// the same loads whatever the alignment, and realigned in compute().  Every
// byte read lies in [block - 2, block + 210); a block at offset 2 mod 4 is
// never the first of its allocation.
template <int R>
struct Q6K {
    static constexpr int kType = MXH_Q6_K;
    static constexpr bool kIntX = true;
    static constexpr int kChunkShift = 6;
    static constexpr int kLoads = 19;
    struct Buf {
        uint32_t qa[R][5], qb[R][5], qh[R][5], sc[R][3], d[R];
        bool odd[R];  // the block starts at 2 mod 4
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
        const int blk = c >> 2, h = (c >> 1) & 1, p = c & 1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* bp = w + (size_t)rows[r] * rb + (size_t)blk * 210;
            b.odd[r] = ((uintptr_t)bp & 2) != 0;
            const uint8_t* ap = bp - ((uintptr_t)bp & 2);  // 4-aligned
            auto piece = [&](int off, int nd, uint32_t* out) {
                const uint32_t* wp = reinterpret_cast<const uint32_t*>(ap + off);
                for (int i = 0; i < nd; ++i) out[i] = __builtin_nontemporal_load(wp + i);
                out[nd] = *reinterpret_cast<const uint16_t*>(bp + off + 4 * nd - 2);
            };
            piece(64 * h + 16 * p, 4, b.qa[r]);
            piece(64 * h + 32 + 16 * p, 4, b.qb[r]);
            piece(128 + 32 * h + 16 * p, 4, b.qh[r]);
            piece(192 + 8 * h, 2, b.sc[r]);
            b.d[r] = *reinterpret_cast<const uint16_t*>(bp + 208);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const XQ& x, int, float (&acc)[R]) {
        Q6KPieces pc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool o = b.odd[r];
            auto u4 = [&](const uint32_t* v) {
                return o ? make_uint4((v[0] >> 16) | (v[1] << 16), (v[1] >> 16) | (v[2] << 16),
                                      (v[2] >> 16) | (v[3] << 16), (v[3] >> 16) | (v[4] << 16))
                         : make_uint4(v[0], v[1], v[2], v[3]);
            };
            const uint32_t* s = b.sc[r];
            const uint2 sc = o ? make_uint2((s[0] >> 16) | (s[1] << 16), (s[1] >> 16) | (s[2] << 16))
                               : make_uint2(s[0], s[1]);
            pc[r] = Q6KPieces{u4(b.qa[r]), u4(b.qb[r]), u4(b.qh[r]), sc, h2f(b.d[r])};
        }
        q6k_accum<R>(pc, c, x, acc);
    }
};

// F16 rows, 32-element chunks (64 bytes, four 16-byte loads); x in fp32
template <int R>
struct F16W {
    static constexpr int kType = MXH_F16;
    static constexpr bool kIntX = false;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 4;
    struct Buf {
        uint4 v[R][4];
    };
    static __device__ __forceinline__ void load(const uint8_t* w, size_t rb, const int (&rows)[R], int c, Buf& b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* p = w + (size_t)rows[r] * rb + (size_t)c * 64;
#pragma unroll
            for (int i = 0; i < 4; ++i) b.v[r][i] = ldg16(p + 16 * i);
        }
    }
    static __device__ __forceinline__ void compute(const Buf& b, int c, const float* xs, int, float (&acc)[R]) {
        const int e0 = 32 * c;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 xa = lds4(xs, e0 + 8 * i), xb = lds4(xs, e0 + 8 * i + 4);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float2 w0 = h2f2(b.v[r][i].x), w1 = h2f2(b.v[r][i].y), w2 = h2f2(b.v[r][i].z),
                             w3 = h2f2(b.v[r][i].w);
                float a = acc[r];
                a = fmaf(xa.x, w0.x, a);
                a = fmaf(xa.y, w0.y, a);
                a = fmaf(xa.z, w1.x, a);
                a = fmaf(xa.w, w1.y, a);
                a = fmaf(xb.x, w2.x, a);
                a = fmaf(xb.y, w2.y, a);
                a = fmaf(xb.z, w3.x, a);
                a = fmaf(xb.w, w3.y, a);
                acc[r] = a;
            }
        }
    }
};

template <int R>
struct F32W {
    static constexpr int kType = MXH_F32;
    static constexpr bool kIntX = false;
    static constexpr int kChunkShift = 5;
    static constexpr int kLoads = 8;
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
template <int W>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, const float* __restrict__ nw,
                                        int k, float eps, double* red) {
    constexpr int kThreads = 64 * W;
    if (!nw) {
#pragma unroll 4
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
    const double inv = 1.0 / sqrt(block_sum<W>(red) / (double)k + (double)eps);
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

// Quantize NB units of 4 consecutive staged values of thread `threadIdx.x`
// (unit u: elements e0 + 1024 u .. +3, part of a 32-element sub-block shared
// by 8 consecutive threads) into the limb layout at `smem` (the XQ arrays).
// Runs with the whole wave active (DPP) and without per-lane branches, one
// phase for all units at a time, so the units' dependent chains interleave:
// every lane stores (units past k hold zeros and land in the arrays'
// padding; whole passes past it are skipped), and the
// scale / sum16 entries are stored by every lane of their sub-block / quad
// (the same value to the same address).
//
// X = rint(x / s) with s = max|x| / kXMax fits 24 bits.  With
// Y = X + 0x8080 the signed limbs of X = 65536 hi + 256 mid + lo are
// lo = byte 0 of Y xor 0x80, mid = byte 1 of Y xor 0x80 and hi = byte 2 of Y,
// gathered four elements to a dword by byte permutes; the sub-block sums of
// X are exact in int32 (16 values below 2^23 each).
template <int W, int NB>
__device__ __forceinline__ void quantize_units(const float4 (&v)[NB], int e0, int k, uint32_t* smem) {
    constexpr int kPass = 256 * W;  // elements between a thread's units
    // |x| as integers: for non-negative floats the integer order is the
    // float order, and v_max_u32 takes a DPP operand directly; a NaN among
    // the bit patterns is the largest, so its sub-block's scale becomes NaN
    uint32_t mb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u)
        mb[u] = max(max(__float_as_uint(fabsf(v[u].x)), __float_as_uint(fabsf(v[u].y))),
                    max(__float_as_uint(fabsf(v[u].z)), __float_as_uint(fabsf(v[u].w))));
#pragma unroll
    for (int u = 0; u < NB; ++u) mb[u] = max(mb[u], (uint32_t)dpp_i<0xb1>((int)mb[u]));   // quad_perm [1,0,3,2]
#pragma unroll
    for (int u = 0; u < NB; ++u) mb[u] = max(mb[u], (uint32_t)dpp_i<0x4e>((int)mb[u]));   // quad_perm [2,3,0,1]
#pragma unroll
    for (int u = 0; u < NB; ++u) mb[u] = max(mb[u], (uint32_t)dpp_i<0x141>((int)mb[u]));  // the other quad of the 8
    float sc[NB];
    int X[NB][4];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        // sub-blocks below 1e-30 in magnitude are staged as zero; a NaN
        // maximum stays the scale (an infinite one gives inf * 0 = NaN)
        const float m = __uint_as_float(mb[u]);
        const bool live = m > 1e-30f;
        sc[u] = live ? m * (1.0f / kXMax) : (m == m ? 0.f : m);
        const float is = live ? __builtin_amdgcn_rcpf(m) * kXMax : 0.f;
        X[u][0] = __float2int_rn(v[u].x * is);
        X[u][1] = __float2int_rn(v[u].y * is);
        X[u][2] = __float2int_rn(v[u].z * is);
        X[u][3] = __float2int_rn(v[u].w * is);
    }
    // sums of the 16 X of each quad (every lane of the quad holds its sum)
    int t[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) t[u] = (X[u][0] + X[u][1]) + (X[u][2] + X[u][3]);
#pragma unroll
    for (int u = 0; u < NB; ++u) t[u] += dpp_i<0xb1>(t[u]);
#pragma unroll
    for (int u = 0; u < NB; ++u) t[u] += dpp_i<0x4e>(t[u]);
    // unit u sits kPass u elements on: limb_dwords(kPass) u padded limb
    // dwords, kPass / 32 u scales and kPass / 16 u sums further, so one
    // address per array serves every unit
    const int cap = xq_cap<W>(k), n = limb_dwords(cap);
    uint32_t* lo = smem + limb(e0 >> 2);
    uint32_t* mid = lo + n;
    uint32_t* hi = lo + 2 * n;
    uint32_t* scale = smem + 3 * n + (e0 >> 5);
    uint32_t* sum16 = smem + 3 * n + cap / 32 + (e0 >> 4);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        if (u > 0 && kPass * u >= cap) break;  // (uniform) passes beyond the arrays
        const uint32_t y0 = (uint32_t)X[u][0] + 0x8080u, y1 = (uint32_t)X[u][1] + 0x8080u;
        const uint32_t y2 = (uint32_t)X[u][2] + 0x8080u, y3 = (uint32_t)X[u][3] + 0x8080u;
        const uint32_t a01 = __builtin_amdgcn_perm(y1, y0, 0x05040100u);  // y0.b0 y0.b1 y1.b0 y1.b1
        const uint32_t a23 = __builtin_amdgcn_perm(y3, y2, 0x05040100u);
        lo[limb_dwords(kPass) * u] = __builtin_amdgcn_perm(a23, a01, 0x06040200u) ^ 0x80808080u;
        mid[limb_dwords(kPass) * u] = __builtin_amdgcn_perm(a23, a01, 0x07050301u) ^ 0x80808080u;
        const uint32_t h01 = __builtin_amdgcn_perm(y1, y0, 0x06020602u);  // y0.b2 y1.b2 (twice)
        const uint32_t h23 = __builtin_amdgcn_perm(y3, y2, 0x06020602u);
        hi[limb_dwords(kPass) * u] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
        scale[kPass / 32 * u] = __float_as_uint(sc[u]);
        sum16[kPass / 16 * u] = __float_as_uint(sc[u] * (float)t[u]);
    }
}

// Stage x as 24-bit block fixed point (see the file comment).  Thread t
// handles elements 4t + 1024u (u < NB, NB * 1024 >= k); all of its x (and
// norm weight) loads are issued before any arithmetic, so staging costs one
// memory latency.  With a norm weight x is first replaced by the reference
// rmsnorm x / sqrt(mean(x^2) + eps) * w (rmsnorm.cpp:5-26,
// transformer.cpp:189-214; float products where the reference rounds a
// double product to float, within 1 ulp); the sum of squares is reduced in
// double in a fixed order, so every workgroup stages identical values.
// x as stored in memory
struct PlainIn {
    const float* x;
    typedef float4 Raw;
    __device__ __forceinline__ Raw issue(int e) const { return *reinterpret_cast<const float4*>(x + e); }
    __device__ __forceinline__ float4 finish(const Raw& r) const { return r; }
};

// x of GEMV_ATTN: the decode attention's output, merged from its split
// partials (attention_run).  Element e lies in q head h = e / hd; split s
// left the running max m_s (base-2 units), the sum l_s and the exp-weighted
// V sums V_s over its positions, and the merged value is
// sum_s w_s V_s / sum_s w_s l_s with w_s = 2^(m_s - max_s m_s): the softmax
// of softmax.cpp:4-18 over the union of the splits' positions.  A split
// that held no position this step has m_s = -inf and weight 0 (its V sums
// are stale and are not used).
struct AttnIn {
    const float* part;
    int S, hd, nh;
    struct Raw {
        float4 v[kAttnMaxSplits];
        float2 ml[kAttnMaxSplits];
    };
    __device__ __forceinline__ Raw issue(int e) const {
        Raw r;
        const int h = e / hd, d = e - h * hd;
        const float* pv = part + (size_t)h * S * hd + d;
        const float* ml = part + (size_t)nh * S * hd + (size_t)h * S * 2;
#pragma unroll
        for (int s = 0; s < kAttnMaxSplits; ++s)
            if (s < S) {
                r.v[s] = *reinterpret_cast<const float4*>(pv + (size_t)s * hd);
                r.ml[s] = *reinterpret_cast<const float2*>(ml + 2 * s);
            }
        return r;
    }
    __device__ __forceinline__ float4 finish(const Raw& r) const {
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < kAttnMaxSplits; ++s)
            if (s < S) M = fmaxf(M, r.ml[s].x);
        float den = 0.f;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < kAttnMaxSplits; ++s) {
            if (s >= S) break;
            const float m = r.ml[s].x;
            if (m == -INFINITY) continue;
            const float w = __builtin_amdgcn_exp2f(m - M);
            den = fmaf(w, r.ml[s].y, den);
            a.x = fmaf(w, r.v[s].x, a.x);
            a.y = fmaf(w, r.v[s].y, a.y);
            a.z = fmaf(w, r.v[s].z, a.z);
            a.w = fmaf(w, r.v[s].w, a.w);
        }
        return make_float4(a.x / den, a.y / den, a.z / den, a.w / den);
    }
};

template <int W, int NB, bool NORM, class XS, class F>
__device__ __forceinline__ void stage_xq_nb(float* smem, const XS& xs, const float* __restrict__ nw,
                                            int k, float eps, double* red, F&& after_loads) {
    uint32_t* lo = reinterpret_cast<uint32_t*>(smem);
    constexpr int kStep = 256 * W;
    const int base = threadIdx.x * 4;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    typename XS::Raw raw[NB];
    float4 v[NB], g[NORM ? NB : 1];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const int e = base + u * kStep;
        // unconditional (clamped) loads keep the count of outstanding loads
        // static for the explicit wait in after_loads; out-of-range values
        // are replaced by zero only after that wait
        const int ec = e < k ? e : k - 4;
        raw[u] = xs.issue(ec);
        if (NORM) g[u] = *reinterpret_cast<const float4*>(nw + ec);
    }
    // issues the first weight steps (younger than x) and waits for x only
    after_loads();
#pragma unroll
    for (int u = 0; u < NB; ++u) v[u] = base + u * kStep >= k ? z : xs.finish(raw[u]);
    if (NORM) {
        // per-thread float partials (at most 64 squares), summed in double
        float sf = 0.f;
#pragma unroll
        for (int u = 0; u < NB; ++u)
            sf = fmaf(v[u].x, v[u].x, fmaf(v[u].y, v[u].y, fmaf(v[u].z, v[u].z, fmaf(v[u].w, v[u].w, sf))));
        const double ss = wave_sum_d_lane63((double)sf);
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float inv = (float)rsqrt_d(block_sum<W>(red) / (double)k + (double)eps);
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            v[u].x = v[u].x * inv * g[u].x;
            v[u].y = v[u].y * inv * g[u].y;
            v[u].z = v[u].z * inv * g[u].z;
            v[u].w = v[u].w * inv * g[u].w;
        }
    }
    // units past k hold zeros and store into the spare dword
    quantize_units<W, NB>(v, base, k, lo);
    __syncthreads();
}

// Staging for K above what one thread keeps in registers (k > 12288, or
// k > 4096 with a norm): the same values, x read again per pass.
template <int W>
__device__ __noinline__ void stage_xq_2pass(float* smem, const float* __restrict__ x, const float* __restrict__ nw,
                                            int k, float eps, double* red) {
    // (the first weight steps are issued by the caller before this call)
    uint32_t* lo = reinterpret_cast<uint32_t*>(smem);
    constexpr int kStep = 256 * W;
    double inv = 1.0;
    if (nw) {
        double ss = 0.0;
        for (int e = threadIdx.x * 4; e < k; e += kStep) {
            const float4 v = *reinterpret_cast<const float4*>(x + e);
            ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
        }
        ss = wave_sum_d_lane63(ss);
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        inv = 1.0 / sqrt(block_sum<W>(red) / (double)k + (double)eps);
    }
    // the trip count is uniform across the workgroup (k is a multiple of 32
    // and every pass covers kStep elements), so the DPP runs convergent
    for (int b = 0; b < k; b += kStep) {
        const int e = b + threadIdx.x * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f), g = v;
        if (e < k) v = *reinterpret_cast<const float4*>(x + e);
        if (nw) {
            if (e < k) g = *reinterpret_cast<const float4*>(nw + e);
            v.x = (float)((double)v.x * inv) * g.x;
            v.y = (float)((double)v.y * inv) * g.y;
            v.z = (float)((double)v.z * inv) * g.z;
            v.w = (float)((double)v.w * inv) * g.w;
        }
        const float4 u1[1] = {v};
        quantize_units<W, 1>(u1, e, k, lo);
    }
    __syncthreads();
}

// Stage x (limb layout) and issue the first weight loads through
// `issue_first` right after the x loads.
template <int W, class F>
__device__ __forceinline__ void stage_xq(float* smem, const float* __restrict__ x, const float* __restrict__ nw,
                                         int k, float eps, double* red, F&& issue_first) {
    const int nb = (k + 256 * W - 1) / (256 * W);
    // register budget: the two weight buffers issued during staging stay
    // live, so at most 48 staged registers (x, and the norm weight)
    const PlainIn xs{x};
    if (nw) {
        if constexpr (W > kWaves) {
            if (nb <= 1) return stage_xq_nb<W, 1, true>(smem, xs, nw, k, eps, red, issue_first);
            if (nb <= 2) return stage_xq_nb<W, 2, true>(smem, xs, nw, k, eps, red, issue_first);
        }
        if (nb <= 4) return stage_xq_nb<W, 4, true>(smem, xs, nw, k, eps, red, issue_first);
    } else {
        if (nb <= 4) return stage_xq_nb<W, 4, false>(smem, xs, nw, k, eps, red, issue_first);
        if (nb <= 8) return stage_xq_nb<W, 8, false>(smem, xs, nw, k, eps, red, issue_first);
        if (nb <= 12) return stage_xq_nb<W, 12, false>(smem, xs, nw, k, eps, red, issue_first);
    }
    issue_first();
    stage_xq_2pass<W>(smem, x, nw, k, eps, red);
}

// Staging of GEMV_ATTN (k <= 4096): the attention partials merged by
// AttnIn, in as many units per thread as k needs (a unit past k would load
// every split's partial for nothing), then quantized as any x.
template <int W, class F>
__device__ __forceinline__ void stage_attn(float* smem, const GemvArgs& a, double* red, F&& issue_first) {
    const AttnIn in{a.part, a.part_splits, a.part_hd, a.k / a.part_hd};
    const int nb = (a.k + 256 * W - 1) / (256 * W);
    if constexpr (4096 / (256 * W) >= 4) {
        if (nb > 2) return stage_xq_nb<W, 4096 / (256 * W), false>(smem, in, nullptr, a.k, a.eps, red, issue_first);
    }
    if constexpr (4096 / (256 * W) >= 2) {
        if (nb > 1) return stage_xq_nb<W, 2, false>(smem, in, nullptr, a.k, a.eps, red, issue_first);
    }
    stage_xq_nb<W, 1, false>(smem, in, nullptr, a.k, a.eps, red, issue_first);
}

// Output modes (epilogues) of one GEMV launch.
//  GEMV_PLAIN : y[r] = W[r].x (+ res[r])
//  GEMV_SILU  : W = [gate; up] with n = 2F rows; y[i] = silu(gate_i) * up_i
//               (transformer.cpp:183-185, 696-704) for i < F
//  GEMV_ARGMAX: y = logits; each workgroup also leaves its (largest logit,
//               lowest index) in red_val/red_idx[blockIdx] for argmax_finish
//  GEMV_ATTN  : as PLAIN, with x merged from the decode attention's split
//               partials in the staging (AttnIn; k <= 4096, no norm)
// f(integral_constant<int, K>) for K = 0 .. N-1, expanded at compile time
// (a plain unrolled loop over a register array may be left rolled, which
// sends the array to scratch memory)
template <class F, int... K>
__device__ __forceinline__ void for_each_k(F&& f, std::integer_sequence<int, K...>) {
    (f(std::integral_constant<int, K>{}), ...);
}

// NS = 0: persistent loop, one step of loads ahead.  NS > 0: short form,
// at most NS steps per wave (the launcher sizes the grid for it).
template <template <int> class T, int R, int MODE, int NS, int W = kWaves>
// The arguments a wave needs first (weights, x, norm weight, n, k) also come
// as leading scalars, which the command processor preloads into SGPRs
// (-amdgpu-kernarg-preload-count), so the first loads do not wait for a
// kernel-argument fetch; the rest stay in GemvArgs.  W waves per workgroup.
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint8_t* pw, const float* px, const float* pnw, int pn,
                                                        int pk, GemvArgs a) {
    a.w = pw;
    a.x = px;
    a.norm_w = pnw;
    a.n = pn;
    a.k = pk;
    using Ty = T<R>;
    using Buf = typename Ty::Buf;
    extern __shared__ float xs[];
    __shared__ double red[W];
    __shared__ float wmax[W];
    __shared__ int widx[W];

    // wave index in an SGPR: every per-wave quantity below is provably
    // uniform, so the pipeline's branches are scalar and its waits exact
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // rows a wave accumulates at once; in SILU mode rows [j] and [R/2 + j]
    // are the gate and up rows of output i0 + j
    constexpr int kOut = MODE == GEMV_SILU ? R / 2 : R;
    const int n_out = MODE == GEMV_SILU ? a.n / 2 : a.n;
    const int n_groups = (n_out + kOut - 1) / kOut;
    const int nchunks = a.k >> Ty::kChunkShift;  // chunks of 32 (64 for Q4_K) elements
    const int cpl = (nchunks + 63) >> 6;         // chunk steps per lane per row group
    const size_t rbytes = row_bytes(Ty::kType, a.k);
    const int wave_id = blockIdx.x * W + wave, n_waves = gridDim.x * W;
    const int my_groups = wave_id < n_groups ? (n_groups - 1 - wave_id) / n_waves + 1 : 0;
    const int total = my_groups * cpl;           // (row group, chunk step) pairs of this wave
    float best = -INFINITY;
    int best_i = 0x7fffffff;

    // (chunk step j, row-group ordinal g) cursors: one issues weight loads
    // ahead, one consumes; the loops are unrolled so the register buffers
    // keep fixed names (no copies, no dynamic indexing)
    struct Cursor {
        int j, g;
    };
    const auto xview = [&] {  // layout of the staged x (filled below)
        if constexpr (Ty::kIntX) return xq_view<W>(xs, a.k);
        else return (const float*)xs;
    }();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    // PLAIN mode also prefetches the residual of the row group with each step
    constexpr bool kRes = MODE == GEMV_PLAIN || MODE == GEMV_ATTN;
    constexpr int kL = Ty::kLoads * R + (kRes ? kOut : 0);  // vector loads per step
    static_assert(kL <= 63, "a step's loads fit the wait counter");
    const float* res_src = a.res ? a.res : a.y;  // (not used without a residual)
    struct Step {
        Buf b;
        float rs[kRes ? kOut : 1];
    };
    // every step issues exactly kL loads (chunk and row indices clamped in
    // bounds), so the explicit waits below can count them
    // A step past the wave's last one repeats the last step's addresses (its
    // loads hit lines already in flight and its data is never consumed).
    // both lambdas are inlined at every use: a call would put the state they
    // capture by reference (kernel arguments, cursors, buffers) in scratch
    auto issue = [&](Cursor& cu, Step& st) __attribute__((always_inline)) {
        const bool past = cu.g >= my_groups;
        const int gi = past ? my_groups - 1 : cu.g, ji = past ? cpl - 1 : cu.j;
        const int grp = wave_id + gi * n_waves;
        int rows[R];
#pragma unroll
        for (int r = 0; r < kOut; ++r) {
            const int o = min(max(grp * kOut + r, 0), n_out - 1);
            rows[r] = o;
            if (MODE == GEMV_SILU) rows[kOut + r] = o + n_out;
            if constexpr (kRes) st.rs[r] = res_src[o];
        }
        // past the end every lane reads the same bytes: the loads only keep
        // the count of outstanding operations uniform and cost no bandwidth
        const int c = past ? 0 : min(lane + 64 * ji, nchunks - 1);
        Ty::load(a.w, rbytes, rows, c, st.b);
        if (++cu.j == cpl) {
            cu.j = 0;
            ++cu.g;
        }
    };
    auto consume = [&](Cursor& cu, const Step& st) __attribute__((always_inline)) {
        const int c = lane + 64 * cu.j;
        if (c < nchunks) Ty::compute(st.b, c, xview, a.form, acc);
        if (cu.j == cpl - 1) {
            // row group complete: reduce across lanes (total lands in lane 63) and write
            const int grp = wave_id + cu.g * n_waves;
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = wave_sum_lane63(acc[r]);
            if (lane == 63) {
#pragma unroll
                for (int r = 0; r < kOut; ++r) {
                    const int o = grp * kOut + r;
                    if (o < n_out) {
                        float v;
                        if constexpr (MODE == GEMV_SILU) {
                            const float gt = acc[r];
                            v = gt / (1.0f + expf(-gt)) * acc[kOut + r];
                        } else if constexpr (kRes) {
                            v = a.res ? acc[r] + st.rs[r] : acc[r];
                        } else {
                            v = acc[r];
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
        if (++cu.j == cpl) {
            cu.j = 0;
            ++cu.g;
        }
    };
    Cursor ci{0, 0}, cc{0, 0};
    if constexpr (NS > 0) {
        // The first step's weight loads are issued right after the x loads,
        // and each later step's just before the step ahead of it is consumed,
        // in straight-line code with fixed load counts whose waits the
        // compiler's own analysis leaves alone.  A wave issues its loads in
        // order and stalls at issue while the CU's memory queue is full, so
        // loads queued ahead of the staging or of a step's arithmetic delay
        // that arithmetic: every step issued before the staging (24 loads per
        // wave) ran at 551 tok/s, one step first 579, none first 543.
        // steps of loads issued ahead of consumption (two: 589 against 600-606 tok/s)
        constexpr int kAhead = 1;
        static_assert((kAhead + 1) * kL <= 63, "short form: the loads in flight fit the wait counter");
        Step sb[NS];
        auto issue_all = [&] {
            // every wave's x loads are issued before any wave's weight loads,
            // so x is not queued behind weights in the CU's memory pipeline
            // (a bare s_barrier: no wait for the loads themselves)
            __builtin_amdgcn_s_barrier();
            for_each_k([&](auto kc) { issue(ci, sb[decltype(kc)::value]); }, std::make_integer_sequence<int, kAhead>{});
            wait_vmcnt<kAhead * kL>();
        };
        if constexpr (MODE == GEMV_ATTN) {
            stage_attn<W>(xs, a, red, issue_all);
        } else if constexpr (Ty::kIntX) {
            stage_xq<W>(xs, a.x, a.norm_w, a.k, a.eps, red, issue_all);
        } else {
            issue_all();
            stage_x<W>(xs, a.x, a.norm_w, a.k, a.eps, red);
        }
        // then step K + kAhead is issued before step K is consumed: a wave
        // never has more than kAhead + 1 steps of loads queued, so its
        // consumption does not wait behind stalled issues (all steps queued
        // after the staging: 589 against 606 tok/s).  Steps past the wave's
        // last are issued as well: branching between two wait counts there
        // let the compiler add waits of its own (559 against 599 tok/s).
        for_each_k(
            [&](auto kc) {
                constexpr int K = decltype(kc)::value;
                if constexpr (K + kAhead < NS) {
                    issue(ci, sb[K + kAhead]);
                    wait_vmcnt<kAhead * kL>();
                } else {
                    wait_vmcnt<(NS - 1 - K) * kL>();
                }
                if (K < total) consume(cc, sb[K]);
            },
            std::make_integer_sequence<int, NS>{});
    } else {
        Step s0, s1;
        // the first step's weight loads do not depend on x: they are issued
        // right after the x loads, so both latencies overlap, and the staging
        // arithmetic waits for x only (two steps before it: 580 against 588
        // tok/s)
        auto issue_first = [&] {
            issue(ci, s0);
            wait_vmcnt<kL>();
        };
        if constexpr (MODE == GEMV_ATTN) {
            stage_attn<W>(xs, a, red, issue_first);
        } else if constexpr (Ty::kIntX) {
            stage_xq<W>(xs, a.x, a.norm_w, a.k, a.eps, red, issue_first);
        } else {
            issue_first();
            stage_x<W>(xs, a.x, a.norm_w, a.k, a.eps, red);
        }
        // then one step ahead: step j + 1 is issued just before step j is
        // consumed (two steps ahead measured the same at 12-350 MB shapes and
        // 1-2% slower on the lm-head)
        for (int it = 0; it < total; it += 2) {
            if (it + 1 < total) {
                issue(ci, s1);
                wait_vmcnt<kL>();
            } else {
                wait_vmcnt<0>();
            }
            consume(cc, s0);
            if (it + 1 >= total) break;
            if (it + 2 < total) {
                issue(ci, s0);
                wait_vmcnt<kL>();
            } else {
                wait_vmcnt<0>();
            }
            consume(cc, s1);
        }
    }
    if constexpr (MODE == GEMV_ARGMAX) {
        if (lane == 63) {
            wmax[wave] = best;
            widx[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = wmax[0];
            int bi = widx[0];
            for (int w2 = 1; w2 < W; ++w2)
                if (wmax[w2] > bv || (wmax[w2] == bv && widx[w2] < bi)) {
                    bv = wmax[w2];
                    bi = widx[w2];
                }
            a.red_val[blockIdx.x] = bv;
            a.red_idx[blockIdx.x] = bi;
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

// Resident workgroups of a kernel on the whole device (occupancy x CUs),
// cached per kernel and LDS size: a persistent grid of exactly this size runs
// in one round, so each resident slot stages x once.
int device_cus() {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n_cu = 256;
    }
    return n_cu;
}

int resident_grid(const void* kernel, size_t lds, int threads) {
    struct Entry {
        const void* k;
        size_t lds;
        int grid;
    };
    static Entry cache[64];
    static int n_cache = 0;
    for (int i = 0; i < n_cache; ++i)
        if (cache[i].k == kernel && cache[i].lds == lds) return cache[i].grid;
    const int n_cu = device_cus();
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int grid = per_cu * n_cu;
    if (n_cache < 64) cache[n_cache++] = Entry{kernel, lds, grid};
    return grid;
}

// Epilogue modes built per wave count in launch_gemv: every mode at kWaves,
// the plain and attention-merge epilogues at eight waves.  GEMV_ATTN only
// for the quantized formats (their staging merges the attention partials),
// GEMV_ARGMAX only in the loop form, and the kSiluShortSteps form for
// SwiGLU only.
constexpr bool mode_built(int W, int mode) {
    return W == kWaves || (W == 8 && (mode == GEMV_PLAIN || mode == GEMV_ATTN));
}
template <template <int> class T, int R, int MODE, int NS, int W>
constexpr bool has_instance() {
    if constexpr (!mode_built(W, MODE) || (MODE == GEMV_ATTN && !T<R>::kIntX) || (MODE == GEMV_ARGMAX && NS != 0))
        return false;
    else
        return !(NS == kSiluShortSteps && NS != kShortSteps && MODE != GEMV_SILU);
}

// f(integral_constant<int, MODE>) for the built instance of `mode`, if any
template <template <int> class T, int R, int NS, int W, class F>
__host__ bool with_instance(int mode, F&& f) {
    bool done = false;
    auto pick = [&](auto m) {
        constexpr int M = decltype(m)::value;
        if constexpr (has_instance<T, R, M, NS, W>()) {
            if (mode == M) {
                f(m);
                done = true;
            }
        }
    };
    pick(std::integral_constant<int, GEMV_PLAIN>{});
    pick(std::integral_constant<int, GEMV_SILU>{});
    pick(std::integral_constant<int, GEMV_ARGMAX>{});
    pick(std::integral_constant<int, GEMV_ATTN>{});
    return done;
}

template <template <int> class T, int R, int NS, int W>
const void* kernel_for(int mode) {
    const void* k = nullptr;
    with_instance<T, R, NS, W>(mode, [&](auto m) { k = (const void*)gemv_kernel<T, R, decltype(m)::value, NS, W>; });
    return k;
}

template <template <int> class T, int R, int NS, int W>
void launch_mode(int mode, unsigned grid, size_t lds, const GemvArgs& a, hipStream_t st) {
    with_instance<T, R, NS, W>(mode, [&](auto m) {
        hipLaunchKernelGGL((gemv_kernel<T, R, decltype(m)::value, NS, W>), dim3(grid), dim3(64 * W), lds, st, a.w,
                           a.x, a.norm_w, a.n, a.k, a);
    });
}

template <template <int> class T, int R, int W = kWaves>
int launch_gemv(const GemvArgs& a, int mode, hipStream_t st, int grid_cap = 0) {
    if (!mode_built(W, mode)) return MXH_ERR_UNSUPPORTED;
    const int kout = mode == GEMV_SILU ? R / 2 : R;
    const int64_t n_out = mode == GEMV_SILU ? a.n / 2 : a.n;
    const int64_t n_groups = (n_out + kout - 1) / kout;
    const int64_t need = (n_groups + W - 1) / W;
    const int64_t cpl = ((a.k >> T<R>::kChunkShift) + 63) >> 6;  // chunk steps per row group
    // fp32 x with padding, or the limb layout (2 bytes + 3/16 floats per element)
    const size_t lds = T<R>::kIntX ? (size_t)xq_dwords<W>(a.k) * 4
                                   : (size_t)(a.k + (a.k >> 4)) * sizeof(float);
    const int n_cu = device_cus();
    // Short form: when every wave can finish in at most NS steps with a
    // resident grid, one workgroup per CU where that suffices (x is staged
    // and quantized once per CU), more where NS steps per wave need it.
    constexpr int kLmax = T<R>::kLoads * R + R;  // loads per step, residual included
    if constexpr (3 * kLmax <= 63) {
        if (mode != GEMV_ARGMAX && grid_cap <= 0 && cpl <= 3) {
            auto try_short = [&](auto nsc) -> bool {
                constexpr int NSv = decltype(nsc)::value;
                if constexpr (2 * kLmax > 63) {
                    return false;
                } else {
                    if (NSv < cpl) return false;  // a row group's chunk steps exceed the form
                    const int64_t per_wg = (int64_t)W * (NSv / cpl);
                    const int64_t min_grid = (n_groups + per_wg - 1) / per_wg;
                    int64_t grid = need < n_cu ? need : n_cu;
                    if (grid < min_grid) grid = min_grid;
                    if (grid > resident_grid(kernel_for<T, R, NSv, W>(mode), lds, 64 * W)) return false;
                    launch_mode<T, R, NSv, W>(mode, (unsigned)grid, lds, a, st);
                    return true;
                }
            };
            // steps per wave with one workgroup per CU
            const int64_t steps_one_per_cu = (n_groups + (int64_t)n_cu * W - 1) / ((int64_t)n_cu * W) * cpl;
            if constexpr (W == kWaves) {
                // the longer SwiGLU form only where one workgroup per CU would
                // leave waves more than kShortSteps steps
                if (mode == GEMV_SILU && steps_one_per_cu > kShortSteps &&
                    try_short(std::integral_constant<int, kSiluShortSteps>{}))
                    return MXH_OK;
            }
            // A wave issues the steps past its last too (to keep the wait
            // counts fixed), so where one workgroup per CU leaves each wave
            // one or two steps, the form of exactly that many (the eight-wave
            // o-projection in one step instead of three: 655 against 643
            // tok/s)
            if (steps_one_per_cu == 1 && try_short(std::integral_constant<int, 1>{})) return MXH_OK;
            if (steps_one_per_cu == 2 && try_short(std::integral_constant<int, 2>{})) return MXH_OK;
            if (try_short(std::integral_constant<int, kShortSteps>{})) return MXH_OK;
        }
    }
    int cap = grid_cap > 0 ? grid_cap : resident_grid(kernel_for<T, R, 0, W>(mode), lds, 64 * W);
    // Short runs (a few row groups per wave with one workgroup per CU): one
    // workgroup per CU, so x is staged and quantized once per CU and no CU
    // carries two workgroups' staging while others carry one.  Long runs keep
    // the resident occupancy, whose extra waves hide latency.
    if (grid_cap <= 0 && need > n_cu && (n_groups + (int64_t)n_cu * W - 1) / ((int64_t)n_cu * W) <= 8)
        cap = n_cu;
    const unsigned grid = (unsigned)(need < cap ? need : cap);
    if constexpr (W == kWaves) {
        if (mode == GEMV_ARGMAX) {
            if ((int)grid > a.red_cap) return MXH_ERR_ARG;
            hipLaunchKernelGGL((gemv_kernel<T, R, GEMV_ARGMAX, 0>), dim3(grid), dim3(kThreads), lds, st, a.w, a.x,
                               a.norm_w, a.n, a.k, a);
            hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1024), 0, st, a.red_val, a.red_idx, (int)grid,
                               a.tokens, a.pos);
            return MXH_OK;
        }
    }
    launch_mode<T, R, 0, W>(mode, grid, lds, a, st);
    return MXH_OK;
}

// W waves per workgroup and one workgroup per CU where the row groups give
// every wave exactly one step (rows with the fused rmsnorm, or SwiGLU rows) or
// exactly kSiluShortSteps (SwiGLU), with one chunk step per row group.  x is
// staged once per CU for all W waves and no wave issues steps past its last.
// Twelve waves for Q4_K (the Qwen3-8B q|k|v in one step, gate|up in four:
// 660 against 653 tok/s; q|k|v alone 658, gate|up alone 653), then fourteen
// and ten (the Llama-3-8B gate|up in four, its q|k in one: config 4 546 ->
// 558 tok/s), six for Q8_0 (the Qwen3-0.6B gate|up in one step).  False
// where the shape does not fit.
template <template <int> class T, int R, int W>
bool launch_exact(const GemvArgs& a, int mode, hipStream_t st) {
    if (a.k > 64 << T<R>::kChunkShift || (mode == GEMV_PLAIN ? !a.norm_w : mode != GEMV_SILU)) return false;
    const int64_t n_groups = mode == GEMV_SILU ? a.n / R : (a.n + R - 1) / R;
    const int64_t n_cu = device_cus(), per = n_cu * W;
    if (n_groups % per) return false;
    const int64_t steps = n_groups / per;
    const size_t lds = (size_t)xq_dwords<W>(a.k) * 4;
    auto go = [&](auto kern) {
        if (resident_grid((const void*)kern, lds, 64 * W) < n_cu) return false;
        hipLaunchKernelGGL(kern, dim3(n_cu), dim3(64 * W), lds, st, a.w, a.x, a.norm_w, a.n, a.k, a);
        return true;
    };
    if (mode == GEMV_SILU) {
        if (steps == 1) return go(gemv_kernel<T, R, GEMV_SILU, 1, W>);
        if (steps == kSiluShortSteps) return go(gemv_kernel<T, R, GEMV_SILU, kSiluShortSteps, W>);
        return false;
    }
    return steps == 1 && go(gemv_kernel<T, R, GEMV_PLAIN, 1, W>);
}

}  // namespace

// max K whose padded x fits the 64 KiB of LDS one workgroup may use
constexpr int64_t kGemvMaxK = 15360;

int gemv_run(int type, const GemvArgs& a, int mode, hipStream_t st) {
    if (a.k % 32 || a.k > kGemvMaxK || a.n <= 0 || (mode == GEMV_SILU && a.n % 2)) return MXH_ERR_ARG;
    // the attention merge: at most 4096 inputs (one staging pass), quantized
    // weights, whole q heads of 4 to 128 elements, no norm
    if (mode == GEMV_ATTN &&
        (a.k > 4096 || !a.part || a.norm_w || a.part_splits < 1 || a.part_splits > kAttnMaxSplits ||
         a.part_hd < 4 || a.part_hd > 128 || a.part_hd % 4 || a.k % a.part_hd || !gemv_int_x(type)))
        return MXH_ERR_ARG;
    if (mode == GEMV_ARGMAX && (!a.red_val || !a.red_idx || !a.tokens || !a.pos)) return MXH_ERR_ARG;
    switch (type) {
    case MXH_Q4_K: return launch_gemv<Q4K, 4>(a, mode, st);
    case MXH_Q4_K_TILED:
        // eight waves per workgroup for long plain rows (x staged once per
        // CU for eight waves: the 4096 x 12288 down projection), and for the
        // o-projection's attention merge above 2048 inputs (each thread
        // merges half as many elements: 643 against 625 tok/s)
        if (mode == GEMV_PLAIN && a.k > 8192 && !a.norm_w && xq_dwords<8>(a.k) * 4 <= 65536)
            return launch_gemv<Q4KT, 2, 8>(a, mode, st);
        if (mode == GEMV_ATTN && a.k > 2048) return launch_gemv<Q4KT, 2, 8>(a, mode, st);
        if (launch_exact<Q4KT, 2, 12>(a, mode, st) || launch_exact<Q4KT, 2, 14>(a, mode, st) ||
            launch_exact<Q4KT, 2, 10>(a, mode, st))
            return MXH_OK;
        return launch_gemv<Q4KT, 2>(a, mode, st);
    case MXH_Q8_0_TILED:
        // plain rows without a norm and the attention merge at two rows per
        // wave, so few row groups still fill more CUs (Qwen3-0.6B o and down:
        // 128 workgroups instead of 64; config 1 1,476 -> 1,537 tok/s)
        if (mode == GEMV_ATTN || (mode == GEMV_PLAIN && !a.norm_w)) return launch_gemv<Q80T, 2>(a, mode, st);
        if (launch_exact<Q80T, 4, 6>(a, mode, st)) return MXH_OK;
        return launch_gemv<Q80T, 4>(a, mode, st);
    case MXH_Q5_K_TILED:
        // two rows per wave, so the row groups fill more CUs (Llama-3-8B's
        // 4096 x 14336 down projection at eight waves: 256 workgroups instead
        // of 128, config 4 491 -> 535 tok/s; its 1024-row v: 547)
        if (mode == GEMV_PLAIN && a.k > 8192 && !a.norm_w && xq_dwords<8>(a.k) * 4 <= 65536)
            return launch_gemv<Q5KT, 2, 8>(a, mode, st);
        return launch_gemv<Q5KT, 2>(a, mode, st);
    case MXH_Q6_K_TILED:
        // eight waves for long plain rows, as for Q4_K (the Q6_K ffn_down of
        // Q4_K_M files: 4096 x 12288 / 14336)
        if (mode == GEMV_PLAIN && a.k > 8192 && !a.norm_w && xq_dwords<8>(a.k) * 4 <= 65536)
            return launch_gemv<Q6KT, 2, 8>(a, mode, st);
        return launch_gemv<Q6KT, 2>(a, mode, st);
    case MXH_Q5_K: return launch_gemv<Q5K, 4>(a, mode, st);
    case MXH_Q6_K: return launch_gemv<Q6K, 2>(a, mode, st);
    case MXH_Q8_0: return launch_gemv<Q80, 4>(a, mode, st);
    case MXH_Q5_0: return launch_gemv<Q50, 4>(a, mode, st);
    case MXH_F16: return launch_gemv<F16W, 2>(a, mode, st);
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
