// mxh_prefill_q4k.hip — the prefill GEMM for quantized weights on the fp16
// matrix cores, with every weight exact.
//
// out[m][n] = sum_k a[m][k] w[n][k].  K-quant rows (Q4_K, Q5_K:
// w = d sc_j q - dmin m_j, tensor.cpp:405-432; sub-block j of 32 elements
// inside a 256-element super-block with one d, dmin) are regrouped as
//
//   sum_b d_b[n] . sum_{k in b} a[m][k] (sc_j q_k)          main MFMAs
//   - sum_j dmin[n] m_j . S_j[m],   S_j = sum_{k in j} a[m][k]   correction MFMAs
//
// sc_j q_k is an integer below 2048, exact in fp16, so no weight is rounded:
// the tile holds those integers, d is applied once per super-block to a
// per-block accumulator, and the min terms are a small second contraction
// over sub-blocks (16 at a time).  Rows of 32-element blocks (Q8_0: w = d q,
// Q5_0: w = d (q - 16); tensor.cpp:434-457) hold the integers q (q - 16) in
// the tile and apply d once per block; they need no correction.
// Activations come as a' = a 2^e (e per row, so max |a'| lies in
// [128, 256)) split into fp16 hi + lo (about 22 significant bits), with the
// sub-block sums S of the same values split the same way (rows_to_f16 /
// silu_mul_f16 below); the output is scaled back by 2^-e.  Reference op:
// backend_matmul_rhs_transposed with m > 1
// (src/backend/backend_runtime.cpp:302-319).
//
// Tiles: 128 x TN outputs per workgroup of 2 TN / 64 waves (TN = 128 or
// 256 weight rows, q4_wide_tiles below), each wave 64 x 64 as
// 2 x 2 blocks of v_mfma_f32_32x32x16_f16 (lane l supplies row / column
// l % 32 at k = 8 (l / 32) .. +8; accumulator register i of lane l is row
// 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32).  K steps of 64 elements
// (two sub-blocks); the next step's global loads fly during the MFMAs.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kQM = 128, kQK = 64;  // tile rows (activations) and K step; TN weight rows per tile
constexpr int kQLd = kQK + 8;   // tile row stride in fp16 (144 bytes)
constexpr int kRing = 16;       // sub-blocks per correction round
constexpr int kRLd = kRing + 8; // ring row stride in fp16 (48 bytes)
template <int TN>
constexpr size_t q4_lds_bytes() {
    return (size_t)((2 * kQM + TN) * kQLd + 2 * (kQM + TN) * kRLd) * 2 + 2 * TN * sizeof(float);
}

__device__ __forceinline__ uint16_t f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

// fp16 hi + lo of v (lo = v - hi rounded again) as hi | lo << 16
__device__ __forceinline__ uint32_t split_f16(float v) {
    const __half h = __float2half_rn(v);
    return (uint32_t)__half_as_ushort(h) | ((uint32_t)f16_bits(v - __half2float(h)) << 16);
}

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    // both are integers below 2048: round-toward-zero packing is exact
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Weight formats.  Thread (row r, half h) of a K step at k0 fetches the
// bytes of elements k0 + 32 h .. +31 of its row (fetch, a step ahead) and
// decodes them (decode) into 16 dwords of fp16 integers, with
//   K-quants:   o = sc_j q, d = the super-block's d, mt = -dmin m_j;
//   32-blocks:  o = q (Q5_0: q - 16), d = the block's d.
enum WFmt { WF_Q4K, WF_Q4KT, WF_Q5K, WF_Q5KT, WF_Q80, WF_Q80T, WF_Q50 };

template <int F>
struct WFormat;

// Q4_K: the header and the 32 qs bytes of 64-group g = (k0 % 256) / 64
template <bool TILED>
struct WQ4K {
    static constexpr bool kKQuant = true;
    uint4 hd, qa, qb;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int) {
        const uint8_t* rp = w + (size_t)row * rb;
        if constexpr (TILED) {
            const Q4KTileOffs o = q4k_tile_offsets(k0 >> 6, (int64_t)(rb / 144));
            hd = ld16(rp + o.hd);
            qa = ld16(rp + o.qa);
            qb = ld16(rp + o.qb);
        } else {
            const uint8_t* blk = rp + (size_t)(k0 >> 8) * 144;
            const int g = (k0 & 255) >> 6;
            hd = ld16(blk);
            qa = ld16(blk + 16 + 32 * g);
            qb = ld16(blk + 32 + 32 * g);
        }
    }
    // sub-block j = 2 g + h (tensor.cpp:395-432 with the scale form `form`);
    // byte i of the group's 32 qs holds element i (low nibble) and 32 + i
    // (high nibble)
    __device__ __forceinline__ void decode(int k0, int h, int form, uint32_t (&o)[16], float& d, float& mt) const {
        const int j = 2 * ((k0 & 255) >> 6) + h;
        uint32_t sc, mn;
        k4_scale_min(hd.y, hd.z, hd.w, j, form, sc, mn);
        const float scf = (float)sc;
        const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t nb = (qv[i] >> (4 * h)) & 0x0f0f0f0fu;
            o[2 * i] = pk_f16((float)(nb & 0xffu) * scf, (float)((nb >> 8) & 0xffu) * scf);
            o[2 * i + 1] = pk_f16((float)((nb >> 16) & 0xffu) * scf, (float)(nb >> 24) * scf);
        }
        d = half_bits_to_float(hd.x & 0xffffu);
        mt = -(half_bits_to_float(hd.x >> 16) * (float)mn);
    }
};
template <> struct WFormat<WF_Q4K> : WQ4K<false> {};
template <> struct WFormat<WF_Q4KT> : WQ4K<true> {};

// Q5_K (published ggml layout): the header, the 32 qh bytes (the fifth bit
// of element 64 g + 32 h + i is bit 2 g + h of qh[i]) and the group's 32 qs
template <bool TILED>
struct WQ5K {
    static constexpr bool kKQuant = true;
    uint4 hd, h0, h1, qa, qb;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int) {
        const uint8_t* rp = w + (size_t)row * rb;
        const int g = (k0 & 255) >> 6;
        if constexpr (TILED) {
            // chunks 2 g and 2 g + 1 of the block: adjacent 16-byte qs pieces
            const Q5KTileOffs o = q5k_tile_offsets(8 * (int64_t)(k0 >> 8) + 2 * g, (int64_t)(rb / 176));
            hd = ld16(rp + o.hd);
            h0 = ld16(rp + o.qh);
            h1 = ld16(rp + o.qh + 16);
            qa = ld16(rp + o.qs);
            qb = ld16(rp + o.qs + 16);
        } else {
            const uint8_t* blk = rp + (size_t)(k0 >> 8) * 176;
            hd = ld16(blk);
            h0 = ld16(blk + 16);
            h1 = ld16(blk + 32);
            qa = ld16(blk + 48 + 32 * g);
            qb = ld16(blk + 64 + 32 * g);
        }
    }
    __device__ __forceinline__ void decode(int k0, int h, int form, uint32_t (&o)[16], float& d, float& mt) const {
        const int j = 2 * ((k0 & 255) >> 6) + h;
        uint32_t sc, mn;
        k4_scale_min(hd.y, hd.z, hd.w, j, form, sc, mn);
        const float scf = (float)sc;
        const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const uint32_t hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t nb = ((qv[i] >> (4 * h)) & 0x0f0f0f0fu) | (((hv[i] >> j) & 0x01010101u) << 4);
            o[2 * i] = pk_f16((float)(nb & 0xffu) * scf, (float)((nb >> 8) & 0xffu) * scf);
            o[2 * i + 1] = pk_f16((float)((nb >> 16) & 0xffu) * scf, (float)(nb >> 24) * scf);
        }
        d = half_bits_to_float(hd.x & 0xffffu);
        mt = -(half_bits_to_float(hd.x >> 16) * (float)mn);
    }
};
template <> struct WFormat<WF_Q5K> : WQ5K<false> {};
template <> struct WFormat<WF_Q5KT> : WQ5K<true> {};

// four signed bytes as two dwords of fp16 integers
__device__ __forceinline__ void sbytes_f16(uint32_t v, uint32_t& lo, uint32_t& hi) {
    lo = pk_f16((float)(int)(int8_t)(v & 0xffu), (float)(int)(int8_t)((v >> 8) & 0xffu));
    hi = pk_f16((float)(int)(int8_t)((v >> 16) & 0xffu), (float)(int)(int8_t)(v >> 24));
}

// Q8_0: block (k0 / 32 + h) of the row; the tiled layout keeps its 32 quant
// bytes as two aligned 16-byte pieces, the GGUF one as 2-aligned blocks of 34
template <bool TILED>
struct WQ80 {
    static constexpr bool kKQuant = false;
    uint32_t q[8];
    uint32_t dh;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int h) {
        const uint8_t* rp = w + (size_t)row * rb;
        const int64_t c = (k0 >> 5) + h;
        if constexpr (TILED) {
            const Q80TileOffs o = q80_tile_offsets(c, (int64_t)(rb / 34));
            const uint4 lo = ld16(rp + o.lo), hi = ld16(rp + o.hi);
            q[0] = lo.x; q[1] = lo.y; q[2] = lo.z; q[3] = lo.w;
            q[4] = hi.x; q[5] = hi.y; q[6] = hi.z; q[7] = hi.w;
            dh = ld_u16(rp + o.d);
        } else {
            const uint8_t* blk = rp + (size_t)c * 34;
            dh = ld_u16(blk);
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = ld_u16(blk + 2 + 4 * i) | (ld_u16(blk + 4 + 4 * i) << 16);
        }
    }
    __device__ __forceinline__ void decode(int, int, int, uint32_t (&o)[16], float& d, float& mt) const {
#pragma unroll
        for (int i = 0; i < 8; ++i) sbytes_f16(q[i], o[2 * i], o[2 * i + 1]);
        d = half_bits_to_float(dh);
        mt = 0.f;
    }
};
template <> struct WFormat<WF_Q80> : WQ80<false> {};
template <> struct WFormat<WF_Q80T> : WQ80<true> {};

// Q5_0 (tensor.cpp:434-449): d, a 32-bit high-bit mask, 16 qs bytes; element
// i < 16 is the low nibble of qs[i] with bit i, element 16 + i the high
// nibble with bit 16 + i, value d (q - 16)
template <>
struct WFormat<WF_Q50> {
    static constexpr bool kKQuant = false;
    uint32_t dh, qh, qs[4];
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ w, size_t rb, int row, int k0, int h) {
        const uint8_t* blk = w + (size_t)row * rb + (size_t)((k0 >> 5) + h) * 22;
        dh = ld_u16(blk);
        qh = ld_u16(blk + 2) | (ld_u16(blk + 4) << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = ld_u16(blk + 6 + 4 * i) | (ld_u16(blk + 8 + 4 * i) << 16);
    }
    __device__ __forceinline__ void decode(int, int, int, uint32_t (&o)[16], float& d, float& mt) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[8];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int e = 4 * i + b;
                const uint32_t byte = (qs[i] >> (8 * b)) & 0xffu;
                v[b] = (float)((int)((byte & 15u) | (((qh >> e) & 1u) << 4)) - 16);
                v[4 + b] = (float)((int)((byte >> 4) | (((qh >> (e + 16)) & 1u) << 4)) - 16);
            }
            // elements 4i..4i+3 (low nibbles) and 16+4i.. (high nibbles)
            o[2 * i] = pk_f16(v[0], v[1]);
            o[2 * i + 1] = pk_f16(v[2], v[3]);
            o[8 + 2 * i] = pk_f16(v[4], v[5]);
            o[8 + 2 * i + 1] = pk_f16(v[6], v[7]);
        }
        d = half_bits_to_float(dh);
        mt = 0.f;
    }
};

// Split K: split z takes K steps [z * ksteps, (z + 1) * ksteps), a
// multiple of 4 (whole super-blocks), and with more than one split writes
// its scaled partial tile to part[z][m][n] for gemm_f16_reduce.
template <int F, int TN>
__global__ __launch_bounds__(2 * TN, TN == 128 ? 2 : 1) void gemm_q_f16_kernel(const uint16_t* __restrict__ a_hi,
                                                           const uint16_t* __restrict__ a_lo, int lda,
                                                           const uint16_t* __restrict__ s_hi,
                                                           const uint16_t* __restrict__ s_lo, int lds,
                                                           const float* __restrict__ rscale,
                                                           const uint8_t* __restrict__ w, float* out, int ldo,
                                                           const float* res, int m, int n, int k, int form, int ksteps,
                                                           float* __restrict__ part) {
    extern __shared__ __align__(16) uint16_t smem[];
    // waves: 2 (activation row halves) x TN / 64 (weight row quarters of 64)
    constexpr int WC = TN / 64;
    // activation staging: APT threads per activation row, EPT elements each
    constexpr int APT = 2 * TN / kQM, EPT = kQK / APT;
    uint16_t* Ah = smem;              // [128][kQLd] activations, hi
    uint16_t* Al = Ah + kQM * kQLd;   // lo
    uint16_t* Ws = Al + kQM * kQLd;   // [TN][kQLd] weights sc q
    uint16_t* Sh = Ws + TN * kQLd;    // [128][kRLd] sub-block sums, hi (ring of 16 sub-blocks)
    uint16_t* Sl = Sh + kQM * kRLd;
    uint16_t* Bh = Sl + kQM * kRLd;   // [TN][kRLd] -dmin m_j per weight row, hi
    uint16_t* Bl = Bh + TN * kRLd;
    // [TN] d of the current super-block (K-quants), [2][TN] d of the step's
    // two blocks (32-element blocks)
    float* dcol = reinterpret_cast<float*>(Bl + TN * kRLd);
    using WF = WFormat<F>;
    constexpr bool KQ = WF::kKQuant;

    // Work item w = (split z, row tile y, column tile x), x fastest, and
    // workgroup ids dealt so that XCD q (ids q, q + 8, ...) takes the
    // contiguous range [q * per, (q + 1) * per) of items: the workgroups of
    // one XCD share their activation rows (and K range) in its L2.
    const int tn = (n + TN - 1) / TN, tm = (m + kQM - 1) / kQM, splits = (k / kQK + ksteps - 1) / ksteps;
    const int total = tn * tm * splits, per = (int)gridDim.x / 8;
    const int wi = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (wi >= total) return;
    const int tx = wi % tn, ty = (wi / tn) % tm, tz = wi / (tn * tm);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave / WC, wc = wave % WC;
    const int m0 = ty * kQM, n0 = tx * TN;
    const int kb = tz * ksteps * kQK, ke = min(k, kb + ksteps * kQK);
    const size_t rb = row_bytes(F == WF_Q4K || F == WF_Q4KT   ? MXH_Q4_K
                                : F == WF_Q5K || F == WF_Q5KT ? MXH_Q5_K
                                : F == WF_Q50                 ? MXH_Q5_0
                                                              : MXH_Q8_0,
                                k);
    // staging roles: thread t owns weight row t / 2 of the tile and sub-block
    // half t % 2 of the step, and activation row ra = t / APT, elements
    // EPT aq .. of the step (aq = t % APT), with the sum of sub-block sa
    const int t = threadIdx.x, r = t >> 1, h = t & 1;
    const int ra = t / APT, aq = t % APT, sa = aq * EPT / 32;
    const bool s_owner = (aq * EPT) % 32 == 0;
    const int wrow = min(n0 + r, n - 1);
    const bool arow = m0 + ra < m;
    const int lr = lane & 31, lk = 8 * (lane >> 5);

    f32x16 acc[2][2], P[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = P[i][j][e] = 0.f;

    // rows past m read row m - 1 and are zeroed when staged
    const int arow_c = min(m0 + ra, m - 1);
    const uint16_t* pa_h = a_hi + (size_t)arow_c * lda + EPT * aq;
    const uint16_t* pa_l = a_lo + (size_t)arow_c * lda + EPT * aq;
    const uint16_t* ps_h = s_hi + (size_t)arow_c * lds + sa;
    const uint16_t* ps_l = s_lo + (size_t)arow_c * lds + sa;
    constexpr int AV = EPT / 8;  // 16-byte pieces per thread and limb
    uint4 ahv[AV], alv[AV];
    uint32_t sh_g = 0, sl_g = 0;
    WF wq;
#define MXH_Q4F16_FETCH(K0)                                                   \
    do {                                                                     \
        const uint4* qh_ = reinterpret_cast<const uint4*>(pa_h + (K0));      \
        const uint4* ql_ = reinterpret_cast<const uint4*>(pa_l + (K0));      \
        _Pragma("unroll") for (int v_ = 0; v_ < AV; ++v_) {                  \
            ahv[v_] = qh_[v_];                                               \
            alv[v_] = ql_[v_];                                               \
        }                                                                    \
        if constexpr (KQ) {                                                  \
            sh_g = ps_h[(K0) >> 5];                                          \
            sl_g = ps_l[(K0) >> 5];                                          \
        }                                                                    \
        wq.fetch(w, rb, wrow, (K0), h);                                      \
    } while (0)
    MXH_Q4F16_FETCH(kb);

    int step = 0;
    for (int k0 = kb; k0 < ke; k0 += kQK, ++step) {
        const int slot = 2 * (step & 7) + h;  // ring slot of this thread's weight sub-block
        {
            uint4* dh = reinterpret_cast<uint4*>(Ah + ra * kQLd + EPT * aq);
            uint4* dl = reinterpret_cast<uint4*>(Al + ra * kQLd + EPT * aq);
            const uint32_t am = arow ? 0xffffffffu : 0u;
            auto msk = [am](uint4 v) { return make_uint4(v.x & am, v.y & am, v.z & am, v.w & am); };
#pragma unroll
            for (int v = 0; v < AV; ++v) {
                dh[v] = msk(ahv[v]);
                dl[v] = msk(alv[v]);
            }
            if (KQ && s_owner) {
                Sh[ra * kRLd + 2 * (step & 7) + sa] = (uint16_t)(sh_g & am);
                Sl[ra * kRLd + 2 * (step & 7) + sa] = (uint16_t)(sl_g & am);
            }
            // this thread's 32 weights as fp16 integers, and their scales
            uint32_t o[16];
            float dq, mt;
            wq.decode(k0, h, form, o, dq, mt);
            uint4* dw = reinterpret_cast<uint4*>(Ws + r * kQLd + 32 * h);
#pragma unroll
            for (int q = 0; q < 4; ++q) dw[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
            if constexpr (KQ) {
                const uint32_t bsplit = split_f16(mt);
                Bh[r * kRLd + slot] = (uint16_t)bsplit;
                Bl[r * kRLd + slot] = (uint16_t)(bsplit >> 16);
                if (h == 0) dcol[r] = dq;
            } else {
                dcol[h * TN + r] = dq;
            }
        }
        __syncthreads();
        if (k0 + kQK < ke) MXH_Q4F16_FETCH(k0 + kQK);

#pragma unroll
        for (int ks = 0; ks < kQK; ks += 16) {
            f16x8 ah[2], al[2], bw[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ao = (wr * 64 + i * 32 + lr) * kQLd + ks + lk;
                const int bo = (wc * 64 + i * 32 + lr) * kQLd + ks + lk;
                ah[i] = *reinterpret_cast<const f16x8*>(Ah + ao);
                al[i] = *reinterpret_cast<const f16x8*>(Al + ao);
                bw[i] = *reinterpret_cast<const f16x8*>(Ws + bo);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j], P[i][j], 0, 0, 0);
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j], P[i][j], 0, 0, 0);
                }
            if (!KQ && (ks & 31) == 16) {
                // end of a 32-element block: acc += d[n] . P
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float dc = dcol[(ks >> 5) * TN + wc * 64 + j * 32 + lr];
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            acc[i][j][e] = fmaf(dc, P[i][j][e], acc[i][j][e]);
                            P[i][j][e] = 0.f;
                        }
                }
            }
        }
        const bool last = k0 + kQK >= ke;
        if (KQ && (((k0 + kQK) & 255) == 0 || last)) {
            // end of a super-block: acc += d[n] . P (each lane's accumulators share one column)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float dc = dcol[wc * 64 + j * 32 + lr];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        acc[i][j][e] = fmaf(dc, P[i][j][e], acc[i][j][e]);
                        P[i][j][e] = 0.f;
                    }
            }
        }
        if (KQ && ((step & 7) == 7 || last)) {
            // correction round over the sub-blocks staged since the last one;
            // ring slots past `used` hold older values and are zeroed here
            const int used = 2 * ((step & 7) + 1);
            f16x8 sh[2], sl[2], bh[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                sh[i] = *reinterpret_cast<const f16x8*>(Sh + (wr * 64 + i * 32 + lr) * kRLd + lk);
                sl[i] = *reinterpret_cast<const f16x8*>(Sl + (wr * 64 + i * 32 + lr) * kRLd + lk);
                bh[i] = *reinterpret_cast<const f16x8*>(Bh + (wc * 64 + i * 32 + lr) * kRLd + lk);
                bl[i] = *reinterpret_cast<const f16x8*>(Bl + (wc * 64 + i * 32 + lr) * kRLd + lk);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (lk + e >= used) sh[i][e] = sl[i][e] = bh[i][e] = bl[i][e] = (_Float16)0.f;
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh[i], bl[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh[i], bh[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
    }

    const bool partial = splits > 1;
    float* dst = partial ? part + (size_t)tz * m * n : out;
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
                    const float v = acc[i][j][e] * rscale[row];
                    if (partial) dst[o] = v;
                    else dst[o] = res ? v + res[o] : v;
                }
            }
        }
}

#undef MXH_Q4F16_FETCH

// ---- Q4_K on a direct-to-LDS pipeline ------------------------------------
//
// The same product as gemm_q_f16_kernel for Q4_K rows (GGUF or tiled order),
// organised around the matrix cores: global memory goes straight into LDS
// (global_load_lds_dwordx4, no registers, no conversion), three K steps in
// flight, one barrier per step, and each wave decodes the weight rows it
// multiplies from their raw bytes in LDS into MFMA operands itself.
//
// Tile 128 activation rows x 128 weight rows per workgroup of 8 waves (2 x 4,
// 64 x 32 each, two per SIMD), one workgroup per CU.  Per stage (one 64-element K step):
//   activations hi and lo, [row][8 x 16 bytes], 16-byte chunk c of row r at
//   c ^ swz(r) (conflict-free MFMA operand reads),
//   raw weight bytes, [row][header, first 16 qs bytes, last 16 qs bytes].
// K order inside a step: the MFMA's 16-element slices are taken so that the
// lane holding weight row n, half h, reads one 16-byte qs piece: slice jj of
// half h covers elements 8 ((jj & 1) + 2 h + 4 (jj >> 1)) .. + 7 of the step
// (low nibbles of bytes 8 (jj & 1) .. of piece h for jj < 2, high nibbles for
// jj >= 2), and the activation operand reads the same elements.
// Sub-block sums S (for the min terms) come in a ring of 16 sub-blocks per
// round of 8 steps, double-buffered; the -dmin m_j values of a round are
// written to a second ring by the decoding waves; the correction MFMAs of a
// round run at the top of the step after it.
// Geometry for WJ blocks of 32 weight rows per wave: the 4 waves along the
// weight rows cover BN = 128 WJ of them.  WJ = 2 stages each activation tile
// once for 256 weight rows, half the activation bytes per MFMA of WJ = 1, in
// two stages instead of three (the LDS holds no more).
template <int WJ>
struct Q4P {
    static constexpr int BM = 128, BN = 128 * WJ, BK = 64, NST = WJ == 1 ? 3 : 2;
    static constexpr int kStageA = 2 * BM * 128;              // hi + lo
    static constexpr int kWChunks = 3 * BN;                   // 16-byte (header, qs, qs) chunks
    static constexpr int kWLoads = (kWChunks + 511) / 512;    // direct loads per wave and stage
    static constexpr int kStageW = kWLoads * 512 * 16;        // (padding lanes repeat a real chunk)
    static constexpr int kStage = kStageA + kStageW;
    static constexpr int kRingS = 2 * BM * 16 * 2;            // activation sums [limb][row][16 slots] fp16
    static constexpr int kRingB = 2 * BN * 16 * 2;            // -dmin m [limb][weight row][16 slots] fp16
    static constexpr size_t kLds = (size_t)NST * kStage + 2 * (size_t)kRingS + 2 * (size_t)kRingB;
    static constexpr int kLoadsStep = 4 + kWLoads;            // per wave: activation + weight chunks
};

__device__ __forceinline__ int q4p_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// 16 bytes per lane from global memory straight into LDS: lane i writes
// lds_wave_base + 16 i.  Issued as inline assembly so that the compiler does
// not wait for every such load before the next LDS read (it cannot tell the
// stages apart); the pipeline waits for them itself (wait_vm).
__device__ __forceinline__ void g2l16(const void* g, uint8_t* lds_wave_base) {
    const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds_wave_base;
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(l) : "memory");
}

// timeline hook for out-of-tree probes (empty in the library)
#ifndef MXH_Q4P_STAMP
#define MXH_Q4P_STAMP(t, i)
#endif

// Workgroup barrier for the pipeline: LDS writes of this wave complete, then
// s_barrier, with no wait for outstanding global loads (__syncthreads' fence
// would drain the loads of the steps in flight).  The direct-to-LDS loads of
// a stage are waited for with wait_vm before it.
__device__ __forceinline__ void q4p_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
    // vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// fp16 pairs of (4 nibble bytes in n, selected by the perm) x sc, exact:
// bytes q0, q1 become fp16 1024 + q (high byte 0x64), then
// (1024 + q) sc - 1024 sc in one fused fp16 operation
__device__ __forceinline__ uint32_t q4p_pair(uint32_t n, uint32_t sel, h2v scv, h2v offv) {
    const uint32_t b = __builtin_amdgcn_perm(0x64u, n, sel);
    const h2v r = __builtin_elementwise_fma(__builtin_bit_cast(h2v, b), scv, offv);
    return __builtin_bit_cast(uint32_t, r);
}

// eight weights (bytes 0-3 and 4-7 of (lo, hi), nibble at `shift`) as fp16
// integers times sc
__device__ __forceinline__ f16x8 q4p_slice(uint32_t w0, uint32_t w1, int shift, h2v scv, h2v offv) {
    const uint32_t n0 = (w0 >> shift) & 0x0f0f0f0fu, n1 = (w1 >> shift) & 0x0f0f0f0fu;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const u4v r = {q4p_pair(n0, 0x04010400u, scv, offv), q4p_pair(n0, 0x04030402u, scv, offv),
                   q4p_pair(n1, 0x04010400u, scv, offv), q4p_pair(n1, 0x04030402u, scv, offv)};
    return __builtin_bit_cast(f16x8, r);
}

template <bool TILED, int WJ>
__global__ __launch_bounds__(512, 1) void gemm_q4k_pipe_kernel(const uint16_t* __restrict__ a_hi,
                                                               const uint16_t* __restrict__ a_lo, int lda,
                                                               const uint16_t* __restrict__ s_hi,
                                                               const uint16_t* __restrict__ s_lo, int lds,
                                                               const float* __restrict__ rscale,
                                                               const uint8_t* __restrict__ w, float* out, int ldo,
                                                               const float* res, int m, int n, int k, int form,
                                                               int ksteps, float* __restrict__ part) {
    using G = Q4P<WJ>;
    constexpr int BM = G::BM, BN = G::BN, BK = G::BK, NST = G::NST, kStageA = G::kStageA, kStage = G::kStage;
    constexpr int kRingS = G::kRingS, kRingB = G::kRingB, kLoadsStep = G::kLoadsStep;
    extern __shared__ __align__(16) uint8_t smem8[];
    uint8_t* ringS = smem8 + (size_t)NST * kStage;  // [2][kRingS]
    uint8_t* ringB = ringS + 2 * kRingS;             // [2][kRingB]

    // work item as in gemm_q_f16_kernel (XCD-contiguous ranges)
    const int tn = (n + BN - 1) / BN, tm = (m + BM - 1) / BM, splits = (k / BK + ksteps - 1) / ksteps;
    const int total = tn * tm * splits, per = (int)gridDim.x / 8;
    const int wi = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (wi >= total) return;
    const int tx = wi % tn, ty = (wi / tn) % tm, tz = wi / (tn * tm);
    // 8 waves: 2 along the activation rows (64 each) x 4 along the weight rows (32 WJ each)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave >> 2, wc = wave & 3;
    const int m0 = ty * BM, n0 = tx * BN;
    const int kb = tz * ksteps * BK, ke = min(k, kb + ksteps * BK);
    const int nsteps = (ke - kb) / BK;
    const size_t rb = (size_t)(k / 256) * 144;
    const int64_t nblk = k / 256;
    const int lr = lane & 31, hh = lane >> 5;

    // ---- global -> LDS load roles (fixed per lane; the step adds k0) ----
    // activations: load u of this wave fills LDS chunks (4 wave + u) * 64 + lane
    const uint16_t* aptr[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int slot = (wave * 4 + u) * 64 + lane, limb = slot >> 10, P = slot & 1023;
        const int row = P >> 3, c = (P & 7) ^ q4p_swz(row);
        const int grow = min(m0 + row, m - 1);
        aptr[u] = (limb ? a_lo : a_hi) + (size_t)grow * lda + 8 * c;
    }
    // weights: load u of this wave fills raw chunk Q = 512 u + wave * 64 + lane
    // (row Q / 3, part Q % 3)
    int wpart[G::kWLoads];
    const uint8_t* wrow[G::kWLoads];
#pragma unroll
    for (int u = 0; u < G::kWLoads; ++u) {
        int Qw = 512 * u + wave * 64 + lane;
        if (Qw >= G::kWChunks) Qw -= G::kWChunks;  // padding lanes repeat a real chunk
        wpart[u] = Qw % 3;
        wrow[u] = w + (size_t)min(n0 + Qw / 3, n - 1) * rb;
    }
    auto w_addr = [&](int u, int step) -> const uint8_t* {
        const int64_t c = (int64_t)(kb / BK + step);  // 64-element chunk of the row
        if constexpr (TILED) {
            const Q4KTileOffs o = q4k_tile_offsets(c, nblk);
            return wrow[u] + (wpart[u] == 0 ? o.hd : wpart[u] == 1 ? o.qa : o.qb);
        } else {
            const size_t blk = (size_t)(c >> 2) * 144;
            return wrow[u] + blk + (wpart[u] == 0 ? 0 : 16 + 32 * (int)(c & 3) + 16 * (wpart[u] - 1));
        }
    };
    // sub-block sums: this wave's load fills ring chunk wave * 64 + lane
    const int s_slot = wave * 64 + lane, s_half = s_slot & 1;
    const uint16_t* sptr = ((s_slot >> 8) ? s_lo : s_hi) + (size_t)min(m0 + ((s_slot >> 1) & 127), m - 1) * lds +
                           8 * s_half;
    const int nsb = k / 32;
    // load q (0 .. kLoadsStep - 1) of a stage: the activation chunks, then the
    // weight chunks
    auto issue_load = [&](int step, int q) {
        const int st = min(step, nsteps - 1);  // past the end: the last step again (never read)
        uint8_t* base = smem8 + (size_t)(step % NST) * kStage;
        if (q < 4) g2l16(aptr[q] + kb + st * BK, base + (wave * 4 + q) * 1024);
        else g2l16(w_addr(q - 4, st), base + kStageA + (512 * (q - 4) + wave * 64) * 16);
    };
    auto issue_stage = [&](int step) {
#pragma unroll
        for (int q = 0; q < kLoadsStep; ++q) issue_load(step, q);
    };
    auto issue_sums = [&](int round) {
        int j0 = kb / 32 + 16 * round;
        // chunks past the row (rounds beyond this work item) read sub-block 0
        if (j0 + 8 * s_half >= nsb) j0 = -8 * s_half;
        g2l16(sptr + j0, ringS + (size_t)(round & 1) * kRingS + wave * 1024);
    };

    f32x16 acc[2][WJ], P[2][WJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = P[i][j][e] = 0.f;

    // this lane's weight rows in the tile: block j of the wave
    int col[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) col[j] = wc * 32 * WJ + 32 * j + lr;
    // correction of round r over its first `used` sub-block slots:
    // acc += S . (-dmin m) with S and -dmin m split hi / lo
    auto correction = [&](int r, int used) {
        const uint8_t* sb = ringS + (size_t)(r & 1) * kRingS;
        const uint8_t* bb = ringB + (size_t)(r & 1) * kRingB;
        f16x8 sh[2], sl[2], bh[WJ], bl[WJ];
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            bh[j] = *reinterpret_cast<const f16x8*>(bb + col[j] * 32 + hh * 16);
            bl[j] = *reinterpret_cast<const f16x8*>(bb + BN * 32 + col[j] * 32 + hh * 16);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = wr * 64 + i * 32 + lr;
            sh[i] = *reinterpret_cast<const f16x8*>(sb + row * 32 + hh * 16);
            sl[i] = *reinterpret_cast<const f16x8*>(sb + BM * 32 + row * 32 + hh * 16);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (8 * hh + e >= used) {
#pragma unroll
                for (int j = 0; j < WJ; ++j) bh[j][e] = bl[j][e] = (_Float16)0.f;
                sh[0][e] = sl[0][e] = sh[1][e] = sl[1][e] = (_Float16)0.f;
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < WJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh[i], bl[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh[i], bh[j], acc[i][j], 0, 0, 0);
            }
    };

    // prologue: round 0's sums, the first NST - 1 steps
    issue_sums(0);
#pragma unroll
    for (int q = 0; q < NST - 1; ++q) issue_stage(q);

    for (int t = 0; t < nsteps; ++t) {
        // stage t complete: only the loads issued after it may be outstanding
        // (the later stages in flight, and round sums issued after them)
        MXH_Q4P_STAMP(t, 0);
        if (t == 0 || ((t - 1) & 7) != 1) wait_vm<(NST - 2) * kLoadsStep>();
        else wait_vm<(NST - 2) * kLoadsStep + 1>();
        MXH_Q4P_STAMP(t, 1);
        q4p_barrier();
        MXH_Q4P_STAMP(t, 2);
        if (t > 0 && (t & 7) == 0) correction((t >> 3) - 1, 16);
        issue_stage(t + NST - 1);
        MXH_Q4P_STAMP(t, 5);

        const uint8_t* stg = smem8 + (size_t)(t % NST) * kStage;
        const int k0 = kb + t * BK, g = (k0 >> 6) & 3;
        // this lane's weight rows: header and its 16-byte qs piece
        f16x8 bw[WJ][4];
        float dcol[WJ];
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const uint4 hd = *reinterpret_cast<const uint4*>(stg + kStageA + col[j] * 48);
            const uint4 q = *reinterpret_cast<const uint4*>(stg + kStageA + col[j] * 48 + 16 + 16 * hh);
            uint32_t scp, mnp;
            k4_pair(hd.y, hd.z, hd.w, g, form, scp, mnp);
            // hardware conversion: d and dmin only scale sums (a NaN payload need not survive)
            dcol[j] = __half2float(__ushort_as_half((uint16_t)(hd.x & 0xffffu)));
            const float dmin = __half2float(__ushort_as_half((uint16_t)(hd.x >> 16)));
            const _Float16 sc0 = (_Float16)(float)(scp & 0xffu), sc1 = (_Float16)(float)(scp >> 8);
            const h2v sv0 = {sc0, sc0}, sv1 = {sc1, sc1};
            const h2v ov0 = {(_Float16)(-1024.f) * sc0, (_Float16)(-1024.f) * sc0};
            const h2v ov1 = {(_Float16)(-1024.f) * sc1, (_Float16)(-1024.f) * sc1};
            bw[j][0] = q4p_slice(q.x, q.y, 0, sv0, ov0);
            bw[j][1] = q4p_slice(q.z, q.w, 0, sv0, ov0);
            bw[j][2] = q4p_slice(q.x, q.y, 4, sv1, ov1);
            bw[j][3] = q4p_slice(q.z, q.w, 4, sv1, ov1);
            if (wr == 0) {
                // -dmin m of sub-block 2g (lanes of half 0) or 2g + 1 (half 1)
                const float mt = -(dmin * (float)(hh ? (mnp >> 8) : (mnp & 0xffu)));
                const uint32_t sp = split_f16(mt);
                uint16_t* bb = reinterpret_cast<uint16_t*>(ringB + (size_t)((t >> 3) & 1) * kRingB);
                const int slot = 2 * (t & 7) + hh;
                bb[col[j] * 16 + slot] = (uint16_t)sp;
                bb[BN * 16 + col[j] * 16 + slot] = (uint16_t)(sp >> 16);
            }
        }
        MXH_Q4P_STAMP(t, 3);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int c = (jj & 1) + 2 * hh + 4 * (jj >> 1);
            f16x8 ah[2], al[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wr * 64 + i * 32 + lr;
                const int off = row * 128 + 16 * (c ^ q4p_swz(row));
                ah[i] = *reinterpret_cast<const f16x8*>(stg + off);
                al[i] = *reinterpret_cast<const f16x8*>(stg + BM * 128 + off);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j) {
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j][jj], P[i][j], 0, 0, 0);
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j][jj], P[i][j], 0, 0, 0);
                }
        }
        if ((t & 7) == 1) issue_sums((t >> 3) + 1);
        MXH_Q4P_STAMP(t, 4);
        if (((k0 + BK) & 255) == 0 || t == nsteps - 1) {
            // end of a super-block: acc += d[n] . P
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        acc[i][j][e] = fmaf(dcol[j], P[i][j][e], acc[i][j][e]);
                        P[i][j][e] = 0.f;
                    }
        }
    }
    wait_vm<0>();
    q4p_barrier();
    {
        const int r = (nsteps - 1) >> 3;
        correction(r, 2 * (nsteps - 8 * r));
    }

    const bool partial = splits > 1;
    float* dst = partial ? part + (size_t)tz * m * n : out;
    const int ld = partial ? n : ldo;
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
        const int ocol = n0 + col[j];
        if (ocol < n) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wr * 64 + i * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
                    if (row < m) {
                        const size_t o = (size_t)row * ld + ocol;
                        const float v = acc[i][j][e] * rscale[row];
                        if (partial) dst[o] = v;
                        else dst[o] = res ? v + res[o] : v;
                    }
                }
        }
    }
}

__global__ void gemm_f16_reduce_kernel(const float* __restrict__ part, int splits, float* out, int ldo,
                                       const float* res, int m, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * n) return;
    const int r = i / n, c = i % n;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += part[(size_t)s * m * n + i];
    const size_t o = (size_t)r * ldo + c;
    out[o] = res ? v + res[o] : v;
}

// the same sums, four adjacent outputs per thread (n, ldo multiples of 4 and
// 16-byte aligned rows)
__global__ void gemm_f16_reduce4_kernel(const float4* __restrict__ part, int splits, float* out, int ldo,
                                        const float* res, int m, int n4) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * n4) return;
    const int r = i / n4, c = i - r * n4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < splits; ++s) {
        const float4 p = part[(size_t)s * m * n4 + i];
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    const size_t o = (size_t)r * ldo + 4 * (size_t)c;
    if (res) {
        const float4 q = *reinterpret_cast<const float4*>(res + o);
        v.x += q.x;
        v.y += q.y;
        v.z += q.z;
        v.w += q.w;
    }
    *reinterpret_cast<float4*>(out + o) = v;
}

void reduce_launch(const float* part, int splits, float* out, int ldo, const float* res, int m, int n,
                   hipStream_t st) {
    const bool vec = n % 4 == 0 && ldo % 4 == 0 && (uintptr_t)part % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                     (uintptr_t)res % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(gemm_f16_reduce4_kernel, dim3((m * (n / 4) + 255) / 256), dim3(256), 0, st,
                           reinterpret_cast<const float4*>(part), splits, out, ldo, res, m, n / 4);
    else
        hipLaunchKernelGGL(gemm_f16_reduce_kernel, dim3((m * n + 255) / 256), dim3(256), 0, st, part, splits, out,
                           ldo, res, m, n);
}

// power-of-two scale 2^e that brings the row maximum into [128, 256)
__device__ __forceinline__ int row_exponent(float maxv) {
    if (!(maxv > 0.f) || maxv > 3.0e38f) return 0;
    int ex;
    (void)frexpf(maxv, &ex);  // maxv in [2^(ex-1), 2^ex)
    const int e = 8 - ex;
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

// block-wide max of non-negative floats (256 threads)
__device__ __forceinline__ float block_max_256(float v, float* red) {
    v = wave_max_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

// Writes row values v (sub-block sb of 32, thread-owned) as a' = v 2^e split
// into fp16 hi / lo, and the split sum of each sub-block's hi + lo.
__device__ __forceinline__ void emit_subblock(const float* v, float scale, uint16_t* ah, uint16_t* al, uint16_t* sh,
                                              uint16_t* sl) {
    float s = 0.f;
    uint32_t ph[16], pl[16];
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        const uint32_t p0 = split_f16(v[i] * scale), p1 = split_f16(v[i + 1] * scale);
        s += (__half2float(__ushort_as_half((uint16_t)p0)) + __half2float(__ushort_as_half((uint16_t)(p0 >> 16)))) +
             (__half2float(__ushort_as_half((uint16_t)p1)) + __half2float(__ushort_as_half((uint16_t)(p1 >> 16))));
        ph[i / 2] = (p0 & 0xffffu) | (p1 << 16);
        pl[i / 2] = (p0 >> 16) | (p1 & 0xffff0000u);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        reinterpret_cast<uint4*>(ah)[q] = make_uint4(ph[4 * q], ph[4 * q + 1], ph[4 * q + 2], ph[4 * q + 3]);
        reinterpret_cast<uint4*>(al)[q] = make_uint4(pl[4 * q], pl[4 * q + 1], pl[4 * q + 2], pl[4 * q + 3]);
    }
    const uint32_t ps = split_f16(s);
    *sh = (uint16_t)ps;
    *sl = (uint16_t)(ps >> 16);
}

// Rows of x (optionally the reference rmsnorm x / sqrt(mean(x^2) + eps) * w,
// rmsnorm.cpp:5-26, sum of squares in double, the same float products as
// rows_to_bf16) as GEMM input of gemm_q_f16.  One workgroup per row; k a
// multiple of 32 and at most 2 * 256 * 32.
constexpr int kRowSub = 2;  // sub-blocks per thread
__global__ __launch_bounds__(256) void rows_to_f16_kernel(const float* __restrict__ x, int ldx,
                                                          const float* __restrict__ nw, float eps, int k,
                                                          uint16_t* __restrict__ a_hi, uint16_t* __restrict__ a_lo,
                                                          int lda, uint16_t* __restrict__ s_hi,
                                                          uint16_t* __restrict__ s_lo, int lds,
                                                          float* __restrict__ rscale) {
    __shared__ double red[4];
    __shared__ float redf[4];
    const int row = blockIdx.x, nsb = k / 32;
    const float* xr = x + (size_t)row * ldx;
    float v[kRowSub][32];
    double ss = 0.0;
    float mx = 0.f;
#pragma unroll
    for (int u = 0; u < kRowSub; ++u) {
        const int sb = threadIdx.x + 256 * u;
#pragma unroll
        for (int i = 0; i < 32; ++i) v[u][i] = 0.f;
        if (sb < nsb) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = reinterpret_cast<const float4*>(xr + 32 * sb)[q];
                v[u][4 * q] = f.x;
                v[u][4 * q + 1] = f.y;
                v[u][4 * q + 2] = f.z;
                v[u][4 * q + 3] = f.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) ss += (double)v[u][i] * v[u][i];
    }
    float inv = 1.f;
    if (nw) {
        ss = wave_sum_d_lane63(ss);
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        inv = (float)(1.0 / sqrt(((red[0] + red[1]) + (red[2] + red[3])) / (double)k + (double)eps));
    }
#pragma unroll
    for (int u = 0; u < kRowSub; ++u) {
        const int sb = threadIdx.x + 256 * u;
        if (nw && sb < nsb) {
#pragma unroll
            for (int i = 0; i < 32; ++i) v[u][i] = v[u][i] * inv * nw[32 * sb + i];
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[u][i]));
    }
    const int e = row_exponent(block_max_256(mx, redf));
    const float scale = ldexpf(1.f, e);
    if (threadIdx.x == 0) rscale[row] = ldexpf(1.f, -e);
#pragma unroll
    for (int u = 0; u < kRowSub; ++u) {
        const int sb = threadIdx.x + 256 * u;
        if (sb < nsb)
            emit_subblock(v[u], scale, a_hi + (size_t)row * lda + 32 * sb, a_lo + (size_t)row * lda + 32 * sb,
                          s_hi + (size_t)row * lds + sb, s_lo + (size_t)row * lds + sb);
    }
}

// h = silu(gate) * up (transformer.cpp:183-185) as gemm_q_f16 input; gu
// rows are [gate | up], f a multiple of 32 and at most 2 * 256 * 32.
__global__ __launch_bounds__(256) void silu_mul_f16_kernel(const float* __restrict__ gu, int f,
                                                           uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo,
                                                           uint16_t* __restrict__ s_hi, uint16_t* __restrict__ s_lo,
                                                           float* __restrict__ rscale) {
    __shared__ float redf[4];
    const int row = blockIdx.x, nsb = f / 32, lds = nsb;
    const float* g = gu + (size_t)row * 2 * f;
    float v[kRowSub][32];
    float mx = 0.f;
#pragma unroll
    for (int u = 0; u < kRowSub; ++u) {
        const int sb = threadIdx.x + 256 * u;
#pragma unroll
        for (int i = 0; i < 32; ++i) v[u][i] = 0.f;
        if (sb < nsb) {
            // the sub-block's 32 gate and 32 up values as 16-byte loads
            const float4* gp = reinterpret_cast<const float4*>(g + 32 * sb);
            const float4* up = reinterpret_cast<const float4*>(g + f + 32 * sb);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 a = gp[q], b = up[q];
                const float ga[4] = {a.x, a.y, a.z, a.w}, ub[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) v[u][4 * q + j] = ga[j] / (1.0f + expf(-ga[j])) * ub[j];
            }
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[u][i]));
    }
    const int e = row_exponent(block_max_256(mx, redf));
    const float scale = ldexpf(1.f, e);
    if (threadIdx.x == 0) rscale[row] = ldexpf(1.f, -e);
#pragma unroll
    for (int u = 0; u < kRowSub; ++u) {
        const int sb = threadIdx.x + 256 * u;
        if (sb < nsb)
            emit_subblock(v[u], scale, h_hi + (size_t)row * f + 32 * sb, h_lo + (size_t)row * f + 32 * sb,
                          s_hi + (size_t)row * lds + sb, s_lo + (size_t)row * lds + sb);
    }
}

// TN = 128: 4 waves, two workgroups per CU; TN = 256: 8 waves, one per CU,
// each activation tile staged once for twice the weight rows (half the
// activation traffic per MFMA)
template <int F, int TN>
int gemm_q_f16_launch(const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi,
                        const uint16_t* s_lo, int lds, const float* rscale, const uint8_t* w, float* out, int ldo,
                        const float* res, int m, int n, int k, int form, float* part, size_t part_floats,
                        hipStream_t st) {
    constexpr size_t lds_bytes = q4_lds_bytes<TN>();
    static bool attr_set = false;  // above 64 KiB of LDS needs the opt-in, once per kernel
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)gemm_q_f16_kernel<F, TN>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes) != hipSuccess)
            return MXH_ERR_HIP;
        attr_set = true;
    }
    const int tn = (n + TN - 1) / TN, tm = (m + kQM - 1) / kQM, steps = k / kQK;
    // split K (whole super-blocks, at most 4 ways) while the tile grid leaves CUs idle
    constexpr int target = TN == 128 ? 512 : 256;  // resident workgroups
    int splits = 1;
    while (splits < 4 && tn * tm * splits * 2 <= target && steps % (splits * 2 * 4) == 0 &&
           (size_t)(splits * 2) * m * n <= part_floats)
        splits *= 2;
    // one dimension of workgroup ids, a multiple of 8 (the kernel's XCD mapping)
    const int items = tn * tm * splits;
    const dim3 grid((unsigned)((items + 7) / 8 * 8));
    hipLaunchKernelGGL((gemm_q_f16_kernel<F, TN>), grid, dim3(2 * TN), lds_bytes, st, a_hi, a_lo, lda, s_hi,
                       s_lo, lds, rscale, w, out, ldo, res, m, n, k, form, steps / splits, part);
    if (splits > 1)
        reduce_launch(part, splits, out, ldo, res, m, n, st);
    return MXH_OK;
}

// Split K for the pipelined kernel (one workgroup per CU): the fewest splits
// (1, 2, 4 or 8, whole super-blocks, within the partial buffer) that minimise
// rounds x steps per work item.
int q4p_splits(int tiles, int steps, int n_cu, size_t mn, size_t part_floats) {
    int best = 1;
    long best_cost = -1;
    for (int s = 1; s <= 8; s *= 2) {
        if (steps % (4 * s)) break;
        if (s > 1 && (size_t)s * mn > part_floats) break;
        const long rounds = ((long)tiles * s + n_cu - 1) / n_cu;
        const long cost = rounds * (steps / s);
        if (best_cost < 0 || cost < best_cost) {
            best = s;
            best_cost = cost;
        }
    }
    return best;
}

template <bool TILED, int WJ>
int gemm_q4k_pipe_launch(const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi,
                         const uint16_t* s_lo, int lds, const float* rscale, const uint8_t* w, float* out, int ldo,
                         const float* res, int m, int n, int k, int form, float* part, size_t part_floats,
                         hipStream_t st) {
    using G = Q4P<WJ>;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)gemm_q4k_pipe_kernel<TILED, WJ>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)G::kLds) != hipSuccess)
            return MXH_ERR_HIP;
        attr_set = true;
    }
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n_cu = 256;
    }
    const int tn = (n + G::BN - 1) / G::BN, tm = (m + G::BM - 1) / G::BM, steps = k / G::BK;
    const int splits = q4p_splits(tn * tm, steps, n_cu, (size_t)m * n, part ? part_floats : 0);
    const int items = tn * tm * splits;
    const dim3 grid((unsigned)((items + 7) / 8 * 8));
    hipLaunchKernelGGL((gemm_q4k_pipe_kernel<TILED, WJ>), grid, dim3(512), G::kLds, st, a_hi, a_lo, lda, s_hi, s_lo,
                       lds, rscale, w, out, ldo, res, m, n, k, form, steps / splits, part);
    if (splits > 1)
        reduce_launch(part, splits, out, ldo, res, m, n, st);
    return MXH_OK;
}

// Weight-row blocks per wave of the pipelined Q4_K GEMM for a shape: the
// tiling with the lower estimate of rounds x (K steps per work item + 8, the
// pipeline's fill and epilogue), a 256-row step counted as 1.7 128-row ones
// (measured at M = 512: 256 rows faster for q|k|v 6144 x 4096 and down
// 4096 x 12288, slower for o 4096 x 4096 and gate|up 24576 x 4096, whose
// 384 wide tiles take two rounds on 256 CUs).
static int q4p_wj(int m, int n, int k, size_t part_floats) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n_cu = 256;
    }
    double best = 0.0;
    int wj = 1;
    for (int j = 1; j <= 2; ++j) {
        const int bn = 128 * j, tiles = ((n + bn - 1) / bn) * ((m + 127) / 128), steps = k / 64;
        const int s = q4p_splits(tiles, steps, n_cu, (size_t)m * n, part_floats);
        const long rounds = ((long)tiles * s + n_cu - 1) / n_cu;
        const double cost = (double)rounds * (steps / s + 8) * (j == 2 ? 1.7 : 1.0);
        if (j == 1 || cost < best) {
            best = cost;
            wj = j;
        }
    }
    return wj;
}

template <bool TILED>
int gemm_q4k_pipe_run(const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi, const uint16_t* s_lo,
                      int lds, const float* rscale, const uint8_t* w, float* out, int ldo, const float* res, int m,
                      int n, int k, int form, float* part, size_t part_floats, hipStream_t st) {
    if (q4p_wj(m, n, k, part ? part_floats : 0) == 1)
        return gemm_q4k_pipe_launch<TILED, 1>(a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, w, out, ldo, res, m, n, k,
                                              form, part, part_floats, st);
    return gemm_q4k_pipe_launch<TILED, 2>(a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, w, out, ldo, res, m, n, k, form,
                                          part, part_floats, st);
}

// the pipelined kernel's 16-byte direct loads need 16-byte aligned rows
bool q4p_aligned(const void* a_hi, const void* a_lo, int lda, const void* s_hi, const void* s_lo, int lds,
                 const void* w) {
    auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    return al(a_hi) && al(a_lo) && al(s_hi) && al(s_lo) && al(w) && lda % 8 == 0 && lds % 8 == 0;
}

}  // namespace

// Wide (256-row) weight tiles stage each activation tile once for twice the
// weight rows; with one 8-wave workgroup per CU they are worth it only when
// the whole tile grid fits in one round (measured at M = 512: o, down and
// q|k|v 3-5% faster, gate|up with 384 tiles 13% slower).
static bool q4_wide_tiles(int m, int n) {
    const int tiles = ((n + 255) / 256) * ((m + kQM - 1) / kQM);
    return m > kQM && n >= 2048 && tiles <= 256;
}

static int f16_format(int type) {
    switch (type) {
    case MXH_Q4_K: return WF_Q4K;
    case MXH_Q4_K_TILED: return WF_Q4KT;
    case MXH_Q5_K: return WF_Q5K;
    case MXH_Q5_K_TILED: return WF_Q5KT;
    case MXH_Q8_0: return WF_Q80;
    case MXH_Q8_0_TILED: return WF_Q80T;
    case MXH_Q5_0: return WF_Q50;
    }
    return -1;
}

bool gemm_q_f16_supported(int type, int k) {
    return f16_format(type) >= 0 && k % 256 == 0 && k <= kRowSub * 256 * 32;
}

template <int TN>
static int gemm_q_f16_dispatch(int type, const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi,
                               const uint16_t* s_lo, int lds, const float* rscale, const uint8_t* wb, float* out,
                               int ldo, const float* res, int m, int n, int k, int form, float* part,
                               size_t part_floats, hipStream_t st) {
#define MXH_QF16_CASE(F)                                                                                         \
    case F:                                                                                                      \
        return gemm_q_f16_launch<F, TN>(a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, wb, out, ldo, res, m, n, k, form, \
                                        part, part_floats, st);
    switch (f16_format(type)) {
        MXH_QF16_CASE(WF_Q4K)
        MXH_QF16_CASE(WF_Q4KT)
        MXH_QF16_CASE(WF_Q5K)
        MXH_QF16_CASE(WF_Q5KT)
        MXH_QF16_CASE(WF_Q80)
        MXH_QF16_CASE(WF_Q80T)
        MXH_QF16_CASE(WF_Q50)
    }
#undef MXH_QF16_CASE
    return MXH_ERR_UNSUPPORTED;
}

int gemm_q_f16_run(int type, const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi,
                     const uint16_t* s_lo, int lds, const float* rscale, const void* w, float* out, int ldo,
                     const float* res, int m, int n, int k, int form, float* part, size_t part_floats,
                     hipStream_t st) {
    if (m <= 0 || n <= 0 || !gemm_q_f16_supported(type, k) || lda < k || lds < k / 32 || ldo < n) return MXH_ERR_ARG;
    if (!part) part_floats = 0;
    const uint8_t* wb = (const uint8_t*)w;
    if ((type == MXH_Q4_K || type == MXH_Q4_K_TILED) && q4p_aligned(a_hi, a_lo, lda, s_hi, s_lo, lds, w)) {
        if (type == MXH_Q4_K_TILED)
            return gemm_q4k_pipe_run<true>(a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, wb, out, ldo, res, m, n, k,
                                              form, part, part_floats, st);
        return gemm_q4k_pipe_run<false>(a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, wb, out, ldo, res, m, n, k, form,
                                           part, part_floats, st);
    }
    if (q4_wide_tiles(m, n))
        return gemm_q_f16_dispatch<256>(type, a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, wb, out, ldo, res, m, n, k,
                                        form, part, part_floats, st);
    return gemm_q_f16_dispatch<128>(type, a_hi, a_lo, lda, s_hi, s_lo, lds, rscale, wb, out, ldo, res, m, n, k, form,
                                    part, part_floats, st);
}

int rows_to_f16_launch(const float* x, int ldx, const float* nw, float eps, int k, uint16_t* a_hi, uint16_t* a_lo,
                       int lda, uint16_t* s_hi, uint16_t* s_lo, int lds, float* rscale, int m, hipStream_t st) {
    if (m <= 0 || k % 32 || k > kRowSub * 256 * 32 || lda < k || lds < k / 32) return MXH_ERR_ARG;
    hipLaunchKernelGGL(rows_to_f16_kernel, dim3(m), dim3(256), 0, st, x, ldx, nw, eps, k, a_hi, a_lo, lda, s_hi, s_lo,
                       lds, rscale);
    return MXH_OK;
}

int silu_mul_f16_launch(const float* gu, int f, uint16_t* h_hi, uint16_t* h_lo, uint16_t* s_hi, uint16_t* s_lo,
                        float* rscale, int m, hipStream_t st) {
    if (m <= 0 || f % 32 || f > kRowSub * 256 * 32) return MXH_ERR_ARG;
    hipLaunchKernelGGL(silu_mul_f16_kernel, dim3(m), dim3(256), 0, st, gu, f, h_hi, h_lo, s_hi, s_lo, rscale);
    return MXH_OK;
}

}  // namespace mxh
