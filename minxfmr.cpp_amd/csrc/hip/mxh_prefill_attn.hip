// mxh_prefill_attn.hip — causal attention of a chunk of prompt tokens on the
// fp16 matrix cores, in flash form (running max and sum per query, no score
// matrix in memory).
//
// Reference op: the attention of transformer.cpp:529-629 for each prompt
// token (scores q.k / sqrt(hd) over cache positions 0 .. pos, softmax
// softmax.cpp:4-18, weighted sum of V rows), with the chunk's own K/V rows
// already appended to the fp16 cache by qkv_prep_rows_kernel.
//
// Workgroup (g, y) serves kv head g and 64 query rows: the `group` q heads
// of g for T = 64 / group consecutive tokens (row r = token r / group, head
// r % group).  Keys stream through LDS in stages of 64, double-buffered.
// Wave w of four takes query rows 32 (w & 1) .. +32 and key half w >> 1 of
// every stage; the two waves of a query set see disjoint keys and merge
// their (max, sum, V sum) at the end.  Per 32-key block a wave computes
//
//   S^T = K Q^T      v_mfma_f32_32x32x16_f16; q is pre-scaled by
//                    log2(e) / sqrt(hd) and split into fp16 hi + lo (about
//                    22 significant bits); K is exact (the cache is fp16)
//   O^T += V^T P^T   P = exp2(S - max) split into fp16 hi + lo; V exact
//
// Lane l owns query l % 32 in both products (accumulator register i of lane l
// is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32), so the softmax
// statistics are per lane; lanes l and l ^ 32 hold the two halves of a
// block's keys for the same query.  The K rows enter the first product in
// the order pi (bits 2 and 3 of the row index swapped), which puts keys
// 16 s + 8 (l / 32) .. +8 in registers 8 s .. 8 s + 7 of lane l: the B
// operand of k step s of the second product, with no exchange between lanes.
//
// LDS per stage: K as [64 keys][hd] with the 16-byte pieces of a row rotated
// by an XOR of the key (conflict-free first-product reads), and V transposed
// as [hd][64 + 8 keys] (a lane's 8 keys contiguous; the 144-byte row stride
// spreads 16 rows over all banks).  The next stage's global loads are in
// flight during the current stage's products.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPaRows = 64;        // query rows per workgroup
constexpr int kPaKeys = 64;        // keys per stage
constexpr int kPaVst = kPaKeys + 8;  // transposed V row stride (halves)

__host__ __device__ constexpr int pa_stage_halves(int hd) { return kPaKeys * hd + hd * kPaVst; }
__host__ __device__ constexpr size_t pa_lds_bytes(int hd) { return (size_t)2 * pa_stage_halves(hd) * 2; }

// row m of a 32-key block -> key (bits 2 and 3 swapped)
__device__ __forceinline__ int pa_pi(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

template <int HD>
__device__ __forceinline__ int pa_swz(int key) {
    constexpr int NCH = HD / 8, RS = HD == 128 ? 0 : HD == 64 ? 1 : 2;  // rows per 256 bytes = 1 << RS
    return (key >> RS) & (NCH - 1);
}

template <int HD>
__global__ __launch_bounds__(256) void attention_rows_mfma_kernel(const float* __restrict__ q,
                                                                  const __half* __restrict__ kc,
                                                                  const __half* __restrict__ vc,
                                                                  float* __restrict__ att, int p0, int m, int nh,
                                                                  int nkv, float qscale) {
    constexpr int NCH = HD / 8, KS = HD / 16, DB = HD / 32;
    constexpr int NKL = kPaKeys * NCH / 256;  // K pieces per thread per stage
    constexpr int NVB = 16 * NCH;             // 4-key x 8-dim V blocks per stage
    extern __shared__ __align__(16) _Float16 pa_smem[];

    const int g = blockIdx.x, group = nh / nkv, T = kPaRows / group;
    const int t0 = blockIdx.y * T;
    const int kvd = nkv * HD, qd = nh * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qg = wave & 1, kh = wave >> 1, n = lane & 31, h = lane >> 5;

    const int tmax = min(t0 + T, m) - 1;
    const int kend = p0 + tmax + 1;             // keys [0, kend) for the workgroup
    const int lim_min = p0 + t0 + 1;            // smallest per-row limit
    const int nst = (kend + kPaKeys - 1) / kPaKeys;

    // this lane's query row
    const int r = 32 * qg + n, tl = r / group, hh = r % group, tok = t0 + tl;
    const bool valid = r < T * group && tok < m;
    const int lim = valid ? p0 + tok + 1 : lim_min;

    f16x8 qh[KS], ql[KS];
    {
        const float* qp = q + (size_t)tok * qd + (size_t)(g * group + hh) * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            float v[8];
            if (valid) {
                const float4 a = *reinterpret_cast<const float4*>(qp + 16 * ks + 8 * h);
                const float4 b = *reinterpret_cast<const float4*>(qp + 16 * ks + 8 * h + 4);
                v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = 0.f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = v[e] * qscale;
                const _Float16 hi = (_Float16)x;
                qh[ks][e] = hi;
                ql[ks][e] = (_Float16)(x - (float)hi);
            }
        }
    }

    // stage loads: K pieces (key, 16-byte chunk) and V blocks (4 keys x 8 dims)
    uint4 kraw[NKL], vraw[4];
    const size_t col = (size_t)g * HD;
    auto load = [&](int st) {
        const int k0 = st * kPaKeys;
#pragma unroll
        for (int u = 0; u < NKL; ++u) {
            const int i = tid + 256 * u, key = k0 + i / NCH, c = i % NCH;
            kraw[u] = key < kend ? *reinterpret_cast<const uint4*>(kc + (size_t)key * kvd + col + 8 * c)
                                 : make_uint4(0, 0, 0, 0);
        }
        if (tid < NVB) {
            const int kg = tid & 15, c = tid >> 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + 4 * kg + i;
                vraw[i] = key < kend ? *reinterpret_cast<const uint4*>(vc + (size_t)key * kvd + col + 8 * c)
                                     : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store = [&](int buf) {
        _Float16* Ks = pa_smem + buf * pa_stage_halves(HD);
        _Float16* Vt = Ks + kPaKeys * HD;
#pragma unroll
        for (int u = 0; u < NKL; ++u) {
            const int i = tid + 256 * u, key = i / NCH, c = i % NCH;
            *reinterpret_cast<uint4*>(Ks + key * HD + 8 * (c ^ pa_swz<HD>(key))) = kraw[u];
        }
        if (tid < NVB) {
            const int kg = tid & 15, c = tid >> 4;
            const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&vraw[0]);
            const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&vraw[1]);
            const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&vraw[2]);
            const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&vraw[3]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int sh = 16 * (e & 1), wi = e >> 1;
                const uint32_t lo = ((w0[wi] >> sh) & 0xffffu) | (((w1[wi] >> sh) & 0xffffu) << 16);
                const uint32_t hi = ((w2[wi] >> sh) & 0xffffu) | (((w3[wi] >> sh) & 0xffffu) << 16);
                *reinterpret_cast<uint2*>(Vt + (8 * c + e) * kPaVst + 4 * kg) = make_uint2(lo, hi);
            }
        }
    };

    load(0);
    store(0);
    if (nst > 1) load(1);
    __syncthreads();

    float mrun = -INFINITY, lrun = 0.f;
    f32x16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[d][v] = 0.f;
    const int krow = 32 * kh + pa_pi(n);

    for (int st = 0; st < nst; ++st) {
        const _Float16* Ks = pa_smem + (st & 1) * pa_stage_halves(HD);
        const _Float16* Vt = Ks + kPaKeys * HD;
        f32x16 s;
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f16x8 a =
                *reinterpret_cast<const f16x8*>(Ks + krow * HD + 8 * ((2 * ks + h) ^ pa_swz<HD>(krow)));
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qh[ks], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ql[ks], s, 0, 0, 0);
        }
        const int kb = st * kPaKeys + 32 * kh;  // first key of this wave's block
        if (kb + 31 >= lim_min) {
#pragma unroll
            for (int v = 0; v < 16; ++v)
                if (kb + 16 * (v >> 3) + 8 * h + (v & 7) >= lim) s[v] = -INFINITY;
        }
        float mx = s[0];
#pragma unroll
        for (int v = 1; v < 16; ++v) mx = fmaxf(mx, s[v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(mrun, mx);
        const float mref = mnew == -INFINITY ? 0.f : mnew;  // a block with every key masked so far
        const float alpha = __builtin_amdgcn_exp2f(mrun - mref);
        mrun = mnew;
        float p[16], ps = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            p[v] = __builtin_amdgcn_exp2f(s[v] - mref);
            ps += p[v];
        }
        lrun = lrun * alpha + ps;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[d][v] *= alpha;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            f16x8 bh, bl;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const _Float16 hi = (_Float16)p[8 * t + u];
                bh[u] = hi;
                bl[u] = (_Float16)(p[8 * t + u] - (float)hi);
            }
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(Vt + (32 * d + n) * kPaVst + 32 * kh + 16 * t + 8 * h);
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, o[d], 0, 0, 0);
            }
        }
        if (st + 1 < nst) store((st + 1) & 1);
        __syncthreads();
        if (st + 2 < nst) load(st + 2);
    }

    // merge the two key halves of each query set (stage buffers are free now)
    const float lsum = lrun + __shfl_xor(lrun, 32, 64);
    float* mb = reinterpret_cast<float*>(pa_smem) + qg * (HD * 32 + 64);
    if (kh == 1) {
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int v = 0; v < 16; ++v) mb[(32 * d + 8 * (v >> 2) + 4 * h + (v & 3)) * 32 + n] = o[d][v];
        if (h == 0) {
            mb[HD * 32 + n] = mrun;
            mb[HD * 32 + 32 + n] = lsum;
        }
    }
    __syncthreads();
    if (kh == 0 && valid) {
        const float m1 = mb[HD * 32 + n], l1 = mb[HD * 32 + 32 + n];
        const float M = fmaxf(mrun, m1);  // mrun is finite: key 0 is in this wave's first block
        const float a0 = __builtin_amdgcn_exp2f(mrun - M), a1 = __builtin_amdgcn_exp2f(m1 - M);
        const float inv = 1.0f / (a0 * lsum + a1 * l1);
        float* op = att + (size_t)tok * qd + (size_t)(g * group + hh) * HD;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int dim = 32 * d + 8 * i + 4 * h;
                float4 w;
                w.x = (a0 * o[d][4 * i + 0] + a1 * mb[(dim + 0) * 32 + n]) * inv;
                w.y = (a0 * o[d][4 * i + 1] + a1 * mb[(dim + 1) * 32 + n]) * inv;
                w.z = (a0 * o[d][4 * i + 2] + a1 * mb[(dim + 2) * 32 + n]) * inv;
                w.w = (a0 * o[d][4 * i + 3] + a1 * mb[(dim + 3) * 32 + n]) * inv;
                *reinterpret_cast<float4*>(op + dim) = w;
            }
    }
}

template <int HD>
int attention_rows_mfma_launch_hd(const float* q, const __half* kc, const __half* vc, float* att, int p0, int m,
                                  int nh, int nkv, float qscale, hipStream_t st) {
    static bool attr_set = false;  // above 64 KiB of LDS needs the opt-in, once per kernel
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)attention_rows_mfma_kernel<HD>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)pa_lds_bytes(HD)) != hipSuccess)
            return MXH_ERR_HIP;
        attr_set = true;
    }
    const int T = kPaRows / (nh / nkv);
    const dim3 grid((unsigned)nkv, (unsigned)((m + T - 1) / T));
    hipLaunchKernelGGL(attention_rows_mfma_kernel<HD>, grid, dim3(256), pa_lds_bytes(HD), st, q, kc, vc, att, p0, m,
                       nh, nkv, qscale);
    return MXH_OK;
}

}  // namespace

int attention_rows_mfma_launch(const float* q, const __half* kc, const __half* vc, float* att, int p0, int m, int nh,
                               int nkv, int hd, float scale, hipStream_t st) {
    if (m <= 0 || p0 < 0 || !attention_supported(nh, nkv, hd)) return MXH_ERR_ARG;
    const float qscale = scale * 1.4426950408889634f;  // scores in base-2 units
    switch (hd) {
    case 32: return attention_rows_mfma_launch_hd<32>(q, kc, vc, att, p0, m, nh, nkv, qscale, st);
    case 64: return attention_rows_mfma_launch_hd<64>(q, kc, vc, att, p0, m, nh, nkv, qscale, st);
    default: return attention_rows_mfma_launch_hd<128>(q, kc, vc, att, p0, m, nh, nkv, qscale, st);
    }
}

}  // namespace mxh
