// mxh_layer.hip — the non-GEMV kernels of one decoder step, kept on the device.
//
// Reference semantics (minXfmr.cpp):
//   rmsnorm + weight        src/transformer/rmsnorm.cpp:5-26, transformer.cpp:189-214
//   RoPE                    src/transformer/rope.cpp:6-57  (pairs (2i,2i+1) or NeoX)
//   attention (decode)      src/transformer/transformer.cpp:529-629, softmax.cpp:4-18
//   SiLU * up               src/transformer/transformer.cpp:183-185, 696-704
//   greedy / top-k          src/api/minxfmr.cpp:2091-2171
// Qwen3 QK-norm (absent from the reference) is a per-head rmsnorm of q and k
// after the projection and before RoPE.  The KV cache is fp16 in HBM,
// [layer][position][kv_dim] for K and for V.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "mxh_device.h"
#include "mxh_internal.h"
#include "mxh_quant.h"

namespace mxh {
namespace {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// block-wide double sum (blockDim.x a multiple of 64, <= 1024)
__device__ double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// y = float(x / sqrt(mean(x^2) + eps)) * w   (sum of squares in double)
__global__ void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int n,
                               float eps) {
    __shared__ double red[16];
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += (double)x[i] * (double)x[i];
    ss = block_sum_d(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = (float)((double)x[i] * inv);
        y[i] = w ? v * w[i] : v;
    }
}

// timeline hook for out-of-tree probes (empty in the library)
#ifndef MXH_ATTN_STAMP
#define MXH_ATTN_STAMP(i)
#endif

constexpr int kAttnMaxGroup = 8;    // q heads per kv head
// Splits per q head: the grid holds ceil(n_ctx / kAttnSplitPos) of them (at
// most kAttnMaxSplits), and a launch uses min(grid, ceil(L / kAttnRunSplitPos)),
// so short contexts spread over every split the grid has (the o-projection
// merges the grid's partials whatever L is: 607 against 615 tok/s with
// 256-position splits at run time too)
constexpr int kAttnSplitPos = 256;
constexpr int kAttnRunSplitPos = 128;
// Contexts of at least kAttnGroupMinCtx positions run the grouped kernel
// (attention_group_kernel: one workgroup per kv head and split), with the
// grid's splits sized to its capacity and at least kAttnGroupRunPos
// positions per active split
constexpr int kAttnGroupMinCtx = 4096;
constexpr int kAttnGroupRunPos = 64;
constexpr int kAttnGroupBlocks = 3;  // 16-position blocks per wave: 384 positions per workgroup

// Bias, per-head rmsnorm (QK-norm) and RoPE of one head slice, done by one
// wave in two parts: head_fetch requests every global input (so a kernel can
// issue it ahead of its other loads, which complete in order), head_finish
// computes into dst (LDS).  `src` is the raw projection; hd <= 128, lane l
// holds elements l and l + 64.
struct HeadIn {
    float v[2], g[2];
    double c, s;
};

__device__ __forceinline__ HeadIn head_fetch(const float* __restrict__ src, const float* __restrict__ bias,
                                             const float* __restrict__ nw, const double* __restrict__ cs, int hd) {
    const int lane = threadIdx.x & 63, half = hd / 2;
    HeadIn in{{0.f, 0.f}, {1.f, 1.f}, 1.0, 0.0};
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) {
            in.v[r] = src[t] + (bias ? bias[t] : 0.f);
            if (nw) in.g[r] = nw[t];
        }
    }
    if (lane < half) {
        in.c = cs[2 * lane];
        in.s = cs[2 * lane + 1];
    }
    return in;
}

__device__ void head_finish(HeadIn in, bool norm, float* dst, int hd, float eps, int neox) {
    const int lane = threadIdx.x & 63, half = hd / 2;
    if (norm) {
        const double ss = wave_sum_d_all((double)in.v[0] * in.v[0] + (double)in.v[1] * in.v[1]);
        const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
#pragma unroll
        for (int r = 0; r < 2; ++r) in.v[r] = (float)((double)in.v[r] * inv) * in.g[r];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) dst[t] = in.v[r];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // RoPE (rope.cpp:6-57): pair i = (2i, 2i+1), or (i, i + hd/2) for NeoX;
    // lane i reads and rewrites only pair i
    if (lane < half) {
        const int ia = neox ? lane : 2 * lane, ib = neox ? lane + half : 2 * lane + 1;
        const double x0 = dst[ia], x1 = dst[ib];
        dst[ia] = (float)(x0 * in.c - x1 * in.s);
        dst[ib] = (float)(x0 * in.s + x1 * in.c);
    }
}

__device__ void head_prep(const float* __restrict__ src, const float* __restrict__ bias,
                          const float* __restrict__ nw, const double* __restrict__ cs, float* dst, int hd, float eps,
                          int neox) {
    head_finish(head_fetch(src, bias, nw, cs, hd), nw != nullptr, dst, hd, eps, neox);
}

// sum over aligned groups of LPP lanes (a power of two <= 16); every lane of
// the group ends with the group sum
template <int LPP>
__device__ __forceinline__ float lane_group_sum(float v) {
    if (LPP >= 2) v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
    if (LPP >= 4) v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
    if (LPP >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if (LPP >= 16) v += dpp_f<0x140>(v); // row_mirror
    return v;
}

__device__ __forceinline__ void half8_to_float(const uint4& raw, float* f) {
    const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float2 t = __half22float2(h[e]);
        f[2 * e] = t.x;
        f[2 * e + 1] = t.y;
    }
}

// sum over the lanes of a wave with the same lane % LPP (the position
// groups), with VALU lane swaps where the offsets allow
template <int LPP>
__device__ __forceinline__ float fold_position_groups(float v) {
    if constexpr (LPP <= 4) v += lane_xor<4>(v);
    if constexpr (LPP <= 8) v += lane_xor<8>(v);
    if constexpr (LPP <= 16) v += lane_xor<16>(v);
    return v + lane_xor<32>(v);
}

template <int LPP>
__device__ __forceinline__ float fold_position_groups_max(float v) {
    if constexpr (LPP <= 4) v = fmaxf(v, lane_xor<4>(v));
    if constexpr (LPP <= 8) v = fmaxf(v, lane_xor<8>(v));
    if constexpr (LPP <= 16) v = fmaxf(v, lane_xor<16>(v));
    return fmaxf(v, lane_xor<32>(v));
}

// Decode attention (transformer.cpp:529-629, softmax.cpp:4-18) for one q
// head over a split of the L = pos + 1 positions, head_dim = 8 * LPP.
//
// Workgroup (i, s): q head qh of kv head g = i % nkv (qh = g * group +
// i / nkv, so the q heads that share a kv head have workgroup ids equal
// modulo 8 and run on one XCD, whose L2 serves their common K/V rows once),
// split s of S = min(gridDim.y, ceil(L / kAttnRunSplitPos)) contiguous position
// ranges.  It leaves the split's running max m (base-2 units), sum l and
// exp-weighted V sums in `part`; the o-projection's x staging merges the S
// partials of each q head (GEMV_ATTN), so no workgroup waits for another.
// Workgroups past S leave an empty partial (m = -inf, l = 0).
//
// Inside a workgroup each of the 8 waves takes chunks w, w + 8, ... of the
// range (4 positions per lane: 16 positions at head_dim 128), with DB
// chunks' K and V rows in flight per wave (a lane holds 8 dims, one 16-byte
// fp16 load, of each of its positions), and keeps its own running softmax in
// registers; scores are reduced over the LPP lanes of a position with DPP.
// The eight wave partials are merged through LDS at the end.
//
// q is prepared (bias, QK-norm, RoPE) by each workgroup of its head; in the
// last split, which holds position pos, k and v of the current token too,
// rounded through fp16 as every cached position and used from LDS; the
// workgroup of the kv head's first q head appends them to the cache.  No
// cache row written in this launch is read in it.
template <int LPP, int DB, bool RING>
// pos, the caches and q|k|v, needed first, also come as leading scalars that
// the command processor preloads into SGPRs (-amdgpu-kernarg-preload-count).
__global__ __launch_bounds__(512) void attention_kernel(const int* ppos, __half* pkc, __half* pvc, const float* pqkv,
                                                        AttnArgs a) {
    a.pos = ppos;
    a.kc = pkc;
    a.vc = pvc;
    a.qkv = pqkv;
    MXH_ATTN_STAMP(0);
    constexpr int HD = LPP * 8, PR = 64 / LPP, NP = 4, CH = NP * PR, NW = 8;
    __shared__ float qs[HD];
    __shared__ float kvt[HD];
    __shared__ __align__(16) __half kvh[2][HD];
    __shared__ float wm[NW], wl[NW];
    __shared__ __align__(16) float wacc[NW][HD];

    const int group = a.nh / a.nkv, kvd = a.nkv * HD, qd = a.nh * HD;
    const int g = (int)blockIdx.x % a.nkv, qh = g * group + (int)blockIdx.x / a.nkv;
    const int s = blockIdx.y, SM = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane % LPP, pr = lane / LPP;
    // the rows attended: positions 0 .. pos of the window that starts at
    // cache row wrow (RING, past a full ring: the last `ring` tokens, oldest
    // first, then the current one at pos = ring, also its RoPE position)
    const int P = *a.pos;
    const bool wrapped = RING && P >= a.ring;
    const int pos = wrapped ? a.ring : P, L = pos + 1;
    const int wrow = wrapped ? (P + 1) % (a.ring + 1) : 0;
    const int S = min(SM, (L + kAttnRunSplitPos - 1) / kAttnRunSplitPos);
    MXH_ATTN_STAMP(1);
    float* part_v = a.part;                              // [nh][SM][HD]
    float* part_ml = a.part + (size_t)a.nh * SM * HD;    // [nh][SM][2]
    const size_t slot = (size_t)qh * SM + s;
    if (s >= S) {
        if (tid == 0) {
            part_ml[slot * 2] = -INFINITY;
            part_ml[slot * 2 + 1] = 0.f;
        }
        return;
    }
    // this split's positions [p0, p1); the last one ends at pos, which comes
    // from LDS, so the cache rows read are [p0, min(p1, pos))
    const int p0 = (int)((int64_t)L * s / S), p1 = (int)((int64_t)L * (s + 1) / S);
    const bool last = s == S - 1;
    const int rows_end = last ? pos : p1;
    const int nch = (p1 - p0 + CH - 1) / CH;
    const size_t col = (size_t)g * HD + sub * 8;

    // K and V through buffer descriptors over the rows [0, rows_end): rows
    // past them read 0 without a branch, so every wait below is for exactly
    // the loads it needs (predicated loads left the compiler waiting for all)
    uint4 kraw[DB][NP], vraw[DB][NP];
    const __amdgpu_buffer_rsrc_t krs = buf_rsrc(a.kc + (size_t)wrow * kvd, rows_end * kvd * 2);
    const __amdgpu_buffer_rsrc_t vrs = buf_rsrc(a.vc + (size_t)wrow * kvd, rows_end * kvd * 2);
    auto load = [&](int b, int c) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int j = p0 + c * CH + i * PR + pr;
            kraw[b][i] = ld_buf16(krs, (j * kvd + (int)col) * 2);
            vraw[b][i] = ld_buf16(vrs, (j * kvd + (int)col) * 2);
        }
    };
    // wave 0: q; in the last split wave 1: k, wave 2: v of the current
    // token.  Their inputs are requested first, then the wave's first DB
    // chunks (loads complete in order, so the preparation does not wait for
    // the chunks).
    const double* cs = a.rope_cs + (size_t)pos * HD;  // (hd/2) pairs of (cos, sin)
    const bool prep = wave == 0 || (last && wave <= 2), is_k = wave == 1;
    const size_t off = wave == 0 ? (size_t)qh * HD : (is_k ? qd : qd + kvd) + (size_t)g * HD;
    HeadIn hin{};
    if (prep)
        hin = head_fetch(a.qkv + off, a.bias ? a.bias + off : nullptr,
                         wave == 0 ? a.q_norm : is_k ? a.k_norm : nullptr, cs, HD);
    // unconditionally (chunks past the split read zeros and are not used), so
    // the preparation below waits for its own inputs only
#pragma unroll
    for (int b = 0; b < DB; ++b) load(b, wave + NW * b);
    MXH_ATTN_STAMP(2);

    if (wave == 0) {
        head_finish(hin, a.q_norm != nullptr, qs, HD, a.eps, a.neox);
    } else if (prep) {
        if (is_k) {
            head_finish(hin, a.k_norm != nullptr, kvt, HD, a.eps, a.neox);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        }
        // rounded through fp16 like every cached position; appended once
        // per kv head (past a full ring to both copies of the token's slot)
        const bool append = qh % group == 0;
        const int prow = wrow + pos;
        __half* cache = (is_k ? a.kc : a.vc) + (size_t)prow * kvd + (size_t)g * HD;
        __half* twin = wrapped ? cache + (prow <= a.ring ? 1 : -1) * (ptrdiff_t)(a.ring + 1) * kvd : nullptr;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int t = lane + 64 * r;
            if (t < HD) {
                const __half hv = __float2half_rn(is_k ? kvt[t] : hin.v[r]);
                kvh[is_k ? 0 : 1][t] = hv;
                if (append) {
                    cache[t] = hv;
                    if (twin) twin[t] = hv;
                }
            }
        }
    }
    __syncthreads();
    MXH_ATTN_STAMP(3);

    float qreg[8], acc[8], run_m = -INFINITY, run_l = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        qreg[e] = qs[sub * 8 + e];
        acc[e] = 0.f;
    }
    // scores in base-2 units (exp(x - m) == exp2(x log2 e - m log2 e))
    const float scale2 = a.scale * 1.4426950408889634f;
    auto chunk = [&](int b, int c) {
        // the current position (last split) from the LDS copies
        if (last && c == (pos - p0) / CH) {
#pragma unroll
            for (int i = 0; i < NP; ++i)
                if (p0 + c * CH + i * PR + pr == pos) {
                    kraw[b][i] = *reinterpret_cast<const uint4*>(&kvh[0][sub * 8]);
                    vraw[b][i] = *reinterpret_cast<const uint4*>(&kvh[1][sub * 8]);
                }
        }
        float sc[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int j = p0 + c * CH + i * PR + pr;
            float kf[8];
            half8_to_float(kraw[b][i], kf);
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qreg[e], kf[e], d);
            d = lane_group_sum<LPP>(d);
            sc[i] = j < p1 ? d * scale2 : -INFINITY;
        }
        // running softmax over this wave's positions (every chunk holds at
        // least one position, so the new max is finite unless a score is
        // NaN, which then propagates)
        float mc = sc[0];
#pragma unroll
        for (int i = 1; i < NP; ++i) mc = fmaxf(mc, sc[i]);
        mc = fold_position_groups_max<LPP>(mc);
        const float mn = fmaxf(run_m, mc);
        const float al = __builtin_amdgcn_exp2f(run_m - mn);
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            sc[i] = __builtin_amdgcn_exp2f(sc[i] - mn);
            ps += sc[i];
        }
        run_l = run_l * al + fold_position_groups<LPP>(ps);
        run_m = mn;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= al;
        // exp-weighted V
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            float vf[8];
            half8_to_float(vraw[b][i], vf);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(sc[i], vf[e], acc[e]);
        }
    };
    // chunks wave, wave + 8, ...: the wave's k-th chunk sits in buffer
    // k % DB, which is refilled with the chunk DB further on once consumed
    for (int c0 = wave; c0 < nch; c0 += NW * DB) {
#pragma unroll
        for (int b = 0; b < DB; ++b) {
            const int c = c0 + NW * b;
            if (c < nch) {
                chunk(b, c);
                if (c + NW * DB < nch) load(b, c + NW * DB);
            }
        }
    }
    MXH_ATTN_STAMP(4);

    // the wave's partial (V sums folded over its position rows) to LDS
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fold_position_groups<LPP>(acc[e]);
    if (lane < LPP) {
        float4* dst = reinterpret_cast<float4*>(&wacc[wave][sub * 8]);
        dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    if (lane == 0) {
        wm[wave] = run_m;
        wl[wave] = run_l;
    }
    __syncthreads();
    MXH_ATTN_STAMP(5);
    // merge the waves (a wave without chunks has m = -inf, weight 0) and
    // store the workgroup's partial
    if (tid < HD) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w]);
        float l = 0.f, v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = wm[w];
            const float ww = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
            l = fmaf(ww, wl[w], l);
            v = fmaf(ww, wacc[w][tid], v);
        }
        part_v[slot * HD + tid] = v;
        if (tid == 0) {
            part_ml[slot * 2] = M;
            part_ml[slot * 2 + 1] = l;
        }
    }
}

// Fold v[0..N) (N a multiple of 4) over the lanes of equal lane % LPP
// (sums over the position groups of a wave), two values per lane swap for
// lane bits 5 and 4: afterwards register w[k] holds, in 16-lane row r, the
// sum of v[4 k + c(r)], c = {0, 2, 1, 3}; lanes below 16 in row r with
// lane % 16 < LPP carry it (lane bits below 4 and at or above log2 LPP were
// folded lane by lane first).
template <int LPP, int N>
__device__ __forceinline__ void fold_pairs(float (&v)[N], float (&w)[N / 4]) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if constexpr (LPP <= 4) v[k] += lane_xor<4>(v[k]);
        if constexpr (LPP <= 8) v[k] += lane_xor<8>(v[k]);
    }
    float u[N / 2];
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2 * k]), __float_as_uint(v[2 * k + 1]),
                                                        false, false);
        u[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(u[2 * k]), __float_as_uint(u[2 * k + 1]),
                                                        false, false);
        w[k] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
}

// Decode attention for long contexts (transformer.cpp:529-629), grouped by
// kv head: workgroup (g, s) serves all G = nh / nkv q heads of kv head g over
// split s of the L = pos + 1 positions, so each K/V byte of the cache is read
// into one CU once.
//
// S = min(gridDim.y, ceil(L / kAttnGroupRunPos)) splits are active; split s
// holds positions [L s / S, L (s + 1) / S), at most 8 waves x NB blocks x 16
// = 384, which the grid size guarantees (attention_splits).  Wave w takes the
// 16-position blocks w, w + 8, w + 16; waves 0 .. G-1 first prepare one q
// head each (bias, QK-norm, RoPE) and publish it through an LDS counter that
// the others poll before their first scores (no barrier behind any wave's
// load issue), and each wave issues block b + 1's K and V loads before block
// b is computed (a
// wave's loads issue in order and stall while the CU's memory queue is full,
// so work placed behind later loads waits for their issue).  Loads go through buffer
// descriptors over the cache rows [0, rows_end): rows past them read 0
// without a branch, so every wait is for exactly the loads it needs; blocks
// past the split are loaded as zeros and not computed.  Per block:
//   - scores on the matrix cores: S[p][h] = K[p] . q'[h] by
//     v_mfma_f32_16x16x32_f16 with K (exact fp16) as A, lane l holding
//     position l % 16 and dims 32 ks + 8 (l / 16) .. +8 of k-step ks, and q' =
//     q scale log2 e as B, columns h < G, split into fp16 hi and lo (two
//     products, about 22 significant bits of q).  Lane l then holds head
//     l % 16 at positions 4 (l / 16) + i;
//   - the running max and sum per head (online softmax); the probabilities
//     and the rescale factor go through LDS to the layout of the V rows;
//   - exp-weighted V on the VALU, lane l holding 8 dims (l % LPP) of position
//     row l / LPP, V as loaded (16 bytes per lane and row).
// The eight wave partials merge through LDS; the split's partial (max in
// base-2 units, sum, V sums) goes to `part` in attention_kernel's layout,
// slot (g G + h) gridDim.y + s, for attention_merge_kernel.  In the last
// split the wave whose blocks hold position pos prepares the current token's
// k and v, rounds them through fp16, appends them to the cache and uses them
// from LDS, as attention_kernel does.
template <int LPP, int G, bool RING>
__global__ __launch_bounds__(512) void attention_group_kernel(const int* ppos, __half* pkc, __half* pvc,
                                                              const float* pqkv, AttnArgs a) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    MXH_ATTN_STAMP(0);
    a.pos = ppos;
    a.kc = pkc;
    a.vc = pvc;
    a.qkv = pqkv;
    constexpr int HD = LPP * 8, PR = 64 / LPP, NW = 8, NB = kAttnGroupBlocks, KS = HD / 32, RB = 16 / PR;
    static_assert(G <= NW, "one preparing wave per q head");
    __shared__ float qs[G][HD];
    __shared__ int qready;  // q heads published in qs
    __shared__ float kvt[HD];
    __shared__ __align__(16) __half kvh[2][HD];
    __shared__ __align__(16) float ps[NW][16][G];
    __shared__ __align__(16) float pal[NW][G];
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float wacc[NW][G * 8][16];

    const int kvd = a.nkv * HD, qd = a.nh * HD;
    const int g = blockIdx.x, s = blockIdx.y, SM = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane % LPP, pr = lane / LPP, l16 = lane & 15, quad = lane >> 4;
    // the window of rows attended, as in attention_kernel
    const int P = *a.pos;
    const bool wrapped = RING && P >= a.ring;
    const int pos = wrapped ? a.ring : P, L = pos + 1;
    const int wrow = wrapped ? (P + 1) % (a.ring + 1) : 0;
    const int S = min(SM, (L + kAttnGroupRunPos - 1) / kAttnGroupRunPos);
    float* part_v = a.part;                            // [nh][SM][HD]
    float* part_ml = a.part + (size_t)a.nh * SM * HD;  // [nh][SM][2]
    if (s >= S) {
        if (tid < G) {
            const size_t slot = (size_t)(g * G + tid) * SM + s;
            part_ml[slot * 2] = -INFINITY;
            part_ml[slot * 2 + 1] = 0.f;
        }
        return;
    }
    const int p0 = (int)((int64_t)L * s / S), p1 = (int)((int64_t)L * (s + 1) / S);
    const bool last = s == S - 1;
    const int rows_end = last ? pos : p1;  // cache rows read: [p0, rows_end)
    // wave t < G prepares q head t and publishes it; the wave whose blocks
    // hold position pos (last split) prepares the current token's k and v
    const bool q_wave = wave < G;
    const bool kv_wave = last && ((pos - p0) >> 4) % NW == wave;
    if (tid == 0) qready = 0;
    __syncthreads();

    const double* cs = a.rope_cs + (size_t)pos * HD;
    HeadIn qin{}, kin_h{}, vin_h{};
    if (q_wave) {
        const size_t off = (size_t)(g * G + wave) * HD;
        qin = head_fetch(a.qkv + off, a.bias ? a.bias + off : nullptr, a.q_norm, cs, HD);
    }
    if (kv_wave) {
        const size_t ko = (size_t)qd + (size_t)g * HD, vo = (size_t)(qd + kvd) + (size_t)g * HD;
        kin_h = head_fetch(a.qkv + ko, a.bias ? a.bias + ko : nullptr, a.k_norm, cs, HD);
        vin_h = head_fetch(a.qkv + vo, a.bias ? a.bias + vo : nullptr, nullptr, cs, HD);
    }
    if (q_wave) {
        head_finish(qin, a.q_norm != nullptr, qs[wave], HD, a.eps, a.neox);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&qready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (kv_wave) {
        head_finish(kin_h, a.k_norm != nullptr, kvt, HD, a.eps, a.neox);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        // rounded through fp16 like every cached position and appended (this
        // workgroup is the only one of kv head g holding position pos; past a
        // full ring to both copies of the token's slot)
        const int prow = wrow + pos;
        const ptrdiff_t twin = wrapped ? (prow <= a.ring ? 1 : -1) * (ptrdiff_t)(a.ring + 1) * kvd : 0;
        __half* kdst = a.kc + (size_t)prow * kvd + (size_t)g * HD;
        __half* vdst = a.vc + (size_t)prow * kvd + (size_t)g * HD;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int e = lane + 64 * r;
            if (e < HD) {
                const __half kh = __float2half_rn(kvt[e]), vh = __float2half_rn(vin_h.v[r]);
                kvh[0][e] = kh;
                kvh[1][e] = vh;
                kdst[e] = kh;
                vdst[e] = vh;
                if (twin) {
                    kdst[e + twin] = kh;
                    vdst[e + twin] = vh;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    // K (matrix-core operand layout) and V (row layout) of block b into slot b % 2
    uint4 kraw[2][KS], vraw[2][RB];
    const __amdgpu_buffer_rsrc_t krs = buf_rsrc(a.kc + (size_t)wrow * kvd, rows_end * kvd * 2);
    const __amdgpu_buffer_rsrc_t vrs = buf_rsrc(a.vc + (size_t)wrow * kvd, rows_end * kvd * 2);
    auto issue = [&](int b) {
        const int b0 = p0 + (wave + NW * b) * 16;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            kraw[b & 1][ks] = ld_buf16(krs, ((b0 + l16) * kvd + g * HD + 32 * ks + 8 * quad) * 2);
#pragma unroll
        for (int r = 0; r < RB; ++r) vraw[b & 1][r] = ld_buf16(vrs, ((b0 + r * PR + pr) * kvd + g * HD + sub * 8) * 2);
    };
    issue(0);
    MXH_ATTN_STAMP(1);
    // wait until the G q heads are published (the preparing waves never
    // wait on anything; the bound only keeps a wave from spinning forever)
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__hip_atomic_load(&qready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= G) break;
        __builtin_amdgcn_s_sleep(1);
    }
    MXH_ATTN_STAMP(2);

    // q' = q scale log2 e as the B operand: column l16 < G is head l16, fp16
    // hi and lo halves
    const float scale2 = a.scale * 1.4426950408889634f;
    h8 qhi[KS], qlo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = l16 < G ? qs[l16 < G ? l16 : 0][32 * ks + 8 * quad + e] * scale2 : 0.f;
            const _Float16 hi = (_Float16)v;
            qhi[ks][e] = hi;
            qlo[ks][e] = (_Float16)(v - (float)hi);
        }
    // running max / sum per head (score layout: column l16) and V sums
    // (row layout: acc[h 8 + e] is dim sub 8 + e of head h)
    float m_run = -INFINITY, l_run = 0.f;
    float acc[G * 8];
#pragma unroll
    for (int k = 0; k < G * 8; ++k) acc[k] = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b + 1 < NB) issue(b + 1);
        const int b0 = p0 + (wave + NW * b) * 16;  // wave-uniform
        if (b0 >= p1) continue;
        // scores (base-2 units) on the matrix cores; the current position's k
        // (last split) from the LDS copy in place of the zeros its load returned
        uint4 kin[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kin[ks] = kraw[b & 1][ks];
        if (last && pos - b0 < 16) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                if (b0 + l16 == pos) kin[ks] = *reinterpret_cast<const uint4*>(&kvh[0][32 * ks + 8 * quad]);
        }
        f4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const h8 kv = __builtin_bit_cast(h8, kin[ks]);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qhi[ks], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qlo[ks], sacc, 0, 0, 0);
        }
        float sc[4];
        float bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = (l16 < G && b0 + 4 * quad + i < p1) ? sacc[i] : -INFINITY;
            bm = fmaxf(bm, sc[i]);
        }
        bm = fmaxf(bm, lane_xor<16>(bm));
        bm = fmaxf(bm, lane_xor<32>(bm));
        // the block holds at least one position, so mn is finite for l16 < G
        const float mn = fmaxf(m_run, bm);
        const float al = __builtin_amdgcn_exp2f(m_run - mn);  // 0 while m_run = -inf
        float bs = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = __builtin_amdgcn_exp2f(sc[i] - mn);
            bs += sc[i];
        }
        bs += lane_xor<16>(bs);
        bs += lane_xor<32>(bs);
        l_run = fmaf(l_run, al, bs);
        m_run = mn;
        // probabilities and rescale factors to the row layout
        if (l16 < G) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ps[wave][4 * quad + i][l16] = sc[i];
            if (quad == 0) pal[wave][l16] = al;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        float alh[G];
#pragma unroll
        for (int h = 0; h < G; ++h) alh[h] = pal[wave][h];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h * 8 + e] *= alh[h];
        // exp-weighted V; the current position's v from the LDS copy
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int q = r * PR + pr;
            uint4 vin = vraw[b & 1][r];
            if (last && pos - b0 - r * PR >= 0 && pos - b0 - r * PR < PR) {
                if (b0 + q == pos) vin = *reinterpret_cast<const uint4*>(&kvh[1][sub * 8]);
            }
            float p[G];
#pragma unroll
            for (int h = 0; h < G; ++h) p[h] = ps[wave][q][h];
            float vf[8];
            half8_to_float(vin, vf);
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h * 8 + e] = fmaf(p[h], vf[e], acc[h * 8 + e]);
        }
        // the next block's writes to ps / pal come after these reads
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    MXH_ATTN_STAMP(5);
    // the wave's partials (V sums folded over its position rows) to LDS:
    // wacc[wave][h 8 + e][sub] holds dim sub 8 + e of head h
    float wsum[G * 2];
    fold_pairs<LPP, G * 8>(acc, wsum);
    if (l16 < LPP) {
        const int r = quad, c = ((r & 1) << 1) | (r >> 1);
#pragma unroll
        for (int k = 0; k < G * 2; ++k) wacc[wave][4 * k + c][l16] = wsum[k];
    }
    if (lane < G) {
        wm[wave][lane] = m_run;
        wl[wave][lane] = l_run;
    }
    __syncthreads();
    MXH_ATTN_STAMP(6);
    // merge the waves per head and store the split's partials
    for (int i = tid; i < G * HD; i += 64 * NW) {
        const int h = i / HD, t = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][h]);
        float l = 0.f, v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = wm[w][h];
            const float ww = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
            l = fmaf(ww, wl[w][h], l);
            v = fmaf(ww, wacc[w][h * 8 + t % 8][t / 8], v);
        }
        const size_t slot = (size_t)(g * G + h) * SM + s;
        part_v[slot * HD + t] = v;
        if (t == 0) {
            part_ml[slot * 2] = M;
            part_ml[slot * 2 + 1] = l;
        }
    }
    MXH_ATTN_STAMP(7);
}

// ---- batched prefill ---------------------------------------------------------

// Row-batched head preparation for prompt tokens p0 .. p0+m-1: workgroup
// (z, h) is one wave for q head h, k head h - nh or v head h - nh - nkv of
// token z.  q goes to q_out (fp32), k and v (rounded to fp16) to the cache at
// position p0 + z (transformer.cpp:385-470 per token; QK-norm as head_prep).
// Batched prompts stay below a full ring (AttnArgs::ring), whose rows need no
// second copy.
__global__ __launch_bounds__(64) void qkv_prep_rows_kernel(const float* __restrict__ qkv, int ldq,
                                                           const float* __restrict__ bias,
                                                           const float* __restrict__ q_norm,
                                                           const float* __restrict__ k_norm,
                                                           const double* __restrict__ rope_cs, int p0,
                                                           float* __restrict__ q_out, __half* __restrict__ kc,
                                                           __half* __restrict__ vc, int nh, int nkv, int hd,
                                                           int neox, float eps) {
    __shared__ float buf[128];
    const int z = blockIdx.x, hidx = blockIdx.y, lane = threadIdx.x;
    const int pos = p0 + z, qd = nh * hd, kvd = nkv * hd;
    const float* row = qkv + (size_t)z * ldq;
    const double* cs = rope_cs + (size_t)pos * hd;
    if (hidx < nh + nkv) {
        const bool is_q = hidx < nh;
        const size_t off = is_q ? (size_t)hidx * hd : (size_t)qd + (size_t)(hidx - nh) * hd;
        head_prep(row + off, bias ? bias + off : nullptr, is_q ? q_norm : k_norm, cs, buf, hd, eps, neox);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        for (int t = lane; t < hd; t += 64) {
            if (is_q) q_out[(size_t)z * qd + off + t] = buf[t];
            else kc[(size_t)pos * kvd + (size_t)(hidx - nh) * hd + t] = __float2half_rn(buf[t]);
        }
    } else {
        const int g = hidx - nh - nkv;
        const size_t off = (size_t)qd + kvd + (size_t)g * hd;
        for (int t = lane; t < hd; t += 64)
            vc[(size_t)pos * kvd + (size_t)g * hd + t] = __float2half_rn(row[off + t] + (bias ? bias[off + t] : 0.f));
    }
}

// h[i] = silu(g[i]) * u[i], gu = [g | u]
__global__ void silu_mul_kernel(const float* __restrict__ gu, float* __restrict__ h, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gu[i];
    h[i] = g / (1.0f + expf(-g)) * gu[n + i];
}

// x = dequantized row tokens[*pos] of the embedding table
template <int TYPE>
__global__ void embed_kernel(const uint8_t* __restrict__ w, const int* __restrict__ tokens,
                             const int* __restrict__ pos_p, float* __restrict__ x, int cols, int form) {
    const int run = blockIdx.x * blockDim.x + threadIdx.x;  // 32 outputs each
    if (run * 32 >= cols) return;
    const size_t rb = row_bytes(TYPE, cols);
    const uint8_t* rp = w + (size_t)tokens[*pos_p] * rb;
    float* y = x + run * 32;
    if constexpr (TYPE == MXH_Q4_K || TYPE == MXH_Q5_K) {
        constexpr int BB = TYPE == MXH_Q4_K ? 144 : 176;
        const uint8_t* blk = rp + (size_t)(run >> 3) * BB;
        const int j = run & 7;
        auto u16 = [&](int o) { return (uint32_t)blk[o] | ((uint32_t)blk[o + 1] << 8); };
        const float d = half_bits_to_float(u16(0)), dm = half_bits_to_float(u16(2));
        uint32_t sc, mn;
        k4_scale_min(u16(4) | (u16(6) << 16), u16(8) | (u16(10) << 16), u16(12) | (u16(14) << 16), j, form, sc, mn);
        const float ds = d * (float)sc, ms = dm * (float)mn;
        const uint8_t* qs = blk + (TYPE == MXH_Q4_K ? 16 : 48) + 32 * (j >> 1);
        for (int i = 0; i < 32; ++i) {
            uint32_t q = (j & 1) ? (qs[i] >> 4) : (qs[i] & 15u);
            if constexpr (TYPE == MXH_Q5_K) q |= ((blk[16 + i] >> j) & 1u) << 4;
            y[i] = ds * (float)q - ms;
        }
    } else if constexpr (TYPE == MXH_Q8_0) {
        const uint8_t* blk = rp + (size_t)run * 34;
        const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int)(int8_t)blk[2 + i];
    } else if constexpr (TYPE == MXH_F16) {
        for (int i = 0; i < 32; ++i) y[i] = half_bits_to_float((uint32_t)rp[2 * (run * 32 + i)] | ((uint32_t)rp[2 * (run * 32 + i) + 1] << 8));
    } else if constexpr (TYPE == MXH_Q5_0 || TYPE == MXH_Q6_K) {
        float t[32];
        dequant_run32<TYPE>(rp, run, form, t);
        for (int i = 0; i < 32; ++i) y[i] = t[i];
    } else {
        for (int i = 0; i < 32; ++i) y[i] = reinterpret_cast<const float*>(rp)[run * 32 + i];
    }
}

// argmax over n logits, lowest index on ties (minxfmr.cpp:2091-2115: greedy
// takes order[0] of a descending sort); the id becomes tokens[*pos + 1], the
// next step's input.
__global__ void argmax_kernel(const float* __restrict__ logits, int n, int* __restrict__ tokens,
                              const int* __restrict__ pos_p) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = logits[i];
        if (v > best || (v == best && i < idx)) { best = v; idx = i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) { best = bv[w]; idx = bi[w]; }
        if (idx == 0x7fffffff) idx = 0;  // all-NaN logits: token 0
        tokens[*pos_p + 1] = idx;
    }
}

__global__ void add_int_kernel(int* p, int v) {
    if (threadIdx.x == 0) p[0] += v;
}

}  // namespace

int rmsnorm_launch(const float* x, const float* w, float* y, int n, float eps, hipStream_t st) {
    if (n <= 0) return MXH_ERR_ARG;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, y, n, eps);
    return MXH_OK;
}

namespace {

}  // namespace

// Whether a context of n_ctx positions runs the grouped kernel: long
// contexts, and q heads per kv head a power of two
static bool attention_grouped(int n_ctx, int nh, int nkv, int hd) {
    const int G = nkv > 0 ? nh / nkv : 0;
    // the cache's byte offsets are 32-bit buffer offsets
    return n_ctx >= kAttnGroupMinCtx && (G == 1 || G == 2 || G == 4 || G == 8) &&
           (int64_t)n_ctx * nkv * hd * 2 < ((int64_t)1 << 31);
}

// CUs of the current device (256 on MI355X), read once
static int attention_cus() {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu < 1)
            n_cu = 256;
    }
    return n_cu;
}

// Splits (partials per q head) for a context of n_ctx positions.  Per-q-head
// kernel: one per kAttnSplitPos positions, at most kAttnMaxSplits (the
// o-projection merges that many partials per q head in its x staging).
// Grouped kernel: one workgroup per CU over the kv heads (no CU takes two)
// unless a split would then exceed a workgroup's 8 x 16 kAttnGroupBlocks
// positions; the merge kernel combines them before the o-projection.
int attention_splits(int n_ctx, int nh, int nkv, int hd) {
    if (attention_grouped(n_ctx, nh, nkv, hd)) {
        const int cap = 8 * 16 * kAttnGroupBlocks;
        const int need = (n_ctx + cap - 1) / cap, fill = attention_cus() / nkv;
        return need > fill ? need : fill;
    }
    const int S = (n_ctx + kAttnSplitPos - 1) / kAttnSplitPos;
    return S < 1 ? 1 : S > kAttnMaxSplits ? kAttnMaxSplits : S;
}

// head_dim 32, 64 or 128 (8 dims per lane, a power-of-two lane count per
// position); at most kAttnMaxGroup q heads per kv head
bool attention_supported(int nh, int nkv, int hd) {
    return nkv > 0 && nh % nkv == 0 && nh / nkv <= kAttnMaxGroup && (hd == 32 || hd == 64 || hd == 128);
}

template <int LPP, bool RING>
static void attention_group_launch(const AttnArgs& a, dim3 grid, hipStream_t st) {
#define MXH_GROUP_CASE(G) \
    hipLaunchKernelGGL((attention_group_kernel<LPP, G, RING>), grid, dim3(512), 0, st, a.pos, a.kc, a.vc, a.qkv, a)
    switch (a.nh / a.nkv) {
    case 1: MXH_GROUP_CASE(1); break;
    case 2: MXH_GROUP_CASE(2); break;
    case 4: MXH_GROUP_CASE(4); break;
    default: MXH_GROUP_CASE(8); break;
    }
#undef MXH_GROUP_CASE
}

template <bool RING>
static void attention_dispatch(const AttnArgs& a, int n_ctx, hipStream_t st) {
    if (attention_grouped(n_ctx, a.nh, a.nkv, a.hd)) {
        const dim3 grid(a.nkv, attention_splits(n_ctx, a.nh, a.nkv, a.hd));
        switch (a.hd) {
        case 32: attention_group_launch<4, RING>(a, grid, st); break;
        case 64: attention_group_launch<8, RING>(a, grid, st); break;
        default: attention_group_launch<16, RING>(a, grid, st); break;
        }
        return;
    }
    const dim3 grid(a.nh, attention_splits(n_ctx, a.nh, a.nkv, a.hd));
#define MXH_HEAD_CASE(LPP) \
    hipLaunchKernelGGL((attention_kernel<LPP, 1, RING>), grid, dim3(512), 0, st, a.pos, a.kc, a.vc, a.qkv, a)
    switch (a.hd) {
    case 32: MXH_HEAD_CASE(4); break;
    case 64: MXH_HEAD_CASE(8); break;
    default: MXH_HEAD_CASE(16); break;
    }
#undef MXH_HEAD_CASE
}

// ring > 0 selects the kernels that handle a full ring; a step below a full
// cache runs the same on either (the host picks them only for steps at or
// past n_ctx tokens, which keeps the others free of the ring's arithmetic)
int attention_run(const AttnArgs& a, int n_ctx, hipStream_t st) {
    if (!attention_supported(a.nh, a.nkv, a.hd)) return MXH_ERR_UNSUPPORTED;
    if (a.ring > 0) attention_dispatch<true>(a, n_ctx, st);
    else attention_dispatch<false>(a, n_ctx, st);
    return MXH_OK;
}

// att[h][t] = sum_s w_s V_s[t] / sum_s w_s l_s, w_s = 2^(m_s - max m) over
// the splits of q head h (a split with m_s = -inf held no position).  One
// wave per (q head, 8 dims): lane s takes splits s, s + 64, ..., keeping a
// running (max, sum, 8 V sums), so with at most 64 splits every load of the
// wave is in flight at once; the lanes then merge by wave reductions.
__global__ __launch_bounds__(256) void attention_merge_kernel(const float* __restrict__ part, int S, int nh, int hd,
                                                              float* __restrict__ att) {
    const int lane = threadIdx.x & 63, groups = hd / 8;
    const int wid = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    if (wid >= nh * groups) return;  // whole waves
    const int h = wid / groups, t0 = (wid % groups) * 8;
    const float* ml = part + (size_t)nh * S * hd + (size_t)h * S * 2;
    const float* pv = part + (size_t)h * S * hd + t0;
    float m = -INFINITY, l = 0.f, v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = lane; s < S; s += 64) {
        const float2 q = *reinterpret_cast<const float2*>(ml + 2 * s);
        const float4 a = *reinterpret_cast<const float4*>(pv + (size_t)s * hd);
        const float4 b = *reinterpret_cast<const float4*>(pv + (size_t)s * hd + 4);
        // an empty split's V partial is whatever an earlier launch left
        // (possibly not finite): skip it rather than weight it by 0
        if (q.x == -INFINITY) continue;
        const float mn = fmaxf(m, q.x);
        const float al = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
        const float w = __builtin_amdgcn_exp2f(q.x - mn);
        const float u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        l = fmaf(w, q.y, l * al);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = fmaf(w, u[e], v[e] * al);
        m = mn;
    }
    const float M = wave_max_all(m);
    const float sc = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    const float den = wave_sum_all(l * sc);
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = wave_sum_all(v[e] * sc);
    if (lane == 0) {
        float4* dst = reinterpret_cast<float4*>(att + (size_t)h * hd + t0);
        dst[0] = make_float4(out[0] / den, out[1] / den, out[2] / den, out[3] / den);
        dst[1] = make_float4(out[4] / den, out[5] / den, out[6] / den, out[7] / den);
    }
}

int attention_merge_launch(const float* part, int splits, int nh, int hd, float* att, hipStream_t st) {
    if (splits < 1 || nh < 1 || hd < 8 || hd % 8) return MXH_ERR_ARG;
    const int waves = nh * (hd / 8);
    hipLaunchKernelGGL(attention_merge_kernel, dim3((waves + 3) / 4), dim3(256), 0, st, part, splits, nh, hd, att);
    return MXH_OK;
}

// V partials [nh][S][hd] followed by (max, sum) pairs [nh][S][2]
size_t attention_scratch_floats(int nh, int nkv, int hd, int n_ctx) {
    return (size_t)nh * attention_splits(n_ctx, nh, nkv, hd) * (hd + 2);
}

int qkv_prep_rows_launch(const float* qkv, int ldq, const float* bias, const float* q_norm, const float* k_norm,
                         const double* rope_cs, int p0, int m, float* q_out, __half* kc, __half* vc, int nh, int nkv,
                         int hd, int neox, float eps, hipStream_t st) {
    if (m <= 0 || !attention_supported(nh, nkv, hd)) return MXH_ERR_ARG;
    hipLaunchKernelGGL(qkv_prep_rows_kernel, dim3(m, nh + 2 * nkv), dim3(64), 0, st, qkv, ldq, bias, q_norm, k_norm,
                       rope_cs, p0, q_out, kc, vc, nh, nkv, hd, neox, eps);
    return MXH_OK;
}

int silu_mul_launch(const float* gu, float* h, int n, hipStream_t st) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, st, gu, h, n);
    return MXH_OK;
}

int embed_launch(int type, const void* w, const int* tokens, const int* pos, float* x, int cols, int form,
                 hipStream_t st) {
    const int runs = cols / 32;
    dim3 grid((runs + 63) / 64), block(64);
    switch (type) {
    case MXH_Q4_K: hipLaunchKernelGGL(embed_kernel<MXH_Q4_K>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_Q5_K: hipLaunchKernelGGL(embed_kernel<MXH_Q5_K>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_Q8_0: hipLaunchKernelGGL(embed_kernel<MXH_Q8_0>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_Q5_0: hipLaunchKernelGGL(embed_kernel<MXH_Q5_0>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_Q6_K: hipLaunchKernelGGL(embed_kernel<MXH_Q6_K>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_F16: hipLaunchKernelGGL(embed_kernel<MXH_F16>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    case MXH_F32: hipLaunchKernelGGL(embed_kernel<MXH_F32>, grid, block, 0, st, (const uint8_t*)w, tokens, pos, x, cols, form); break;
    default: return MXH_ERR_UNSUPPORTED;
    }
    return MXH_OK;
}

int argmax_launch(const float* logits, int n, int* tokens, const int* pos, hipStream_t st) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, logits, n, tokens, pos);
    return MXH_OK;
}

int add_int_launch(int* p, int v, hipStream_t st) {
    hipLaunchKernelGGL(add_int_kernel, dim3(1), dim3(64), 0, st, p, v);
    return MXH_OK;
}

}  // namespace mxh
