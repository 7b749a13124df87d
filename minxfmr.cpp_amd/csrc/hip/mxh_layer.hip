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

constexpr int kAttnMaxGroup = 8;    // q heads per kv head
constexpr int kAttnChunk = 64;      // positions per pass of a workgroup (one per lane in the softmax)
constexpr int kAttnMaxSplits = 128;  // partials per kv head (two per lane in the merge)

// Bias, per-head rmsnorm (QK-norm) and RoPE of one head slice, done by one
// wave; `src` is the raw projection, the result goes to dst (LDS).
__device__ void head_prep(const float* __restrict__ src, const float* __restrict__ bias,
                          const float* __restrict__ nw, const double* __restrict__ cs, float* dst, int hd, float eps,
                          int neox) {
    const int lane = threadIdx.x & 63, half = hd / 2;
    // every global input is requested before any arithmetic
    float v[2] = {0.f, 0.f}, g[2] = {1.f, 1.f};  // hd <= 128: elements lane and lane + 64
    double c = 1.0, s = 0.0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) {
            v[r] = src[t] + (bias ? bias[t] : 0.f);
            if (nw) g[r] = nw[t];
        }
    }
    if (lane < half) {
        c = cs[2 * lane];
        s = cs[2 * lane + 1];
    }
    if (nw) {
        const double ss = wave_sum_d_all((double)v[0] * v[0] + (double)v[1] * v[1]);
        const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
#pragma unroll
        for (int r = 0; r < 2; ++r) v[r] = (float)((double)v[r] * inv) * g[r];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) dst[t] = v[r];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // RoPE (rope.cpp:6-57): pair i = (2i, 2i+1), or (i, i + hd/2) for NeoX;
    // lane i reads and rewrites only pair i
    if (lane < half) {
        const int ia = neox ? lane : 2 * lane, ib = neox ? lane + half : 2 * lane + 1;
        const double x0 = dst[ia], x1 = dst[ib];
        dst[ia] = (float)(x0 * c - x1 * s);
        dst[ib] = (float)(x0 * s + x1 * c);
    }
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

// Decode attention for kv head g over the L = pos+1 positions
// (transformer.cpp:529-629), head_dim = 8 * LPP.
//
// Positions are taken in chunks of 64; workgroup s of the S per kv head takes
// chunks s, s+S, ...  Thread (position group pg, lane sub) holds 8 dims
// (one 16-byte fp16 load) of NP positions of K and of V, so a chunk's cache
// rows are read with every load in flight at once.  Scores are reduced over
// the LPP lanes of a position with DPP; one wave per q head keeps a running
// softmax (max, sum) across chunks, and the exp-weighted V sums stay in
// registers, rescaled per chunk.
//
// The current token's k and v are prepared, appended (fp16) to the cache and
// used from LDS copies for position pos, so no workgroup reads a cache row
// written in this launch: by the workgroup holding chunk pos/64 when the
// context is one chunk (it then writes the normalised output directly), else
// by an extra workgroup per kv head (blockIdx.y == S) whose partial is that
// one position.  Each partial is (max, sum, V sums) per q head; the last
// workgroup to finish merges them.  GM (4 or 8) bounds the q heads per kv head held in registers;
// GM = 4 keeps the kernel near 128 VGPRs, so more workgroups are resident.
template <int LPP, int GM>
// pos, the caches and q|k|v, needed first, also come as leading scalars that
// the command processor preloads into SGPRs (-amdgpu-kernarg-preload-count).
__global__ __launch_bounds__(256) void attention_kernel(const int* ppos, __half* pkc, __half* pvc, const float* pqkv,
                                                        AttnArgs a) {
    a.pos = ppos;
    a.kc = pkc;
    a.vc = pvc;
    a.qkv = pqkv;
    constexpr int HD = LPP * 8, NPG = 256 / LPP, NP = kAttnChunk / NPG;
    __shared__ float qs[kAttnMaxGroup][HD];
    __shared__ float kvt[HD];
    __shared__ __align__(16) __half kvh[2][HD];
    __shared__ float sc[kAttnMaxGroup][kAttnChunk];
    __shared__ float run_m[kAttnMaxGroup], run_l[kAttnMaxGroup], alpha[kAttnMaxGroup];
    __shared__ __align__(16) float red[4][kAttnMaxGroup][HD];
    __shared__ float wgt[kAttnMaxGroup][kAttnMaxSplits];
    __shared__ int last;

    // blockIdx.y < S: chunk splits; blockIdx.y == S: the current-token
    // workgroup (see `sep`)
    const int g = blockIdx.x, s = blockIdx.y, S = gridDim.y - 1;
    const int group = a.nh / a.nkv, kvd = a.nkv * HD, qd = a.nh * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = tid % LPP, pg = tid / LPP;
    const int pos = *a.pos, L = pos + 1;
    // With more than one chunk the partials are merged anyway, and the
    // current token (q, k and v preparation, its k/v append and its own
    // score) goes to a workgroup of its own instead of the chunk holding pos,
    // which would otherwise finish a preparation round after the others.
    // The chunks then cover the cached positions [0, pos) only (every chunk
    // holds at least one of them).
    const bool sep = L > kAttnChunk;
    const int nch = ((sep ? pos : L) + kAttnChunk - 1) / kAttnChunk;
    const int sact = nch < S ? nch : S;        // chunk workgroups with work
    const int nparts = sact + (sep ? 1 : 0);  // partials to merge
    const bool cur = s == S;
    if (cur ? !sep : s >= sact) return;
    const int own_chunk = pos / kAttnChunk;
    const bool owns = cur || (!sep && own_chunk % S == s);
    const int lim = sep ? pos : L;  // chunk positions below lim
    const size_t col = (size_t)g * HD + sub * 8;

    uint4 kraw[NP], vraw[NP];
    // cache rows of this thread's positions in chunk c; positions >= pos are
    // not read (pos itself comes from LDS)
    auto load = [&](uint4* raw, const __half* cache, int c) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int j = c * kAttnChunk + i * NPG + pg;
            raw[i] = j < pos ? *reinterpret_cast<const uint4*>(cache + (size_t)j * kvd + col) : make_uint4(0, 0, 0, 0);
        }
    };
    if (!cur) {
        load(kraw, a.kc, s);
        load(vraw, a.vc, s);
    }

    // q heads (and k, v of the current token) of this kv head
    const double* cs = a.rope_cs + (size_t)pos * HD;  // (hd/2) pairs of (cos, sin)
    const int njobs = group + (owns ? 2 : 0);
    for (int job = wave; job < njobs; job += 4) {
        if (job < group) {
            const int qh = g * group + job;
            head_prep(a.qkv + (size_t)qh * HD, a.bias ? a.bias + (size_t)qh * HD : nullptr, a.q_norm, cs, qs[job], HD,
                      a.eps, a.neox);
            continue;
        }
        const bool is_k = job == group;
        const size_t off = (is_k ? qd : qd + kvd) + (size_t)g * HD;
        if (is_k) {
            head_prep(a.qkv + off, a.bias ? a.bias + off : nullptr, a.k_norm, cs, kvt, HD, a.eps, a.neox);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        }
        // rounded through fp16 like every cached position, and appended
        __half* cache = (is_k ? a.kc : a.vc) + (size_t)pos * kvd + (size_t)g * HD;
        for (int t = lane; t < HD; t += 64) {
            const float v = is_k ? kvt[t] : a.qkv[off + t] + (a.bias ? a.bias[off + t] : 0.f);
            const __half hv = __float2half_rn(v);
            kvh[is_k ? 0 : 1][t] = hv;
            cache[t] = hv;
        }
    }
    if (tid < kAttnMaxGroup) {
        run_m[tid] = -INFINITY;
        run_l[tid] = 0.f;
    }
    __syncthreads();

    float qreg[GM][8], acc[GM][8];
#pragma unroll
    for (int h = 0; h < GM; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qreg[h][e] = h < group ? qs[h][sub * 8 + e] : 0.f;
            acc[h][e] = 0.f;
        }

    // scores in base-2 units (exp(x - m) == exp2(x log2 e - m log2 e)): the
    // running max and the split maxima below are in the same units
    const float scale2 = a.scale * 1.4426950408889634f;
    for (int c = cur ? nch : s; c < nch; c += S) {
        if (!sep && c == own_chunk) {
#pragma unroll
            for (int i = 0; i < NP; ++i)
                if (c * kAttnChunk + i * NPG + pg == pos) {
                    kraw[i] = *reinterpret_cast<const uint4*>(&kvh[0][sub * 8]);
                    vraw[i] = *reinterpret_cast<const uint4*>(&kvh[1][sub * 8]);
                }
        }
        // scores
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int jl = i * NPG + pg, j = c * kAttnChunk + jl;
            float kf[8];
            half8_to_float(kraw[i], kf);
#pragma unroll
            for (int h = 0; h < GM; ++h) {
                if (h >= group) break;
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qreg[h][e], kf[e], d);
                d = lane_group_sum<LPP>(d);
                if (sub == 0) sc[h][jl] = j < lim ? d * scale2 : -INFINITY;
            }
        }
        if (c + S < nch) load(kraw, a.kc, c + S);
        __syncthreads();
        // running softmax per q head (softmax.cpp:4-18, normalised at the end)
        for (int h = wave; h < group; h += 4) {
            const float sv = sc[h][lane];
            const float mo = run_m[h], mn = fmaxf(mo, wave_max_all(sv));
            const float p = __builtin_amdgcn_exp2f(sv - mn), al = __builtin_amdgcn_exp2f(mo - mn);
            const float ps = wave_sum_all(p);
            sc[h][lane] = p;
            if (lane == 0) {
                run_m[h] = mn;
                run_l[h] = run_l[h] * al + ps;
                alpha[h] = al;
            }
        }
        __syncthreads();
        // exp-weighted V
#pragma unroll
        for (int h = 0; h < GM; ++h) {
            if (h >= group) break;
            const float al = alpha[h];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] *= al;
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            float vf[8];
            half8_to_float(vraw[i], vf);
#pragma unroll
            for (int h = 0; h < GM; ++h) {
                if (h >= group) break;
                const float p = sc[h][i * NPG + pg];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
            }
        }
        if (c + S < nch) load(vraw, a.vc, c + S);
        __syncthreads();  // sc and alpha are rewritten by the next chunk
    }

    const int SP = S + 1;                                   // partial slots per q head
    float* part_v = a.part;                                 // [nh][SP][hd]
    float* part_ml = a.part + (size_t)a.nh * SP * HD;       // [nh][SP][2]
    if (cur) {
        // the current token's partial (slot sact): score q_h . k with k and v
        // rounded through fp16 as every cached position, max = that score,
        // sum 1, V sums = v
        for (int h = wave; h < group; h += 4) {
            float d = 0.f;
            for (int t = lane; t < HD; t += 64) d = fmaf(qs[h][t], __half2float(kvh[0][t]), d);
            d = wave_sum_all(d) * scale2;
            const size_t slot = ((size_t)g * group + h) * SP + sact;
            for (int t = lane; t < HD; t += 64) st_agent(part_v + slot * HD + t, __half2float(kvh[1][t]));
            if (lane == 0) {
                st_agent(part_ml + slot * 2, d);
                st_agent(part_ml + slot * 2 + 1, 1.0f);
            }
        }
    } else {
        // sum the V partials of the position groups: lanes of a wave with the
        // same `sub`, then the four waves through LDS
#pragma unroll
        for (int h = 0; h < GM; ++h) {
            if (h >= group) break;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = fold_position_groups<LPP>(acc[h][e]);
            if (lane < LPP) {
                float4* dst = reinterpret_cast<float4*>(&red[wave][h][sub * 8]);
                dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
                dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
            }
        }
        __syncthreads();
        for (int i = tid; i < group * HD; i += 256) {
            const int h = i / HD, t = i % HD;
            const float v = red[0][h][t] + red[1][h][t] + red[2][h][t] + red[3][h][t];
            const size_t qh = (size_t)g * group + h;
            if (nparts == 1) {
                a.att[qh * HD + t] = v / run_l[h];
            } else {
                st_agent(part_v + (qh * SP + s) * HD + t, v);
                if (t == 0) {
                    st_agent(part_ml + (qh * SP + s) * 2, run_m[h]);
                    st_agent(part_ml + (qh * SP + s) * 2 + 1, run_l[h]);
                }
            }
        }
        if (nparts == 1) return;
    }

    // the last workgroup of kv head g to finish merges the partials; they
    // were stored device-coherently and are complete before the count (the
    // hand-off protocol written out at st_agent in mxh_device.h: sc1 stores,
    // a full vmcnt wait, the relaxed add; the add's return value, sc1 loads)
    wait_mem();
    __syncthreads();
    if (tid == 0) last = add_agent(a.counter + g, 1) == nparts - 1;
    __syncthreads();
    if (!last) return;
    // (q head, 4 dims) items; the splits of an item are shared by `per`
    // threads.  The first kPre splits of each thread are requested together
    // with the (max, sum) pairs, so most merges cost one memory round trip.
    constexpr int kPre = 16;
    const int items = group * HD / 4, per = 256 / items;
    const int item = tid % items, part = tid / items;
    const int hi = item / (HD / 4), d4 = item % (HD / 4);
    // byte offsets into the V partials, read as 16-byte agent-coherent loads
    const __amdgpu_buffer_rsrc_t prs = agent_rsrc(part_v, (int)((size_t)a.nh * SP * HD * sizeof(float)));
    const int src = (int)((((size_t)g * group + hi) * SP * HD + 4 * d4) * sizeof(float));
    float4 pre[kPre];
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        const int i = part + per * k;
        pre[k] = part < per && i < nparts ? ld_agent4(prs, src + i * HD * (int)sizeof(float))
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int h = wave; h < group; h += 4) {
        // splits lane and lane + 64
        const float* ml = part_ml + ((size_t)g * group + h) * SP * 2;
        const bool in0 = lane < nparts, in1 = lane + 64 < nparts;
        const float m0 = in0 ? ld_agent(ml + 2 * lane) : -INFINITY;
        const float l0 = in0 ? ld_agent(ml + 2 * lane + 1) : 0.f;
        const float m1 = in1 ? ld_agent(ml + 2 * lane + 128) : -INFINITY;
        const float l1 = in1 ? ld_agent(ml + 2 * lane + 129) : 0.f;
        const float M = wave_max_all(fmaxf(m0, m1));
        const float w0 = in0 ? __builtin_amdgcn_exp2f(m0 - M) : 0.f;
        const float w1 = in1 ? __builtin_amdgcn_exp2f(m1 - M) : 0.f;
        const float den = wave_sum_all(w0 * l0 + w1 * l1);
        wgt[h][lane] = w0 / den;
        wgt[h][lane + 64] = w1 / den;
    }
    __syncthreads();
    float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (part < per) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int i = part + per * k;
            if (i < nparts) {
                const float w = wgt[hi][i];
                s4.x = fmaf(w, pre[k].x, s4.x);
                s4.y = fmaf(w, pre[k].y, s4.y);
                s4.z = fmaf(w, pre[k].z, s4.z);
                s4.w = fmaf(w, pre[k].w, s4.w);
            }
        }
#pragma unroll 8
        for (int i = part + per * kPre; i < nparts; i += per) {
            const float4 v = ld_agent4(prs, src + i * HD * (int)sizeof(float));
            const float w = wgt[hi][i];
            s4.x = fmaf(w, v.x, s4.x);
            s4.y = fmaf(w, v.y, s4.y);
            s4.z = fmaf(w, v.z, s4.z);
            s4.w = fmaf(w, v.w, s4.w);
        }
    }
    float4* r4 = reinterpret_cast<float4*>(&red[0][0][0]);  // 256 float4 fit: 4 * 8 * HD floats >= 1024
    __syncthreads();
    r4[tid] = s4;
    __syncthreads();
    if (tid < items) {
        float4 t4 = r4[tid];
        for (int p = 1; p < per; ++p) {
            const float4 u = r4[p * items + tid];
            t4.x += u.x;
            t4.y += u.y;
            t4.z += u.z;
            t4.w += u.w;
        }
        const int h = tid / (HD / 4), d4 = tid % (HD / 4);
        reinterpret_cast<float4*>(a.att + ((size_t)g * group + h) * HD)[d4] = t4;
    }
    if (tid == 0) st_agent(a.counter + g, 0);
}

// ---- batched prefill ---------------------------------------------------------

// Row-batched head preparation for prompt tokens p0 .. p0+m-1: workgroup
// (z, h) is one wave for q head h, k head h - nh or v head h - nh - nkv of
// token z.  q goes to q_out (fp32), k and v (rounded to fp16) to the cache at
// position p0 + z (transformer.cpp:385-470 per token; QK-norm as head_prep).
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

const void* attention_kernel_for(int nh, int nkv, int hd) {
    const bool g4 = nh / nkv <= 4;
    switch (hd) {
    case 32: return g4 ? (const void*)attention_kernel<4, 4> : (const void*)attention_kernel<4, 8>;
    case 64: return g4 ? (const void*)attention_kernel<8, 4> : (const void*)attention_kernel<8, 8>;
    default: return g4 ? (const void*)attention_kernel<16, 4> : (const void*)attention_kernel<16, 8>;
    }
}

}  // namespace

// Workgroups per kv head: one per 64-position chunk of the context up to 64
// chunks.  Beyond that, enough for at most two chunks each (a workgroup's
// chunks run one after another), as far as all of them stay resident at
// once (more would run in a second round), and at most kAttnMaxSplits.
int attention_splits(int n_ctx, int nh, int nkv, int hd) {
    const int nch = (n_ctx + kAttnChunk - 1) / kAttnChunk;
    if (nch <= 64) return nch < 1 ? 1 : nch;
    int dev = 0, n_cu = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attention_kernel_for(nh, nkv, hd), 256, 0) != hipSuccess)
        n_cu = per_cu = 0;
    const int cap = nkv > 0 ? per_cu * n_cu / nkv - 1 : 0;  // (one current-token workgroup per kv head)
    int S = (nch + 1) / 2;
    if (S > cap) S = cap;
    if (S > kAttnMaxSplits - 1) S = kAttnMaxSplits - 1;  // partials: S chunk splits and the current token
    return S < 64 ? 64 : S;
}

// head_dim 32, 64 or 128 (8 dims per lane, a power-of-two lane count per
// position); at most kAttnMaxGroup q heads per kv head
bool attention_supported(int nh, int nkv, int hd) {
    return nkv > 0 && nh % nkv == 0 && nh / nkv <= kAttnMaxGroup && (hd == 32 || hd == 64 || hd == 128);
}

int attention_run(const AttnArgs& a, int n_ctx, hipStream_t st) {
    if (!attention_supported(a.nh, a.nkv, a.hd)) return MXH_ERR_UNSUPPORTED;
    // chunk splits plus the current-token workgroup
    const dim3 grid(a.nkv, attention_splits(n_ctx, a.nh, a.nkv, a.hd) + 1);
    const bool g4 = a.nh / a.nkv <= 4;
    switch (a.hd) {
    case 32:
        if (g4) hipLaunchKernelGGL((attention_kernel<4, 4>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        else hipLaunchKernelGGL((attention_kernel<4, 8>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        break;
    case 64:
        if (g4) hipLaunchKernelGGL((attention_kernel<8, 4>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        else hipLaunchKernelGGL((attention_kernel<8, 8>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        break;
    default:
        if (g4) hipLaunchKernelGGL((attention_kernel<16, 4>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        else hipLaunchKernelGGL((attention_kernel<16, 8>), grid, dim3(256), 0, st, a.pos, a.kc, a.vc, a.qkv, a);
        break;
    }
    return MXH_OK;
}

// V partials [nh][S + 1][hd] followed by (max, sum) pairs [nh][S + 1][2]
size_t attention_scratch_floats(int nh, int nkv, int hd, int n_ctx) {
    return (size_t)nh * (attention_splits(n_ctx, nh, nkv, hd) + 1) * (hd + 2);
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
