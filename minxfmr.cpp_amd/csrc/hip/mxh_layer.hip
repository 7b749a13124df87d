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
constexpr int kAttnMaxPos = 1024;   // positions one workgroup may cover
constexpr int kAttnMaxSplits = 64;  // splits per kv head (one lane each in the merge)

// Bias, per-head rmsnorm (QK-norm) and RoPE of one head slice, done by one
// wave; `src` is the raw projection, the result goes to dst (LDS).
__device__ void head_prep(const float* __restrict__ src, const float* __restrict__ bias,
                          const float* __restrict__ nw, const double* __restrict__ cs, float* dst, int hd, float eps,
                          int neox) {
    const int lane = threadIdx.x & 63;
    float v[2] = {0.f, 0.f};  // hd <= 128: elements lane and lane + 64
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) v[r] = src[t] + (bias ? bias[t] : 0.f);
    }
    if (nw) {
        const double ss = wave_sum_d_all((double)v[0] * v[0] + (double)v[1] * v[1]);
        const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int t = lane + 64 * r;
            if (t < hd) v[r] = (float)((double)v[r] * inv) * nw[t];
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int t = lane + 64 * r;
        if (t < hd) dst[t] = v[r];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // RoPE (rope.cpp:6-57): pair i = (2i, 2i+1), or (i, i + hd/2) for NeoX;
    // each lane reads and rewrites only its own pair
    const int half = hd / 2, i = lane;
    if (i < half) {
        const int ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
        const double c = cs[2 * i], s = cs[2 * i + 1];
        const double x0 = dst[ia], x1 = dst[ib];
        dst[ia] = (float)(x0 * c - x1 * s);
        dst[ib] = (float)(x0 * s + x1 * c);
    }
}

// sum over aligned groups of `lpp` lanes (a power of two <= 16); every lane of
// the group ends with the group sum
__device__ __forceinline__ float lane_group_sum(float v, int lpp) {
    if (lpp >= 2) v += dpp_f<0xb1>(v);
    if (lpp >= 4) v += dpp_f<0x4e>(v);
    if (lpp >= 8) v += dpp_f<0x141>(v);
    if (lpp >= 16) v += dpp_f<0x140>(v);
    return v;
}

// Decode attention for kv head g and split s of the L = pos+1 positions
// (transformer.cpp:529-629).  The group's q heads are normed and rotated in
// LDS.  The split holding position pos also prepares k and v of the current
// token: it appends them (fp16) to the cache and uses its own fp16-rounded
// copies for position pos, so no workgroup reads a cache row written in the
// same launch.  With one split the normalised output goes straight to att;
// with several, each split writes (max, sum of exp, exp-weighted V) per q
// head and the last split to finish merges them in split order.
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
    __shared__ float qs[kAttnMaxGroup * 128];
    __shared__ float sc[kAttnMaxGroup][kAttnMaxPos];
    __shared__ float kvt[2][128];
    __shared__ float vacc[4][kAttnMaxGroup][128];
    __shared__ float ml[kAttnMaxGroup][2];
    __shared__ int last;
    const int g = blockIdx.x, s = blockIdx.y, S = gridDim.y;
    const int hd = a.hd, group = a.nh / a.nkv, kvd = a.nkv * hd, qd = a.nh * hd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = *a.pos, L = pos + 1;
    const int j0 = (int)(((long long)s * L) / S), j1 = (int)(((long long)(s + 1) * L) / S);
    const int nj = j1 - j0;
    const bool owns = nj > 0 && j1 == L;
    const int ncache = owns ? nj - 1 : nj;  // positions read from the cache
    const double* cs = a.rope_cs + (size_t)pos * hd;  // (hd/2) pairs of (cos, sin)

    if (nj > 0) {
        for (int h = wave; h < group; h += 4) {
            const int qh = g * group + h;
            head_prep(a.qkv + (size_t)qh * hd, a.bias ? a.bias + (size_t)qh * hd : nullptr, a.q_norm, cs,
                      qs + h * hd, hd, a.eps, a.neox);
        }
        if (owns && wave >= 2) {
            // k (wave 3) or v (wave 2) of the current token, rounded through
            // fp16 like every cached position, appended to the cache
            float* dst = kvt[wave - 2];
            const size_t off = (wave == 3 ? qd : qd + kvd) + (size_t)g * hd;
            if (wave == 3) {
                head_prep(a.qkv + off, a.bias ? a.bias + off : nullptr, a.k_norm, cs, dst, hd, a.eps, a.neox);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            }
            __half* cache = (wave == 3 ? a.kc : a.vc) + (size_t)pos * kvd + (size_t)g * hd;
            for (int t = lane; t < hd; t += 64) {
                const float v = wave == 3 ? dst[t] : a.qkv[off + t] + (a.bias ? a.bias[off + t] : 0.f);
                const __half hv = __float2half_rn(v);
                dst[t] = __half2float(hv);
                cache[t] = hv;
            }
        }
        __syncthreads();
        // scores of cached positions: lpp lanes per position, 8 dims (one
        // 16-byte load of fp16 K) per lane
        const int lpp = hd / 8, ppw = 64 / lpp;
        const int sub = lane % lpp, slot = lane / lpp;
        float qreg[kAttnMaxGroup][8];
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) qreg[h][e] = h < group ? qs[h * hd + sub * 8 + e] : 0.f;
        const __half* kbase = a.kc + (size_t)j0 * kvd + (size_t)g * hd + sub * 8;
        for (int jb = wave * ppw; jb < ncache; jb += 8 * ppw) {
            // two positions per lane per iteration: both loads in flight together
            float dot[2][kAttnMaxGroup];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int jj = jb + u * 4 * ppw + slot;
                uint4 raw = make_uint4(0, 0, 0, 0);
                if (jj < ncache) raw = *reinterpret_cast<const uint4*>(kbase + (size_t)jj * kvd);
                const __half2* hv = reinterpret_cast<const __half2*>(&raw);
                float kf[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float2 f = __half22float2(hv[e]);
                    kf[2 * e] = f.x;
                    kf[2 * e + 1] = f.y;
                }
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h) {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf(qreg[h][e], kf[e], d);
                    dot[u][h] = d;
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int jj = jb + u * 4 * ppw + slot;
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h) {
                    if (h >= group) break;
                    const float d = lane_group_sum(dot[u][h], lpp);
                    if (sub == 0 && jj < ncache) sc[h][jj] = d * a.scale;
                }
            }
        }
        if (owns && wave == 0) {
            for (int h = 0; h < group; ++h) {
                float d = 0.f;
                for (int t = lane; t < hd; t += 64) d = fmaf(qs[h * hd + t], kvt[0][t], d);
                d = wave_sum_all(d);
                if (lane == 0) sc[h][nj - 1] = d * a.scale;
            }
        }
        __syncthreads();
        // per-head max and exp (softmax.cpp:4-18 up to the final division)
        for (int h = wave; h < group; h += 4) {
            float m = -INFINITY;
            for (int jj = lane; jj < nj; jj += 64) m = fmaxf(m, sc[h][jj]);
            m = wave_max_all(m);
            float l = 0.f;
            for (int jj = lane; jj < nj; jj += 64) {
                const float e = expf(sc[h][jj] - m);
                sc[h][jj] = e;
                l += e;
            }
            l = wave_sum_all(l);
            if (lane == 0) {
                ml[h][0] = m;
                ml[h][1] = l;
            }
        }
        __syncthreads();
        // exp-weighted V: thread = (dim pair, one of four position phases)
        const int npair = hd / 2, phase = tid / npair, t2 = tid % npair;
        if (phase < 4) {
            float acc[kAttnMaxGroup][2];
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h) acc[h][0] = acc[h][1] = 0.f;
            const __half* vbase = a.vc + (size_t)j0 * kvd + (size_t)g * hd + 2 * t2;
            for (int jj = phase; jj < ncache; jj += 8) {
                const float2 v0 = __half22float2(*reinterpret_cast<const __half2*>(vbase + (size_t)jj * kvd));
                float2 v1 = make_float2(0.f, 0.f);
                const bool two = jj + 4 < ncache;
                if (two) v1 = __half22float2(*reinterpret_cast<const __half2*>(vbase + (size_t)(jj + 4) * kvd));
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h) {
                    if (h >= group) break;
                    const float p0 = sc[h][jj], p1 = two ? sc[h][jj + 4] : 0.f;
                    acc[h][0] = fmaf(p1, v1.x, fmaf(p0, v0.x, acc[h][0]));
                    acc[h][1] = fmaf(p1, v1.y, fmaf(p0, v0.y, acc[h][1]));
                }
            }
            if (owns && phase == 0) {
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h) {
                    if (h >= group) break;
                    const float p = sc[h][nj - 1];
                    acc[h][0] = fmaf(p, kvt[1][2 * t2], acc[h][0]);
                    acc[h][1] = fmaf(p, kvt[1][2 * t2 + 1], acc[h][1]);
                }
            }
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h) {
                if (h >= group) break;
                vacc[phase][h][2 * t2] = acc[h][0];
                vacc[phase][h][2 * t2 + 1] = acc[h][1];
            }
        }
        __syncthreads();
        const int nphase = min(4, 256 / npair);
        for (int i = tid; i < group * hd; i += 256) {
            const int h = i / hd, t = i % hd;
            float v = 0.f;
            for (int ph = 0; ph < nphase; ++ph) v += vacc[ph][h][t];
            if (S == 1) {
                a.att[(size_t)(g * group + h) * hd + t] = v / ml[h][1];
            } else {
                float* p = a.part + ((size_t)(g * group + h) * S + s) * (hd + 2);
                p[2 + t] = v;
                if (t == 0) {
                    p[0] = ml[h][0];
                    p[1] = ml[h][1];
                }
            }
        }
    } else {
        for (int i = tid; i < group * (hd + 2); i += 256) {
            const int h = i / (hd + 2), t = i % (hd + 2);
            a.part[((size_t)(g * group + h) * S + s) * (hd + 2) + t] = t == 0 ? -INFINITY : 0.f;
        }
    }
    if (S == 1) return;
    // the last split of kv head g to finish merges the partials
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(a.counter + g, 1) == S - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    // lane i holds split i's (max, sum); weights e^(m_i - M) go through LDS
    for (int h = wave; h < group; h += 4) {
        const float* p = a.part + (size_t)(g * group + h) * S * (hd + 2);
        const float mi = lane < S ? __builtin_nontemporal_load(p + (size_t)lane * (hd + 2)) : -INFINITY;
        const float li = lane < S ? __builtin_nontemporal_load(p + (size_t)lane * (hd + 2) + 1) : 0.f;
        const float M = wave_max_all(mi);
        const float wi = lane < S ? expf(mi - M) : 0.f;
        const float den = wave_sum_all(wi * li);
        sc[h][lane] = wi;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        for (int t = lane; t < hd; t += 64) {
            float num = 0.f;
#pragma unroll 8
            for (int i = 0; i < S; ++i)
                num = fmaf(sc[h][i], __builtin_nontemporal_load(p + (size_t)i * (hd + 2) + 2 + t), num);
            a.att[(size_t)(g * group + h) * hd + t] = num / den;
        }
    }
    if (tid == 0) a.counter[g] = 0;
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

// Splits per kv head: one (no merge pass) up to 256 positions, then about
// 256 positions per split up to kAttnMaxSplits splits, and beyond that as
// many as the LDS score buffer (kAttnMaxPos per split) needs.
int attention_splits(int n_ctx) {
    int S = (n_ctx + 255) / 256;
    S = S < 1 ? 1 : (S > kAttnMaxSplits ? kAttnMaxSplits : S);
    while ((n_ctx + S - 1) / S > kAttnMaxPos) ++S;
    return S;
}

int attention_run(const AttnArgs& a, int n_ctx, hipStream_t st) {
    // head_dim: a multiple of 8 with hd/8 a power of two (lanes per position)
    const int lpp = a.hd / 8;
    if (a.nh % a.nkv || a.nh / a.nkv > kAttnMaxGroup || a.hd > 128 || a.hd % 8 || a.hd < 16 || (lpp & (lpp - 1)))
        return MXH_ERR_UNSUPPORTED;
    const int S = attention_splits(n_ctx);
    if (S > kAttnMaxSplits) return MXH_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(attention_kernel, dim3(a.nkv, S), dim3(256), 0, st, a);
    return MXH_OK;
}

size_t attention_scratch_floats(int nh, int hd, int n_ctx) {
    return (size_t)nh * attention_splits(n_ctx) * (hd + 2);
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
