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

// One wave per head.  Heads [0, nh) are q, [nh, nh+nkv) are k, [nh+nkv,
// nh+2nkv) are v, all in the fused qkv buffer [q | k | v].  q and k get
// optional bias, optional per-head rmsnorm (QK-norm), then RoPE at `pos`
// from the double cos/sin table; k and v are written to the fp16 cache.
__global__ void qkv_post_kernel(float* __restrict__ qkv, const float* __restrict__ bias, const float* __restrict__ qn,
                                const float* __restrict__ kn, const double* __restrict__ rope_cs,
                                const int* __restrict__ pos_p, __half* __restrict__ kc, __half* __restrict__ vc,
                                int nh, int nkv, int hd, float eps, int neox, int rope_half) {
    const int head = blockIdx.x;
    const int lane = threadIdx.x;
    const int pos = *pos_p;
    const int kvd = nkv * hd;
    float* v = qkv + (size_t)head * hd;  // head slices are contiguous in [q | k | v]
    const bool is_q = head < nh, is_k = !is_q && head < nh + nkv;
    if (bias)
        for (int t = lane; t < hd; t += 64) v[t] += bias[(size_t)head * hd + t];
    if (is_q || is_k) {
        const float* nw = is_q ? qn : kn;
        if (nw) {
            double ss = 0.0;
            for (int t = lane; t < hd; t += 64) ss += (double)v[t] * (double)v[t];
            ss = wave_sum_d(ss);
            const double inv = 1.0 / sqrt(ss / (double)hd + (double)eps);
            for (int t = lane; t < hd; t += 64) v[t] = (float)((double)v[t] * inv) * nw[t];
        }
        // RoPE: pair i rotates by pos * theta^(-2i/rot), cos/sin from the table
        const double* cs = rope_cs + (size_t)pos * rope_half * 2;
        for (int i = lane; i < rope_half; i += 64) {
            const int a = neox ? i : 2 * i;
            const int b = neox ? i + rope_half : 2 * i + 1;
            const double c = cs[2 * i], s = cs[2 * i + 1];
            const double x0 = v[a], x1 = v[b];
            v[a] = (float)(x0 * c - x1 * s);
            v[b] = (float)(x0 * s + x1 * c);
        }
    }
    if (!is_q) {
        // round through fp16 into the cache; the current token is read back
        // from the cache by attention like every earlier one
        const int kvh = is_k ? head - nh : head - nh - nkv;
        __half* dst = (is_k ? kc : vc) + (size_t)pos * kvd + (size_t)kvh * hd;
        for (int t = lane; t < hd; t += 64) dst[t] = __float2half_rn(v[t]);
    }
}

constexpr int kAttnChunk = 256;   // positions per split
constexpr int kAttnMaxGroup = 8;  // q heads per kv head handled by one workgroup

// Split-K decode attention, partial pass.  Workgroup (kv head g, split s)
// covers positions [s*C, min(L, s*C + C)) for the `group` q heads of g and
// writes, per q head, the running max m, the sum l of exp(score - m) and the
// unnormalised sum of exp(score - m) * V.
__global__ __launch_bounds__(256) void attn_partial_kernel(const float* __restrict__ q, const __half* __restrict__ kc,
                                                           const __half* __restrict__ vc, const int* __restrict__ pos_p,
                                                           float* __restrict__ part, int nh, int nkv, int hd,
                                                           float scale, int max_splits) {
    __shared__ float qs[kAttnMaxGroup * 256];
    __shared__ float sc[kAttnMaxGroup][kAttnChunk];
    __shared__ float accs[2][kAttnMaxGroup][256];
    const int g = blockIdx.x, s = blockIdx.y;
    const int group = nh / nkv;
    const int L = *pos_p + 1;
    const int j0 = s * kAttnChunk;
    const int jn = min(L - j0, kAttnChunk);
    const int kvd = nkv * hd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (jn <= 0) {
        // empty split: neutral partial
        if (tid < group) {
            float* p = part + ((size_t)(g * group + tid) * max_splits + s) * (hd + 2);
            p[0] = -INFINITY;
            p[1] = 0.f;
        }
        return;
    }
    for (int i = tid; i < group * hd; i += 256) qs[i] = q[(size_t)(g * group) * hd + i];
    __syncthreads();
    // scores: one wave per position, lanes split the head dimension
    for (int jj = wave; jj < jn; jj += 4) {
        const __half* kr = kc + (size_t)(j0 + jj) * kvd + (size_t)g * hd;
        float dot[kAttnMaxGroup];
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) dot[h] = 0.f;
        for (int t = lane; t < hd; t += 64) {
            const float kv = __half2float(kr[t]);
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < group) dot[h] = fmaf(qs[h * hd + t], kv, dot[h]);
        }
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < group) {
                const float d = wave_sum(dot[h]);
                if (lane == 0) sc[h][jj] = d * scale;
            }
    }
    __syncthreads();
    // per-head max and exp
    for (int h = wave; h < group; h += 4) {
        float m = -INFINITY;
        for (int jj = lane; jj < jn; jj += 64) m = fmaxf(m, sc[h][jj]);
        m = wave_max(m);
        float l = 0.f;
        for (int jj = lane; jj < jn; jj += 64) {
            const float e = expf(sc[h][jj] - m);
            sc[h][jj] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            float* p = part + ((size_t)(g * group + h) * max_splits + s) * (hd + 2);
            p[0] = m;
            p[1] = l;
        }
    }
    __syncthreads();
    // weighted V: threads [0, hd) take even positions, [hd, 2hd) odd ones
    const int t = tid % hd, half = tid / hd;
    if (half < 2 && tid < 2 * hd) {
        float acc[kAttnMaxGroup];
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) acc[h] = 0.f;
        for (int jj = half; jj < jn; jj += 2) {
            const float vv = __half2float(vc[(size_t)(j0 + jj) * kvd + (size_t)g * hd + t]);
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < group) acc[h] = fmaf(sc[h][jj], vv, acc[h]);
        }
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < group) accs[half][h][t] = acc[h];
    }
    __syncthreads();
    for (int i = tid; i < group * hd; i += 256) {
        const int h = i / hd, tt = i % hd;
        float* p = part + ((size_t)(g * group + h) * max_splits + s) * (hd + 2);
        p[2 + tt] = accs[0][h][tt] + (2 * hd <= 256 ? accs[1][h][tt] : 0.f);
    }
}

// Merge the splits of one q head: out = sum_s e^(m_s-M) acc_s / sum_s e^(m_s-M) l_s.
__global__ void attn_combine_kernel(const float* __restrict__ part, const int* __restrict__ pos_p,
                                    float* __restrict__ out, int hd, int max_splits) {
    const int h = blockIdx.x;
    const int L = *pos_p + 1;
    const int ns = (L + kAttnChunk - 1) / kAttnChunk;
    const float* p = part + (size_t)h * max_splits * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, p[(size_t)s * (hd + 2)]);
    float den = 0.f;
    for (int s = 0; s < ns; ++s) den += expf(p[(size_t)s * (hd + 2)] - M) * p[(size_t)s * (hd + 2) + 1];
    for (int t = threadIdx.x; t < hd; t += blockDim.x) {
        float num = 0.f;
        for (int s = 0; s < ns; ++s) num += expf(p[(size_t)s * (hd + 2)] - M) * p[(size_t)s * (hd + 2) + 2 + t];
        out[(size_t)h * hd + t] = num / den;
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
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, y, n, eps);
    return MXH_OK;
}

int qkv_post_launch(float* qkv, const float* bias, const float* qn, const float* kn, const double* rope_cs,
                    const int* pos, __half* kc, __half* vc, int nh, int nkv, int hd, float eps, int neox,
                    int rope_half, hipStream_t st) {
    hipLaunchKernelGGL(qkv_post_kernel, dim3(nh + 2 * nkv), dim3(64), 0, st, qkv, bias, qn, kn, rope_cs, pos, kc, vc,
                       nh, nkv, hd, eps, neox, rope_half);
    return MXH_OK;
}

int attention_launch(const float* q, const __half* kc, const __half* vc, const int* pos, float* part, float* out,
                     int nh, int nkv, int hd, int n_ctx, hipStream_t st) {
    if (nh % nkv || nh / nkv > kAttnMaxGroup || hd > 128 || hd % 2) return MXH_ERR_UNSUPPORTED;
    const int max_splits = (n_ctx + kAttnChunk - 1) / kAttnChunk;
    const float scale = 1.0f / sqrtf((float)hd);
    hipLaunchKernelGGL(attn_partial_kernel, dim3(nkv, max_splits), dim3(256), 0, st, q, kc, vc, pos, part, nh, nkv, hd,
                       scale, max_splits);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(nh), dim3(128), 0, st, part, pos, out, hd, max_splits);
    return MXH_OK;
}

size_t attention_scratch_floats(int nh, int hd, int n_ctx) {
    return (size_t)nh * ((n_ctx + kAttnChunk - 1) / kAttnChunk) * (hd + 2);
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
