// mxh_sample.hip — top-k / temperature / top-p / min-p sampling on the device
// (reference: src/api/minxfmr.cpp:2091-2171, with a seeded draw).
//
// top_k up to 64, two passes.  Pass 1: each of W workgroups sorts its slice of the logits in LDS (bitonic,
// 64-bit keys: order-preserving bits of the logit above the complemented id,
// so ties go to the lower id, as the reference's partial_sort with `>` and an
// increasing initial order) and keeps its best kk = pow2(top_k) candidates.
// Pass 2: one workgroup sorts the lists of the top_k groups with the largest
// maxima (they hold every candidate that can rank in the top k), then thread
// 0 forms the probabilities in double exactly as the reference does (exp of
// (l - max) / T, normalise, top-p cut and renormalise, min-p cut and
// renormalise) and draws.  top_k from 65 to 4096: one workgroup selects the
// k best keys by a radix select, sorts them and chooses the same way.  The
// uniform of draw d is splitmix64 at state
// seed + (d + 1) * 0x9E3779B97F4A7C15, the d-th value of the sequence that
// starts at `seed`.
#include <hip/hip_runtime.h>

#include "mxh_device.h"
#include "mxh_internal.h"

namespace mxh {

namespace {

constexpr int kSortMax = 4096;  // keys one workgroup sorts in LDS
constexpr int kTopKMax = 64;      // the two-pass form
constexpr int kTopKLarge = kSampleTopKMax;  // the one-workgroup radix-select form
constexpr int kMaxGroups = 2048;  // pass-1 lists one pass-2 workgroup ranks

__device__ __forceinline__ uint64_t sort_key(float v, int idx) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) u = 0u;  // NaN sorts last
    else u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(~(uint32_t)idx);
}

__device__ __forceinline__ int key_id(uint64_t k) { return (int)(~(uint32_t)(k & 0xffffffffu)); }

// descending bitonic sort of s[0 .. p), p a power of two
__device__ void bitonic_desc(uint64_t* s, int p) {
    for (int k = 2; k <= p; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < p; i += blockDim.x) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = s[i], b = s[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) {
                        s[i] = b;
                        s[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
}

__device__ __forceinline__ int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

__global__ __launch_bounds__(1024) void topk_pass1_kernel(const float* __restrict__ logits, int n, int slice, int kk,
                                                          uint64_t* __restrict__ cand) {
    __shared__ uint64_t s[kSortMax];
    const int b0 = blockIdx.x * slice, b1 = min(n, b0 + slice);
    const int p = pow2_at_least(slice > kk ? slice : kk);  // short slices pad up to the list length
    for (int i = threadIdx.x; i < p; i += blockDim.x) {
        const int idx = b0 + i;
        s[i] = idx < b1 ? sort_key(logits[idx], idx) : 0ull;
    }
    __syncthreads();
    bitonic_desc(s, p);
    for (int i = threadIdx.x; i < kk; i += blockDim.x) cand[(size_t)blockIdx.x * kk + i] = s[i];
}

__device__ __forceinline__ double draw_uniform(uint64_t seed, uint64_t d) {
    uint64_t z = seed + (d + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// The choice among the k best ids in order (ids[0 .. k)), as the reference
// makes it (minxfmr.cpp:2104-2171): the k unnormalised probabilities
// exp((l - max) / T) in double, computed by the workgroup into pr, then in
// thread 0, in the reference's order: normalise, top-p cut and renormalise,
// min-p cut and renormalise, and the draw.  The token goes to out[0] or,
// with tokens/pos, to tokens[*pos + 1] with the position advanced (the
// decode loop on the device); the draw counter advances either way.
// Called by every thread of the workgroup.
__device__ void choose(const float* __restrict__ logits, const int* ids, int k, double* pr, SampleParams* prm,
                       int* out, int* tokens, int* pos) {
    const double temperature = prm->temperature;
    if (temperature > 0.0) {
        const double mx = logits[ids[0]];
        for (int i = threadIdx.x; i < k; i += blockDim.x) pr[i] = exp(((double)logits[ids[i]] - mx) / temperature);
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    double top_p = prm->top_p, min_p = prm->min_p;
    int pick = ids[0];
    if (temperature > 0.0) {
        if (top_p <= 0.0 || top_p > 1.0) top_p = 1.0;
        if (min_p < 0.0) min_p = 0.0;
        if (min_p > 1.0) min_p = 1.0;
        double sum = 0.0;
        for (int i = 0; i < k; ++i) sum += pr[i];
        if (sum > 0.0) {
            for (int i = 0; i < k; ++i) pr[i] /= sum;
            int m = k;
            if (top_p < 1.0) {
                double cum = 0.0;
                m = 0;
                for (int i = 0; i < k; ++i) {
                    cum += pr[i];
                    m = i + 1;
                    if (cum >= top_p) break;
                }
                double r = 0.0;
                for (int i = 0; i < m; ++i) r += pr[i];
                if (r > 0.0)
                    for (int i = 0; i < m; ++i) pr[i] /= r;
            }
            if (min_p > 0.0 && m > 1) {
                const double thr = pr[0] * min_p;
                int keep = 1;
                for (int i = 1; i < m; ++i) {
                    if (pr[i] >= thr) keep = i + 1;
                    else break;
                }
                m = keep;
                double r = 0.0;
                for (int i = 0; i < m; ++i) r += pr[i];
                if (r > 0.0)
                    for (int i = 0; i < m; ++i) pr[i] /= r;
            }
            double total = 0.0;
            for (int i = 0; i < m; ++i) total += pr[i];
            const double u = draw_uniform(prm->seed, prm->draws) * total;
            double cum = 0.0;
            pick = ids[m - 1];
            for (int i = 0; i < m; ++i) {
                cum += pr[i];
                if (u < cum) {
                    pick = ids[i];
                    break;
                }
            }
        }
        prm->draws += 1;
    }
    if (out) out[0] = pick;
    if (tokens) {
        const int q = *pos;
        tokens[q + 1] = pick;
        *pos = q + 1;
    }
}

// Pass 2 (top_k <= kTopKMax): candidates -> token.
//
// Each group's list is sorted, so its first key is the group's maximum.  The
// k-th largest group maximum T bounds the k-th largest key from below (k
// group maxima reach it), and only the k groups whose maximum reaches T can
// hold keys >= T: their lists are the only ones sorted.  Keys are distinct
// (they carry the id), so the order is the full sort's.
__global__ __launch_bounds__(1024) void topk_pass2_kernel(const float* __restrict__ logits, const uint64_t* cand,
                                                          int groups, int kk, SampleParams* prm, int* out,
                                                          int* tokens, int* pos) {
    __shared__ uint64_t s[kSortMax];
    __shared__ uint64_t gmax[kMaxGroups];
    __shared__ double pr[kTopKMax];
    __shared__ int ids[kTopKMax];
    const int k = prm->top_k;
    for (int j = threadIdx.x; j < groups; j += blockDim.x) gmax[j] = cand[(size_t)j * kk];
    __syncthreads();
    const int sel = groups < k ? groups : k;  // groups taken
    for (int j = threadIdx.x; j < groups; j += blockDim.x) {
        const uint64_t v = gmax[j];
        int rank = 0;
        for (int i = 0; i < groups; ++i) rank += gmax[i] > v;
        if (rank < sel)
            for (int i = 0; i < kk; ++i) s[rank * kk + i] = cand[(size_t)j * kk + i];
    }
    const int p = pow2_at_least(sel * kk);
    for (int i = sel * kk + threadIdx.x; i < p; i += blockDim.x) s[i] = 0ull;
    __syncthreads();
    bitonic_desc(s, p);
    for (int i = threadIdx.x; i < k; i += blockDim.x) ids[i] = key_id(s[i]);
    __syncthreads();
    choose(logits, ids, k, pr, prm, out, tokens, pos);
}

// top_k in (kTopKMax, kTopKLarge]: one workgroup finds the k-th largest key T
// by a radix select over the 64-bit keys (8-bit digits, most significant
// first: per digit a histogram of the keys that share the digits chosen so
// far, then the digit whose bin holds the k-th), gathers the k keys >= T
// (exactly k: keys are distinct), sorts them and chooses as pass 2 does.
// Same keys, same order, same choice as the two-pass form.
__global__ __launch_bounds__(1024) void topk_large_kernel(const float* __restrict__ logits, int n, SampleParams* prm,
                                                          int* out, int* tokens, int* pos) {
    __shared__ uint64_t s[kTopKLarge];  // the k keys, then their probabilities (doubles)
    __shared__ int ids[kTopKLarge];
    __shared__ unsigned hist[256];
    __shared__ uint64_t prefix_s;
    __shared__ int need_s, count_s;
    const int k = prm->top_k;
    uint64_t prefix = 0;
    int need = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int b = threadIdx.x; b < 256; b += blockDim.x) hist[b] = 0u;
        __syncthreads();
        const uint64_t hi_mask = shift == 56 ? 0ull : ~0ull << (shift + 8);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const uint64_t key = sort_key(logits[i], i);
            if ((key & hi_mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int above = 0, b = 255;
            for (; b > 0; --b) {
                if (above + (int)hist[b] >= need) break;
                above += (int)hist[b];
            }
            prefix_s = prefix | ((uint64_t)b << shift);
            need_s = need - above;
            count_s = 0;
        }
        __syncthreads();
        prefix = prefix_s;
        need = need_s;
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t key = sort_key(logits[i], i);
        if (key >= prefix) s[atomicAdd(&count_s, 1)] = key;
    }
    const int p = pow2_at_least(k);
    __syncthreads();
    for (int i = k + threadIdx.x; i < p; i += blockDim.x) s[i] = 0ull;
    __syncthreads();
    bitonic_desc(s, p);
    for (int i = threadIdx.x; i < k; i += blockDim.x) ids[i] = key_id(s[i]);
    __syncthreads();
    choose(logits, ids, k, reinterpret_cast<double*>(s), prm, out, tokens, pos);
}

}  // namespace

// Pass-1 workgroups and the per-workgroup list length for n logits and
// top_k: the candidates of all workgroups must fit one LDS sort.
void sample_shape(int n, int top_k, int* groups, int* slice, int* kk) {
    int k2 = 1;
    while (k2 < top_k) k2 <<= 1;
    int w = kSortMax / k2;
    if (w > 256) w = 256;
    int sl = (n + w - 1) / w;
    while (sl > kSortMax) {  // very large vocabularies: fewer, larger lists are not possible
        w *= 2;
        sl = (n + w - 1) / w;
    }
    *groups = (n + sl - 1) / sl;
    *slice = sl;
    *kk = k2;
}

size_t sample_scratch_keys(int n, int top_k) {
    if (top_k > kTopKMax) return 1;  // the radix-select form needs no candidate lists
    int g, sl, kk;
    sample_shape(n, top_k, &g, &sl, &kk);
    return (size_t)g * kk;
}

int sample_launch(const float* logits, int n, SampleParams* prm, int top_k, uint64_t* cand, int* out, int* tokens,
                  int* pos, hipStream_t st) {
    if (n <= 0 || top_k < 1 || top_k > kTopKLarge || top_k > n) return MXH_ERR_ARG;
    if (top_k > kTopKMax) {
        hipLaunchKernelGGL(topk_large_kernel, dim3(1), dim3(1024), 0, st, logits, n, prm, out, tokens, pos);
        return MXH_OK;
    }
    int g, sl, kk;
    sample_shape(n, top_k, &g, &sl, &kk);
    if ((size_t)g * kk > (size_t)kSortMax || g > kMaxGroups) return MXH_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(topk_pass1_kernel, dim3(g), dim3(1024), 0, st, logits, n, sl, kk, cand);
    hipLaunchKernelGGL(topk_pass2_kernel, dim3(1), dim3(1024), 0, st, logits, cand, g, kk, prm, out, tokens, pos);
    return MXH_OK;
}

// ---- logit edits before the choice (minxfmr.cpp:2047-2089) ---------------

namespace {

__device__ __forceinline__ bool edits_active(const EditParams* prm) {
    return prm->repeat_penalty != 1.0 || prm->frequency_penalty != 0.0 || prm->presence_penalty != 0.0;
}

// the penalty window: the last last_n ids of tokens[0 .. pos] (all when
// last_n < 0), as [*h0, *h1)
__device__ __forceinline__ void edit_window(const EditParams* prm, int pos, int* h0, int* h1) {
    const int len = pos + 1;
    int n = prm->last_n < 0 ? len : prm->last_n;
    if (n > len) n = len;
    *h0 = len - n;
    *h1 = len;
}

// suppressed ids to -inf; occurrences of each id in the window counted
__global__ void logit_count_kernel(float* __restrict__ logits, int n_vocab, const int* __restrict__ tokens,
                                   const int* __restrict__ pos_p, const EditParams* __restrict__ prm,
                                   const int* __restrict__ suppress, int* __restrict__ cnt) {
    const int tid = blockIdx.x * blockDim.x + threadIdx.x, nthr = gridDim.x * blockDim.x;
    for (int j = tid; j < prm->n_suppress; j += nthr) {
        const int id = suppress[j];
        if (id >= 0 && id < n_vocab) logits[id] = -INFINITY;
    }
    if (!edits_active(prm)) return;
    int h0, h1;
    edit_window(prm, *pos_p, &h0, &h1);
    for (int i = h0 + tid; i < h1; i += nthr) {
        const int t = tokens[i];
        if (t >= 0 && t < n_vocab) atomicAdd(cnt + t, 1);
    }
}

// each distinct id of the window (the one occurrence whose exchange returns
// its count) gets the reference's penalty, computed in double; the counts go
// back to zero for the next step
__global__ void logit_penalty_kernel(float* __restrict__ logits, int n_vocab, const int* __restrict__ tokens,
                                     const int* __restrict__ pos_p, const EditParams* __restrict__ prm,
                                     int* __restrict__ cnt) {
    if (!edits_active(prm)) return;
    const int tid = blockIdx.x * blockDim.x + threadIdx.x, nthr = gridDim.x * blockDim.x;
    int h0, h1;
    edit_window(prm, *pos_p, &h0, &h1);
    for (int i = h0 + tid; i < h1; i += nthr) {
        const int t = tokens[i];
        if (t < 0 || t >= n_vocab) continue;
        const int c = atomicExch(cnt + t, 0);
        if (c <= 0) continue;
        double l = (double)logits[t];
        if (prm->repeat_penalty != 1.0) l = l <= 0.0 ? l * prm->repeat_penalty : l / prm->repeat_penalty;
        l -= (double)c * prm->frequency_penalty + prm->presence_penalty;
        logits[t] = (float)l;
    }
}

}  // namespace

int logit_edits_launch(float* logits, int n_vocab, const int* tokens, const int* pos, const EditParams* prm,
                       const int* suppress, int* cnt, hipStream_t st) {
    if (n_vocab <= 0) return MXH_ERR_ARG;
    hipLaunchKernelGGL(logit_count_kernel, dim3(64), dim3(256), 0, st, logits, n_vocab, tokens, pos, prm, suppress,
                       cnt);
    hipLaunchKernelGGL(logit_penalty_kernel, dim3(64), dim3(256), 0, st, logits, n_vocab, tokens, pos, prm, cnt);
    return MXH_OK;
}

}  // namespace mxh
