// mxh_internal.h — launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxh_types.h"

namespace mxh {

// Record a failure message for mxh_last_error(); returns `code`.
int set_error(int code, const char* fmt, ...);
// Check a HIP status; on failure record "<what>: <hip error>" and return MXH_ERR_HIP.
int check_hip(hipError_t e, const char* what);

hipStream_t lib_stream();

int gemv_launch(int type, const void* w, const float* x, float* y, const float* res, int64_t n, int64_t k, int form,
                hipStream_t st);

// Fused GEMV launch (see mxh_gemv.hip for the epilogues).
enum { GEMV_PLAIN = 0, GEMV_SILU = 1, GEMV_ARGMAX = 2, GEMV_ATTN = 3 };
struct GemvArgs {
    const uint8_t* w;
    const float* x;
    float* y;
    const float* res;     // residual added to y (PLAIN); may alias y
    const float* norm_w;  // when set, x is rmsnorm(x) * norm_w
    float eps;
    int n, k, form;
    // ARGMAX: per-workgroup winners (red_cap slots), token array and device
    // position
    float* red_val;
    int* red_idx;
    int red_cap;
    int* tokens;
    int* pos;
    // ATTN: x is the decode attention's output, merged here from its split
    // partials (attention_run): V sums [k / part_hd][part_splits][part_hd],
    // then (max in base-2 units, sum) pairs [k / part_hd][part_splits][2];
    // y = W.x (+ res) as in PLAIN
    const float* part;
    int part_splits, part_hd;
};
int gemv_run(int type, const GemvArgs& a, int mode, hipStream_t st);
// Whether the GEMV of this (storage) type stages x as 24-bit block fixed
// point (every quantized type); F32 and F16 rows multiply fp32 x.  Only those
// GEMVs take the attention merge in their staging (GEMV_ATTN).
inline bool gemv_int_x(int type) {
    const int t = type & 0xff;
    return t != MXH_F32 && t != MXH_F16;
}

// Tiled device layout for a weight of this type and row length (the type
// itself when there is none), and the in-place regrouping of `rows` rows at w
// (16-byte aligned) into it.
int tiled_type(int type, int64_t cols);
int tile_rows_launch(int type, void* w, int64_t rows, int64_t cols, hipStream_t st);
int dequant_launch(int type, const void* w, float* out, int64_t rows, int64_t cols, int form, hipStream_t st);

// small F32 vector ops (attention over host caches, F32 weights)
int vec_dot_rows_launch(const float* vec, const float* rows, float* out, int64_t K, int64_t nrows, int64_t stride,
                        int64_t head, int64_t seq_max, hipStream_t st);
int vec_mul_rows_cols_launch(const float* vec, const float* rows, float* out, int64_t nrows, int64_t ncols,
                             int64_t stride, hipStream_t st);
int matmul_f32_launch(const float* a, const float* b, float* out, int64_t m, int64_t k, int64_t n, hipStream_t st);

// decoder-step kernels (mxh_layer.hip)
int rmsnorm_launch(const float* x, const float* w, float* y, int n, float eps, hipStream_t st);
// Fused decode attention: QK-norm, RoPE, fp16 KV append and split-K
// softmax*V (mxh_layer.hip); the splits' partials are merged by the
// o-projection GEMV (GEMV_ATTN).
constexpr int kAttnMaxSplits = 8;  // workgroups (partials) per kv head
struct AttnArgs {
    const float* qkv;     // [q | k | v] raw projections of the current token
    const float* bias;    // [bq | bk | bv] or null
    const float* q_norm;  // per-head rmsnorm weights or null
    const float* k_norm;
    const double* rope_cs;  // [n_ctx + 1][hd/2][cos, sin]
    const int* pos;       // current position (device): tokens run so far
    __half* kc;           // this layer's K cache (see ring)
    __half* vc;
    float* part;          // split partials (attention_scratch_floats)
    int nh, nkv, hd, neox;
    float eps, scale;
    // ring > 0: the cache is the reference's ring of `ring` rows
    // (kv_cache.cpp:50-75) held as ring + 1 slots stored twice,
    // [2 (ring + 1)][nkv*hd]: token p goes to slot p % (ring + 1), and from
    // p = ring on also to that slot's copy ring + 1 rows on, so the rows a
    // step attends are always contiguous (a window [o, o + ring] reads the
    // second copy only of slots below o, all written after the ring filled).
    // Past a full ring RoPE stays at position ring (transformer.cpp:506).
    // ring == 0: the kernels without the ring's arithmetic, for steps below
    // a full cache (the same cache rows: token p at row p).
    int ring;
};
int attention_run(const AttnArgs& a, int n_ctx, hipStream_t st);
// the attention output [nh][hd] merged from `splits` partials (for
// o-projections that do not merge them in their staging)
int attention_merge_launch(const float* part, int splits, int nh, int hd, float* att, hipStream_t st);
int attention_splits(int n_ctx, int nh, int nkv, int hd);
bool attention_supported(int nh, int nkv, int hd);
size_t attention_scratch_floats(int nh, int nkv, int hd, int n_ctx);
int silu_mul_launch(const float* gu, float* h, int n, hipStream_t st);
int embed_launch(int type, const void* w, const int* tokens, const int* pos, float* x, int cols, int form,
                 hipStream_t st);
int argmax_launch(const float* logits, int n, int* tokens, const int* pos, hipStream_t st);
int add_int_launch(int* p, int v, hipStream_t st);

// Batched prefill (mxh_prefill.hip): dequant-to-bf16 MFMA GEMM
// out[m x n] (row stride ldo) = a[m x k] (bf16, row stride lda) . W[n x k]^T (+ res);
// with a_lo (the bf16 residual of a) the split three-product form; `part`
// (part_floats floats, may be null) lets narrow shapes split K
int gemm_bf16_run(int type, const uint16_t* a, const uint16_t* a_lo, int lda, const void* w, float* out, int ldo,
                  const float* res, int m, int n, int k, int form, float* part, size_t part_floats, hipStream_t st);
// Prefill GEMM with exact Q4_K / Q5_K / Q8_0 / Q5_0 weights on the fp16 matrix cores
// (mxh_prefill_q4k.hip): a as fp16 hi / lo of a * 2^e per row, s the split
// sums of every 32-element sub-block of those values (row stride lds),
// rscale = 2^-e per row; inputs from rows_to_f16 / silu_mul_f16
bool gemm_q_f16_supported(int type, int k);
int gemm_q_f16_run(int type, const uint16_t* a_hi, const uint16_t* a_lo, int lda, const uint16_t* s_hi,
                     const uint16_t* s_lo, int lds, const float* rscale, const void* w, float* out, int ldo,
                     const float* res, int m, int n, int k, int form, float* part, size_t part_floats, hipStream_t st);
int rows_to_f16_launch(const float* x, int ldx, const float* nw, float eps, int k, uint16_t* a_hi, uint16_t* a_lo,
                       int lda, uint16_t* s_hi, uint16_t* s_lo, int lds, float* rscale, int m, hipStream_t st);
int silu_mul_f16_launch(const float* gu, int f, uint16_t* h_hi, uint16_t* h_lo, uint16_t* s_hi, uint16_t* s_lo,
                        float* rscale, int m, hipStream_t st);
int rows_to_bf16_launch(const float* x, int ldx, const float* nw, float eps, int k, uint16_t* a, uint16_t* a_lo,
                        int lda, int m, hipStream_t st);
int silu_mul_bf16_launch(const float* gu, int f, uint16_t* h, uint16_t* h_lo, int m, hipStream_t st);
// Device sampling (mxh_sample.hip).  Parameters live in device memory so a
// captured decode graph reads the current values; `draws` counts the random
// draws taken (the stream position of the seeded generator).
struct SampleParams {
    int top_k;
    int pad;
    double temperature, top_p, min_p;
    uint64_t seed;
    uint64_t draws;
};
size_t sample_scratch_keys(int n, int top_k);
// largest top_k the device sampler takes (two passes up to 64, a one-
// workgroup radix select above)
constexpr int kSampleTopKMax = 4096;
// Logit edits before the choice (minxfmr.cpp:2047-2089), parameters in
// device memory: suppressed ids to -inf, then over the last last_n ids of
// tokens[0 .. *pos] (all when last_n < 0) each distinct id with count c:
// l = (l <= 0 ? l * repeat : l / repeat) - c * frequency - presence.  cnt is
// an n_vocab int scratch that is zero before and after.
struct EditParams {
    int last_n;
    int n_suppress;
    double repeat_penalty, frequency_penalty, presence_penalty;
};
int logit_edits_launch(float* logits, int n_vocab, const int* tokens, const int* pos, const EditParams* prm,
                       const int* suppress, int* cnt, hipStream_t st);
int sample_launch(const float* logits, int n, SampleParams* prm, int top_k, uint64_t* cand, int* out, int* tokens,
                  int* pos, hipStream_t st);
int qkv_prep_rows_launch(const float* qkv, int ldq, const float* bias, const float* q_norm, const float* k_norm,
                         const double* rope_cs, int p0, int m, float* q_out, __half* kc, __half* vc, int nh, int nkv,
                         int hd, int neox, float eps, hipStream_t st);
// causal attention of prompt tokens p0 .. p0+m-1 over the fp16 cache, on the
// fp16 matrix cores (mxh_prefill_attn.hip)
int attention_rows_mfma_launch(const float* q, const __half* kc, const __half* vc, float* att, int p0, int m, int nh,
                               int nkv, int hd, float scale, hipStream_t st);
int embed_rows_launch(int type, const void* w, const int* tokens, int p0, int m, float* x, int cols, int form,
                      hipStream_t st);

}  // namespace mxh
