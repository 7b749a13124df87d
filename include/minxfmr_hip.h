/*
 * minxfmr_hip.h — C ABI of the MI355X (gfx950) backend for minXfmr.cpp.
 *
 * Plain C types only: device pointers are `void*` / `float*` obtained from
 * mxh_alloc (or any HIP allocation on the current device), sizes are
 * int64_t/size_t, status is an int (MXH_OK == 0, negative on failure, with a
 * message from mxh_last_error()).  Every launch goes to the library's own
 * stream on the current device and is asynchronous unless the function says
 * otherwise.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the minXfmr.cpp tree).  The library is
 * thread-compatible, not thread-safe: one caller thread per process, as in
 * the reference's single-context runtime (src/api/minxfmr.cpp globals).
 */
#ifndef MINXFMR_HIP_H
#define MINXFMR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor element types, numbered as GGUF type ids.  Replaces DataType
 * (src/tensor/tensor.h:5-14), which lacks F16, Q5_K and Q6_K: the
 * reference converts F16 and Q6_K tensors to F32 when it loads them
 * (third_party/gguf/gguf_reader.cpp:759-785, :905-1008) and has no Q5_K;
 * here all three stay packed in HBM and are decoded by the kernels. */
enum {
    MXH_F32 = 0,
    MXH_F16 = 1,
    MXH_Q5_0 = 6,
    MXH_Q8_0 = 8,
    MXH_Q4_K = 12,
    MXH_Q5_K = 13,
    MXH_Q6_K = 14,
    /* GGUF type 41, which the reference reads in gguf_dequant_q1_0
     * (third_party/gguf/gguf_reader.cpp:1010-1098): its tensor size rule
     * gives 1 byte per element for this type (:575-584), so it takes each
     * byte as the weight's value, 0..255.  mxh_model_open widens such
     * tensors to F32 when it loads them, as the reference does. */
    MXH_Q1_0 = 41
};

/* flag of the tiled weight layout (mxh_tile_rows): MXH_TILED_FLAG | type */
#define MXH_TILED_FLAG 0x100

/* Q4_K/Q5_K 6-bit scale unpacking.  MXH_FORM_REF is the reference CPU
 * decoder (src/tensor/tensor.cpp:395-403) and the default; MXH_FORM_GGML is
 * the ggml decoder used by the reference CUDA kernels
 * (src/backend/cuda/cuda_backend.cu:175-183). */
enum { MXH_FORM_REF = 0, MXH_FORM_GGML = 1 };

enum {
    MXH_OK = 0,
    MXH_ERR_ARG = -1,         /* bad pointer / shape / type combination */
    MXH_ERR_UNSUPPORTED = -2, /* valid request the backend does not implement */
    MXH_ERR_HIP = -3,         /* HIP runtime error */
    MXH_ERR_NODEV = -4,       /* no usable gfx950 device */
    MXH_ERR_OOM = -5          /* device allocation failed */
};

/* ---- lifecycle ------------------------------------------------------ */

/* Select `device`, create the library stream.  Idempotent.
 * Replaces cuda_backend_is_available's lazy ensure_ready
 * (src/backend/cuda/cuda_backend.cu:123-133). */
int mxh_init(int device);

/* 1 when a gfx950 device is usable (initialising on first call).
 * Replaces cuda_backend_is_available (src/backend/cuda/cuda_backend.h:5). */
int mxh_is_available(void);

/* Message of the last failure on this thread ("" when none); library-owned.
 * Replaces cuda_backend_last_error_msg (src/backend/cuda/cuda_backend.h:21)
 * and backend_last_preload_error (src/backend/backend_runtime.h:48). */
const char *mxh_last_error(void);

/* Block until all work on the library stream is done. */
int mxh_synchronize(void);

/* The library stream as an opaque hipStream_t, for callers that order their
 * own work (events, copies) against the library's launches. */
void *mxh_stream(void);

/* ---- device memory (plumbing) ---------------------------------------- */
int mxh_alloc(void **dptr, size_t bytes);
int mxh_free(void *dptr);
int mxh_upload(void *dst, const void *src, size_t bytes);   /* synchronous */
int mxh_download(void *dst, const void *src, size_t bytes); /* synchronous */
int mxh_memset(void *dptr, int value, size_t bytes);        /* async */
int mxh_copy(void *dst, const void *src, size_t bytes);      /* device to device, async */

/* Elapsed time of the work enqueued between begin and end, measured with
 * events on the library stream.  mxh_timer_end synchronizes. */
int mxh_timer_begin(void);
int mxh_timer_end(float *ms);

/* ---- the decode hot path (device pointers) ---------------------------- */

/* y[n] = sum_k x[k] * dequant(W[n, k]) for W a row-major [n x k] tensor of
 * raw GGUF blocks (k a multiple of the block size).  W must be 16-byte
 * aligned for Q4_K/Q5_K/F16/F32 and 4-byte aligned for Q8_0/Q5_0/Q6_K.
 * `type` may also be the tiled id mxh_tile_rows returned for W's rows
 * (16-byte aligned).  F16 and Q6_K rows are multiplied as the values the
 * reference's loader converts them to (gguf_reader.cpp:759-785, :905-1008).
 * Replaces the m == 1 case of backend_matmul_rhs_transposed
 * (src/backend/backend_runtime.cpp:266-376, cuda_backend.cu:1198-1415). */
int mxh_gemv(int type, const void *w, const float *x, float *y, int64_t n, int64_t k, int form);

/* Regroups the bytes of each of `rows` device rows of `cols` elements in
 * place into the tiled order the GEMV reads fastest (every 16-byte load of a
 * wave within whole cache lines), and sets *tiled to the type id to pass to
 * mxh_gemv from then on: MXH_TILED_FLAG | type for Q4_K, Q5_K and Q8_0 with
 * cols a multiple of 256 up to 15360 and for Q6_K with cols a multiple of
 * 2048 up to 15360; otherwise the rows are left as they are and
 * *tiled = type.  W must be 16-byte aligned.  Results through the
 * tiled rows are identical to those through the GGUF rows.  No reference
 * counterpart: the reference has one weight layout, the GGUF block order the
 * CUDA backend uploads (cuda_backend.cu:364-394). */
int mxh_tile_rows(int type, void *w, int64_t rows, int64_t cols, int *tiled);

/* out[m x n] = A[m x k] . dequant(W[n x k])^T for any m (prefill).
 * Replaces backend_matmul_rhs_transposed (src/backend/backend_runtime.h:37). */
int mxh_matmul_rhs_t(int type, const float *a, int64_t m, const void *w, int64_t n, int64_t k, float *out,
                     int form);

/* out[rows x cols] fp32 = dequant(W) — bit-exact with the CPU decoder.
 * Replaces the debug dequant kernels
 * (src/backend/cuda/cuda_backend.cu:583-674, cuda_backend_compare_dequant). */
int mxh_dequant(int type, const void *w, float *out, int64_t rows, int64_t cols, int form);

/* out[m x n] = bf16(a[m x k]) . bf16(dequant(w[n x k]))^T with fp32
 * accumulation on the matrix cores (v_mfma_f32_32x32x16_bf16); device
 * pointers, k a multiple of 64.  The prefill contraction: the reference runs
 * it as backend_matmul_rhs_transposed with m > 1
 * (src/backend/backend_runtime.cpp:302-319); this entry trades its fp32
 * inputs for bf16 ones. */
int mxh_gemm_q_bf16(int type, const float *a, int64_t m, const void *w, int64_t n, int64_t k, float *out, int form);

/* out[m x n] = a[m x k] . dequant(w[n x k])^T on the fp16 matrix cores with
 * every weight exact: the MFMAs multiply the integer codes (Q4_K / Q5_K:
 * sc * q; Q8_0: q; Q5_0: q - 16), exact in fp16, and the block scales are
 * applied to fp32 partial sums (K-quant mins by a second contraction over
 * sub-block sums).  a enters as fp16 hi + lo of a * 2^e per row (about 22
 * significant bits).  Device pointers, a and w 16-byte aligned; type Q4_K,
 * Q5_K, Q8_0 or Q5_0 (or a tiled id of mxh_tile_rows), k a multiple of 256 up
 * to 16384.  The prefill contraction the model runs: the reference's
 * backend_matmul_rhs_transposed with m > 1
 * (src/backend/backend_runtime.cpp:302-319). */
int mxh_gemm_q_f16(int type, const float *a, int64_t m, const void *w, int64_t n, int64_t k, float *out, int form);

/* mxh_gemm_q_f16 without any allocation: the staged activations live in a
 * device scratch array of 12 MiB that every GPU the library runs on holds
 * from load until the process ends, so 4 m k + m k / 8 + 4 m bytes (about
 * 4.1 bytes per element of a) must fit in it; larger requests are rejected
 * with MXH_ERR_ARG and a message.  Calls no hipMalloc / hipFree; results are
 * identical to mxh_gemm_q_f16's.  Every call on a GPU reuses that GPU's
 * scratch, so calls that overlap on one GPU (from several host threads, or
 * with work the caller enqueues on other streams) race.  No counterpart in
 * the reference: for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid allocation). */
int mxh_gemm_q_f16_noalloc(int type, const float *a, int64_t m, const void *w, int64_t n, int64_t k, float *out,
                           int form);

/* Causal attention of m consecutive prompt tokens at positions p0 .. p0+m-1
 * (transformer.cpp:529-629, per token: softmax of q.k / sqrt(hd) over cache
 * positions 0 .. pos, then the weighted sum of V rows), on the fp16 matrix
 * cores; device pointers.  q: [m][nh*hd] fp32 (after RoPE); kc, vc: the fp16
 * cache [>= p0+m][nkv*hd] with rows 0 .. p0+m-1 written; att: [m][nh*hd].
 * nh a multiple of nkv with at most 8 q heads per kv head, hd 32, 64 or 128.
 * The batched prefill's attention step. */
int mxh_attention_prefill(const float *q, const void *kc, const void *vc, float *att, int p0, int m, int nh, int nkv,
                          int hd);

/* ---- per-op backend interface (host pointers) ------------------------- */
/* These keep the reference op semantics for drop-in use: host pointers in
 * and out, one synchronous device round trip per call.  Quantized weights
 * are cached on the device keyed by (host pointer, bytes). */

/* Replaces cuda_backend_preload_tensor (src/backend/cuda/cuda_backend.h:7). */
int mxh_preload(const void *host, size_t bytes);

/* Replaces cuda_backend_release_resources (src/backend/cuda/cuda_backend.h:6). */
void mxh_release_resources(void);

/* Replaces cuda_backend_matmul_rhs_transposed (cuda_backend.h:25). */
int mxh_host_matmul_rhs_t(int type, const float *a, int64_t m, int64_t k, const void *w, size_t w_bytes, int64_t n,
                          float *out, int form);

/* F32 out[m x n] = A[m x k] . B[k x n].  Replaces cuda_backend_matmul for F32
 * operands (cuda_backend.h:24). */
int mxh_host_matmul_f32(const float *a, const float *b, float *out, int64_t m, int64_t k, int64_t n);

/* out[m x n] = A[m x k] . dequant(B[k x n]) with B quantized along its rows
 * (each of its k rows holds n columns as `type` blocks; F32 accepted too).
 * B is cached on the device keyed by (host pointer, b_bytes), decoded there
 * bit-exactly to fp32 and multiplied in fp32.  Replaces cuda_backend_matmul
 * for quantized B (cuda_backend.h:24; CPU semantics cpu_backend.cpp:119-200). */
int mxh_host_matmul_q(int type, const float *a, int64_t m, int64_t k, const void *b, size_t b_bytes, int64_t n,
                      float *out, int form);

/* out[n] = sum_k vec[k] * mat[k * stride + n].
 * Replaces cuda_backend_matvec_strided (cuda_backend.h:26). */
int mxh_host_matvec_strided(const float *vec, const float *mat, float *out, size_t K, size_t N, size_t stride);

/* out[j] = dot(vec, rows[j * stride .. +K]).
 * Replaces cuda_backend_vec_dot_rows (cuda_backend.h:27). */
int mxh_host_vec_dot_rows(const float *vec, const float *rows, float *out, size_t K, size_t nrows, size_t stride);

/* out[j] = dot(vec, ring[((head + j) % seq_max) * stride .. +K]), j < len.
 * Replaces cuda_backend_vec_dot_rows_ring (cuda_backend.h:28). */
int mxh_host_vec_dot_rows_ring(const float *vec, const float *ring, size_t head, size_t seq_max, size_t len,
                               size_t K, size_t stride, float *out);

/* out[c] = sum_r vec[r] * rows[r * stride + c].
 * Replaces cuda_backend_vec_mul_rows_cols (cuda_backend.h:29). */
int mxh_host_vec_mul_rows_cols(const float *vec, const float *rows, float *out, size_t nrows, size_t ncols,
                               size_t stride);

/* ---- device-resident decoder model ------------------------------------ */
/* Replaces the runtime's per-token stack walk (run_stack_forward,
 * src/api/minxfmr.cpp:544-663) and decode loop (src/api/minxfmr.cpp:1849-2390)
 * for llama-family GGUF models (qwen2/qwen3/llama tensor names): weights,
 * fp16 KV cache and activations stay in HBM; one token step is one HIP graph
 * replay with no host round trip. */
typedef struct mxh_model mxh_model;

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx;
    float eps, rope_theta;
    int has_qk_norm, has_bias, type_wq, type_wv, type_wffn_down, type_output, type_embd;
    int64_t weight_bytes;      /* HBM bytes of every uploaded tensor */
    int64_t step_read_bytes;   /* weight bytes one decode step streams (layers + lm-head) */
} mxh_model_config;

enum {
    MXH_MODEL_ROPE_NEOX = 1,    /* (i, i + rot/2) pairs; default (2i, 2i+1) as rope.cpp:39-45 */
    MXH_MODEL_GGML_FORM = 4,    /* ggml Q4_K/Q5_K scale unpacking instead of the reference CPU form */
    MXH_MODEL_NO_QK_NORM = 8,   /* ignore attn_{q,k}_norm (reference layer semantics) */
    MXH_MODEL_NO_GRAPH = 16,    /* enqueue kernels directly instead of replaying HIP graphs */
    MXH_MODEL_TOKEN_PREFILL = 32, /* prompt token by token through the decode step (GEMVs with 24-bit x)
                                     instead of batched on the matrix cores */
    MXH_MODEL_GGUF_LAYOUT = 64,   /* keep the projection weights in their GGUF block order in HBM instead of
                                     the tiled order (same bytes regrouped per row) the kernels read fastest;
                                     results are identical either way */
    MXH_MODEL_BF16_PREFILL = 128  /* batched prefill GEMMs in the split-bf16 form for every weight type; by
                                     default quantized projections use the exact-weight fp16 form (weights as
                                     integer codes, activations as fp16 hi + lo) */
};

/* Load a GGUF file into HBM with a KV cache of n_ctx rows (the reference's
 * seq_max).  Past n_ctx tokens the cache is the reference's ring
 * (src/cache/kv_cache.cpp:50-75): each step attends the last n_ctx cached
 * tokens and itself, RoPE stays at position n_ctx (transformer.cpp:506), and
 * the oldest row is overwritten.  The id history holds max(n_ctx + 1, 2^20)
 * ids; prefill, decode and generate stop with an error before it is full.
 * Replaces minxfmr_open's load path (src/api/minxfmr.cpp:702-1415). */
int mxh_model_open(const char *gguf_path, int n_ctx, int flags, mxh_model **out);
int mxh_model_config_get(const mxh_model *m, mxh_model_config *cfg);
/* Position 0, empty cache.  Replaces kvcache_reset (src/cache/kv_cache.cpp:77-83). */
int mxh_model_reset(mxh_model *m);
int mxh_model_position(const mxh_model *m);
/* Run `token` at the current position and advance.  logits (n_vocab floats)
 * and trace ((n_layer + 1) * n_embd floats: hidden after each layer, then the
 * final-normed hidden) are host buffers and may be NULL.  Synchronous. */
/* Sampling of the next token after each step (replaces the greedy argmax):
 * the top_k (1..4096) largest logits, softmax at `temperature` in double,
 * then the top-p and min-p cuts, then a draw from a seeded splitmix64
 * stream (the d-th draw uses state seed + (d+1) * 0x9E3779B97F4A7C15).
 * temperature <= 0 restores greedy decoding.  mxh_model_reset rewinds the
 * stream to draw 0.  Replaces the sampler of src/api/minxfmr.cpp:2091-2171,
 * whose std::mt19937 is unseeded; the arithmetic before the draw is the
 * same. */
int mxh_model_set_sampling(mxh_model *m, int top_k, double temperature, double top_p, double min_p, uint64_t seed);

/* Logit edits applied before every following choice (greedy or sampled),
 * on the device, as src/api/minxfmr.cpp:2047-2089 applies them: the ids in
 * suppress[0 .. n_suppress) get -inf (the caller passes the reference's
 * special-token ids minus its EOS tokens), then over the last repeat_last_n
 * ids of the history (prompt and generated ids up to the current position;
 * repeat_last_n < 0: all of it) each distinct id with count c has its logit
 * l replaced by (l <= 0 ? l * repeat_penalty : l / repeat_penalty)
 * - c * frequency_penalty - presence_penalty, computed in double (the
 * repeat factor only when repeat_penalty != 1; no penalty pass when the
 * window is empty or all three are neutral).  No ids and neutral penalties
 * restore the fused greedy head.  The reference keeps logits in double; here
 * they are fp32, so the edited value is rounded once to float. */
int mxh_model_set_logit_edits(mxh_model *m, const int *suppress, int n_suppress, int repeat_last_n,
                              double repeat_penalty, double frequency_penalty, double presence_penalty);

/* One sampling decision over n device-resident logits with the rules of
 * mxh_model_set_sampling, using draw number `draw` of the stream; the token
 * id is written to *token (host).  For tests and per-op callers. */
int mxh_sample(const float *logits, int n, int top_k, double temperature, double top_p, double min_p, uint64_t seed,
               uint64_t draw, int *token);

/* Feed n prompt tokens at the current position without producing logits:
 * batched on the matrix cores in chunks of up to 512 tokens (exact-weight fp16
 * MFMA GEMMs, row-batched QK-norm/RoPE/KV append and causal attention) while
 * the cache has room for them, then token by token past a full cache, and
 * token by token throughout when the model was opened with
 * MXH_MODEL_TOKEN_PREFILL.  Replaces the reference's token-by-token prompt
 * loop (src/api/minxfmr.cpp:1503-1548). */
int mxh_model_prefill(mxh_model *m, const int *tokens, int n);
int mxh_model_step(mxh_model *m, int token, float *logits, float *trace);
/* Greedy generation from position 0: prefill n_prompt ids, then n_gen
 * decode steps; out receives n_gen ids.  prefill_ms / decode_ms (nullable)
 * receive the device time of each phase.  Synchronous. */
int mxh_model_generate(mxh_model *m, const int *prompt, int n_prompt, int n_gen, int *out, float *prefill_ms,
                       float *decode_ms);
/* Continue greedy decoding for n_gen steps from the current position (the id
 * at the position is the input); out (nullable) receives n_gen ids. */
int mxh_model_decode(mxh_model *m, int n_gen, int *out, float *decode_ms);
/* Make `token` the id at the current position: the input of the next
 * mxh_model_decode step and the newest entry of the history that the logit
 * edits count (the device token array, which otherwise holds the id the
 * device chose there).  For a host that changes the device's choice: the
 * reference's first-token swap replaces `next` by a visible alternative of
 * its top-k order before it becomes `last` and enters token_history
 * (src/api/minxfmr.cpp:2189-2205, :2388-2389).  Synchronous. */
int mxh_model_set_token(mxh_model *m, int token);
/* Enqueue every GEMV of the model whose weights have `type` (in layer order,
 * then the lm-head) `reps` times on the library stream, on the model's own
 * HBM-resident weights and in the form the decode step launches it (norm
 * fused into the q|k|v and gate|up staging, SwiGLU epilogue for gate|up,
 * residual for o and down; the lm-head plain), writing scratch vectors only;
 * reports device time, launch count and algorithmic bytes (weights + fp32 x
 * and y).  Benchmark support, no reference counterpart. */
int mxh_model_bench_gemv(mxh_model *m, int type, int reps, float *ms, int64_t *launches, int64_t *bytes);
/* Enqueue the decode attention of every layer (and, where the context runs
 * the grouped kernel, its merge) at the model's current position `reps`
 * times on the library stream, as the decode step launches it; reports
 * device time, launch count (layers x reps) and algorithmic bytes (the K and
 * V rows read, 2 pos n_kv head_dim 2 per layer).  It rewrites cache row pos
 * (which the next step writes before any read) and the split partials.
 * Benchmark support, no reference counterpart. */
int mxh_model_bench_attention(mxh_model *m, int reps, float *ms, int64_t *launches, int64_t *bytes);
void mxh_model_close(mxh_model *m);

/* Seeded synthetic GGUF writer (weights N(0, 0.02) quantized per type, norms
 * F32 near 1), for benchmarks on models that cannot be downloaded.  No
 * reference counterpart.  Types are GGUF ids; attn_v_type / ffn_down_type
 * of -1 mean wtype. */
typedef struct {
    const char *arch;
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, ctx;
    float rope_theta, eps;
    int qk_norm, tied, wtype, out_type, embd_type, attn_v_type, ffn_down_type;
} mxh_synth_arch;
int mxh_write_synthetic_gguf(const char *path, const mxh_synth_arch *arch, uint64_t seed, int threads);

#ifdef __cplusplus
}
#endif
#endif /* MINXFMR_HIP_H */
