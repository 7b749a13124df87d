/*
 * mxo — CPU oracle for the minXfmr HIP backend.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU path (minXfmr.cpp: src/tensor, src/backend/backend_runtime.cpp,
 * src/backend/cpu, src/transformer, src/cache, src/api/minxfmr.cpp).  It is
 * the checker the HIP path is compared against; only tests/, the smoke entry
 * and the CPU-baseline leg of the benchmark may load it.  Nothing in the
 * product library links or calls it.
 *
 * Every function cites the reference file:line it restates.  Where the
 * reference has no counterpart (Q5_K, Qwen3 QK-norm, seeded sampling) the
 * comment says so and names the published algorithm followed instead.
 *
 * Pins (tests/test_oracle_pins.py, tests/test_oracle_layer.py,
 * tests/test_oracle_qknorm.py): fp16 decode, Q4_K/Q8_0/Q5_0 dequant,
 * matmul_rhs_t, rmsnorm, rope, softmax and the layer stack (also past a
 * full cache, where the reference's KV ring overwrites the oldest row) are
 * checked against the reference's own KATs, vectors from the reference
 * source compiled under oracle/_ref, closed forms and brute force.  Where the
 * reference has no code:
 *   - mxo_dequant_q6k_block and the F16 decode: pinned against the
 *     reference's own GGUF loader (gguf_dequant_q6_k, gguf_read_f32_tensor)
 *     compiled under oracle/_ref, on random and special blocks;
 *   - mxo_dequant_q5k_block (no reference Q5_K): pinned to the published
 *     ggml layout by its exact reduction to Q4_K with a zero high-bit plane,
 *     the position of each high bit, and quantizer round trips;
 *   - QK-norm placement in the model step (Qwen3 order: after the q/k
 *     projections, before RoPE): pinned by a float64 numpy forward of a tiny
 *     Qwen3 model written from that definition (1e-5), which the other
 *     placements miss by 1e-2;
 *   - mxo_sample's top-k / temperature / top-p / min-p cuts: pinned by
 *     closed-form cases whose kept set and probabilities are known (draws
 *     stay in the set, 20k-draw frequencies match).  The random draw itself
 *     replaces the reference's unseeded mt19937, so which id a given seed
 *     picks has no reference counterpart (parity unpinned for the draw).
 */
#ifndef MXO_H
#define MXO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor element types, numbered as GGUF/ggml type ids. */
enum {
    MXO_F32 = 0,
    MXO_F16 = 1,
    MXO_Q5_0 = 6,
    MXO_Q8_0 = 8,
    MXO_Q4_K = 12,
    MXO_Q5_K = 13,
    MXO_Q6_K = 14,
    /* type 41, read by the reference's gguf_dequant_q1_0
     * (gguf_reader.cpp:1010-1098) as one byte per element, the byte's value
     * (its size rule gives 1 byte per element, :575-584) */
    MXO_Q1_0 = 41,
};

/* Q4_K / Q5_K 6-bit scale unpacking forms.
 *  MXO_FORM_REF : reference CPU decoder (tensor.cpp:395-403); sub-blocks 4..7
 *                 take the top two bits of BOTH scale and min from q[j]>>6.
 *  MXO_FORM_GGML: ggml decoder (scale top bits from q[j-4]>>6), as in the
 *                 reference CUDA decoder (cuda_backend.cu:175-183). */
enum { MXO_FORM_REF = 0, MXO_FORM_GGML = 1 };

float mxo_fp16_to_fp32(uint16_t h);
uint16_t mxo_fp32_to_fp16(float f);

void mxo_scale_min_k4(int j, const uint8_t *scales, int form, uint8_t *sc, uint8_t *mn);

void mxo_dequant_q4k_block(const uint8_t *blk, float *y256, int form);
void mxo_dequant_q5k_block(const uint8_t *blk, float *y256, int form);
void mxo_dequant_q8_0_block(const uint8_t *blk, float *y32);
void mxo_dequant_q5_0_block(const uint8_t *blk, float *y32);
void mxo_dequant_q6k_block(const uint8_t *blk, float *y256);

size_t mxo_block_elems(int type);
size_t mxo_block_bytes(int type);
size_t mxo_row_bytes(int type, size_t cols);

/* Dequantize `rows` rows of a [rows x cols] tensor into out (rows*cols floats). */
int mxo_dequant_rows(int type, const void *w, size_t rows, size_t cols, float *out, int form);

/* out[M x N] = A[M x K] . dequant(B[N x K])^T with the reference's
 * accumulation types and order (backend_runtime.cpp:266-376). */
int mxo_matmul_rhs_t(int type, const float *A, size_t M, size_t K, const void *B, size_t N,
                     float *out, int form, int nthreads);

/* Quantizers (test-data generators for synthetic GGUF models). */
void mxo_quantize_q8_0_row(const float *x, size_t n, uint8_t *out);
void mxo_quantize_q4k_row(const float *x, size_t n, uint8_t *out);
void mxo_quantize_q5k_row(const float *x, size_t n, uint8_t *out);
void mxo_quantize_q5_0_row(const float *x, size_t n, uint8_t *out);
void mxo_quantize_q6k_row(const float *x, size_t n, uint8_t *out);

/* Layer ops (seq = 1). */
void mxo_rmsnorm(const float *x, const float *w, float *y, size_t n, float eps);
void mxo_rope(float *v, size_t n_heads, size_t head_dim, size_t n_rot, size_t pos, float theta, int neox);
void mxo_softmax(float *row, size_t len);
float mxo_silu(float x);

/* ---- whole-model oracle over a GGUF file ---- */
typedef struct mxo_model mxo_model;

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx;
    float eps, rope_theta;
    int has_qk_norm, has_bias, tied_output;
    int type_wq, type_wffn_down, type_output, type_embd;
} mxo_model_info;

/* flags for mxo_model_open */
enum {
    MXO_OPEN_ROPE_NEOX = 1,   /* NeoX (i, i+half) pairs instead of (2i, 2i+1) */
    MXO_OPEN_KV_FP16 = 2,     /* store K/V rounded through fp16 (GPU cache) */
    MXO_OPEN_GGML_FORM = 4,   /* ggml Q4_K/Q5_K scale unpacking */
    MXO_OPEN_NO_QK_NORM = 8,  /* ignore attn_{q,k}_norm (reference layer semantics) */
};

mxo_model *mxo_model_open(const char *path, int n_ctx, int flags, int nthreads);
void mxo_model_close(mxo_model *m);
void mxo_model_info_get(const mxo_model *m, mxo_model_info *info);
void mxo_model_reset(mxo_model *m);
/* Run one token at the next cache position; past n_ctx tokens the cache is
 * the reference's ring (the oldest row is overwritten, RoPE stays at
 * position n_ctx).  logits (n_vocab) may be NULL;
 * hidden_trace, when non-NULL, receives n_layer*n_embd floats (hidden state
 * after each layer) followed by n_embd floats of the final-normed hidden. */
int mxo_model_step(mxo_model *m, int token, float *logits, float *hidden_trace);
int mxo_model_pos(const mxo_model *m);
/* Move the position to `pos` (0 <= pos < n_ctx) without running the
 * positions before it: their cache rows keep what they hold (zeros after
 * open).  For timing steps at a given context length, whose work does not
 * depend on the cached values; not a reference operation. */
int mxo_model_set_pos(mxo_model *m, int pos);

/* argmax with lowest index on ties (minxfmr.cpp:2091-2115, greedy = order[0]) */
int mxo_argmax(const float *logits, size_t n);

/* Seeded top-k / temperature / top-p / min-p draw (minxfmr.cpp:2091-2171,
 * with the unseeded std::mt19937 + discrete_distribution replaced by a
 * splitmix64 uniform and an inverse-CDF pick).  Returns the token id. */
int mxo_sample(const float *logits, size_t n, int top_k, double temperature, double top_p,
               double min_p, uint64_t *rng_state);
double mxo_rng_uniform(uint64_t *state);

/* Logit edits before the choice (minxfmr.cpp:2047-2089): suppressed ids to
 * -inf, then repetition / frequency / presence penalties over the last
 * repeat_last_n ids of history (all when < 0). */
void mxo_logit_edits(float *logits, size_t n, const int *history, size_t n_hist, const int *suppress,
                     size_t n_suppress, int repeat_last_n, double repeat_penalty, double frequency_penalty,
                     double presence_penalty);

#ifdef __cplusplus
}
#endif
#endif
