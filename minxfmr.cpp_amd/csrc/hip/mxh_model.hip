// mxh_model.hip — a GGUF decoder model resident in HBM and its decode step.
//
// One token step runs entirely on the device with no host round trip:
//   embed -> n_layer x [rmsnorm, fused QKV GEMV, bias/QK-norm/RoPE/KV-append,
//   split-K attention, Wo GEMV + residual, rmsnorm, fused gate|up GEMV,
//   SiLU*up, down GEMV + residual] -> final rmsnorm -> lm-head GEMV -> argmax.
// The token and position live in device memory, so the step is captured once
// into a HIP graph and replayed per token; generated ids accumulate in a
// device token array.  Reference path being replaced: run_stack_forward +
// the generate loop (src/api/minxfmr.cpp:544-663, 1417-2171) over
// transformer_forward_single_layer (src/transformer/transformer.cpp:330-755).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <deque>
#include <exception>
#include <new>
#include <initializer_list>
#include <memory>
#include <string>
#include <vector>

#include "../host/mxh_gguf.h"
#include "mxh_internal.h"

using namespace mxh;

namespace {

struct DevW {
    const void* p = nullptr;
    int type = -1;
    int64_t rows = 0, cols = 0;
};

struct Layer {
    DevW qkv;         // fused [Wq; Wk; Wv] when all three share a type
    DevW q, k, v;     // otherwise separate (q covering k too, and k empty, when only q and k share a type)
    bool qkv_fused = false;
    DevW o, gu, g, u, down;
    bool gu_fused = false;
    const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    const float* bias = nullptr;  // [bq | bk | bv] or null
    __half *kc = nullptr, *vc = nullptr;
};

}  // namespace

struct mxh_model {
    mxh_model_config cfg{};
    int form = MXH_FORM_REF;
    int neox = 0;
    std::vector<Layer> layers;
    DevW embd, out;
    const float* out_norm = nullptr;
    // device memory
    uint8_t* blob = nullptr;  // weights + norms
    size_t blob_bytes = 0;
    uint8_t* out_copy = nullptr;  // tiled copy of an embedding table the output projection is tied to
    __half* kv = nullptr;
    double* rope_cs = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr, *h = nullptr, *logits = nullptr,
          *part = nullptr, *trace = nullptr, *red_val = nullptr;
    int* red_idx = nullptr;
    int red_cap = 0;
    int* tokens = nullptr;  // [token_cap]: prompt then generated ids
    int token_cap = 0;      // ids the history holds (steps run while host_pos + 1 < token_cap)
    int* pos = nullptr;     // current position
    int host_pos = 0;
    bool trace_on = false;
    bool token_prefill = false;  // prompt token by token instead of batched
    hipGraphExec_t g_prefill = nullptr, g_decode = nullptr, g_sample = nullptr;
    // the same steps at or past a full cache (the ring's kernels), captured
    // on first use and dropped whenever the ones above change
    hipGraphExec_t g_prefill_w = nullptr, g_decode_w = nullptr, g_sample_w = nullptr;
    // sampling instead of greedy argmax (mxh_model_set_sampling)
    bool sampling = false;
    int top_k = 1;
    SampleParams* sprm = nullptr;  // device copy, draw counter included
    uint64_t* scand = nullptr;     // pass-1 candidates
    // logit edits before the choice (mxh_model_set_logit_edits)
    bool edits = false;
    EditParams* eprm = nullptr;  // device copy
    int* esup = nullptr;         // suppressed ids [n_vocab]
    int* ecnt = nullptr;         // per-id counts [n_vocab], zero between steps
    // batched prefill (allocated on first use): rows of up to pf_rows tokens
    int pf_rows = 0;
    float *pf_x = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_gu = nullptr;
    uint16_t *pf_a = nullptr, *pf_a_lo = nullptr;  // GEMM input as split bf16 (hi, lo)
    // GEMM input of the Q4_K fp16 kernel: fp16 hi / lo of a * 2^e per row,
    // split sub-block sums, 2^-e per row
    uint16_t *pf_h16 = nullptr, *pf_l16 = nullptr, *pf_sh = nullptr, *pf_sl = nullptr;
    float* pf_rscale = nullptr;
    bool bf16_prefill = false;  // every prefill GEMM in the split-bf16 form
    float* pf_part = nullptr;                        // split-K partial tiles
    size_t pf_part_floats = 0;
};

namespace {

int gemv(const DevW& w, const float* x, float* y, const float* res, int form, hipStream_t st,
         const float* norm_w = nullptr, float eps = 0.f, int mode = GEMV_PLAIN, mxh_model* m = nullptr) {
    GemvArgs a{};
    a.w = (const uint8_t*)w.p;
    a.x = x;
    a.y = y;
    a.res = res;
    a.norm_w = norm_w;
    a.eps = eps;
    a.n = (int)w.rows;
    a.k = (int)w.cols;
    a.form = form;
    if (mode == GEMV_ARGMAX) {
        a.red_val = m->red_val;
        a.red_idx = m->red_idx;
        a.red_cap = m->red_cap;
        a.tokens = m->tokens;
        a.pos = m->pos;
    }
    if (mode == GEMV_ATTN) {
        a.part = m->part;
        a.part_splits = attention_splits(m->cfg.n_ctx, m->cfg.n_head, m->cfg.n_head_kv, m->cfg.head_dim);
        a.part_hd = m->cfg.head_dim;
    }
    return gemv_run(w.type, a, mode, st);
}

// Whether the o-projection merges the attention partials in its x staging
// (GEMV_ATTN: quantized rows of at most 4096 inputs, at most kAttnMaxSplits
// partials per q head); otherwise a merge kernel writes the attention output
// first (always for the grouped kernel of long contexts).
bool o_merges(const mxh_model* m, const DevW& o) {
    const mxh_model_config& c = m->cfg;
    return gemv_int_x(o.type) && o.cols <= 4096 &&
           attention_splits(c.n_ctx, c.n_head, c.n_head_kv, c.head_dim) <= kAttnMaxSplits;
}

// the o-projection and residual of the decode step, from the attention partials
int o_proj(mxh_model* m, const Layer& L, hipStream_t st) {
    if (o_merges(m, L.o)) return gemv(L.o, nullptr, m->x, m->x, m->form, st, nullptr, 0.f, GEMV_ATTN, m);
    const mxh_model_config& c = m->cfg;
    int rc = attention_merge_launch(m->part, attention_splits(c.n_ctx, c.n_head, c.n_head_kv, c.head_dim), c.n_head,
                                    c.head_dim, m->att, st);
    return rc | gemv(L.o, m->att, m->x, m->x, m->form, st);
}

// The decode attention of layer L at the device position (wrapped: a step
// at or past n_ctx tokens, which runs the ring's kernels)
AttnArgs attn_args(const mxh_model* m, const Layer& L, bool wrapped) {
    const mxh_model_config& c = m->cfg;
    AttnArgs aa{};
    aa.qkv = m->qkv;
    aa.bias = L.bias;
    aa.q_norm = L.q_norm;
    aa.k_norm = L.k_norm;
    aa.rope_cs = m->rope_cs;
    aa.pos = m->pos;
    aa.kc = L.kc;
    aa.vc = L.vc;
    aa.part = m->part;
    aa.nh = c.n_head;
    aa.nkv = c.n_head_kv;
    aa.hd = c.head_dim;
    aa.neox = m->neox;
    aa.eps = c.eps;
    aa.scale = 1.0f / sqrtf((float)c.head_dim);
    aa.ring = wrapped ? c.n_ctx : 0;
    return aa;
}

// Enqueue one token step at the device position.  with_head: the final
// norm, lm-head and argmax (writing tokens[pos+1]) and the position advance
// are fused into the head GEMV; without: a prompt step.  wrapped: the step
// is at or past n_ctx tokens (the ring's attention kernels).
int enqueue_step(mxh_model* m, bool with_head, bool wrapped, hipStream_t st) {
    const mxh_model_config& c = m->cfg;
    const int d = c.n_embd, hd = c.head_dim, nh = c.n_head, nkv = c.n_head_kv;
    const int qd = nh * hd, kvd = nkv * hd;
    int rc = MXH_OK;
    // embedding of tokens[pos]: the position counter indexes the token array
    rc |= embed_launch(m->embd.type, m->embd.p, m->tokens, m->pos, m->x, d, m->form, st);
    for (int l = 0; l < c.n_layer; ++l) {
        const Layer& L = m->layers[(size_t)l];
        // attention rmsnorm is fused into the projection GEMVs
        if (L.qkv_fused) {
            rc |= gemv(L.qkv, m->x, m->qkv, nullptr, m->form, st, L.attn_norm, c.eps);
        } else {
            rc |= gemv(L.q, m->x, m->qkv, nullptr, m->form, st, L.attn_norm, c.eps);
            if (L.k.p) rc |= gemv(L.k, m->x, m->qkv + qd, nullptr, m->form, st, L.attn_norm, c.eps);
            rc |= gemv(L.v, m->x, m->qkv + qd + kvd, nullptr, m->form, st, L.attn_norm, c.eps);
        }
        rc |= attention_run(attn_args(m, L, wrapped), c.n_ctx, st);
        rc |= o_proj(m, L, st);
        if (L.gu_fused) {
            rc |= gemv(L.gu, m->x, m->h, nullptr, m->form, st, L.ffn_norm, c.eps, GEMV_SILU);
        } else {
            rc |= gemv(L.g, m->x, m->gu, nullptr, m->form, st, L.ffn_norm, c.eps);
            rc |= gemv(L.u, m->x, m->gu + c.n_ff, nullptr, m->form, st, L.ffn_norm, c.eps);
            rc |= silu_mul_launch(m->gu, m->h, c.n_ff, st);
        }
        rc |= gemv(L.down, m->h, m->x, m->x, m->form, st);
        if (m->trace_on) rc |= check_hip(hipMemcpyAsync(m->trace + (size_t)l * d, m->x, sizeof(float) * d,
                                                        hipMemcpyDeviceToDevice, st), "trace copy");
    }
    if (with_head) {
        if (m->trace_on) rc |= rmsnorm_launch(m->x, m->out_norm, m->trace + (size_t)c.n_layer * d, d, c.eps, st);
        if (m->sampling || m->edits) {
            // logits, the reference's edits (suppressed ids, penalties over
            // the history), then top-k / temperature sampling or the argmax
            // writes tokens[pos+1]
            rc |= gemv(m->out, m->x, m->logits, nullptr, m->form, st, m->out_norm, c.eps);
            if (m->edits)
                rc |= logit_edits_launch(m->logits, c.n_vocab, m->tokens, m->pos, m->eprm, m->esup, m->ecnt, st);
            if (m->sampling) {
                rc |= sample_launch(m->logits, c.n_vocab, m->sprm, m->top_k, m->scand, nullptr, m->tokens, m->pos, st);
            } else {
                rc |= argmax_launch(m->logits, c.n_vocab, m->tokens, m->pos, st);
                rc |= add_int_launch(m->pos, 1, st);
            }
        } else {
            rc |= gemv(m->out, m->x, m->logits, nullptr, m->form, st, m->out_norm, c.eps, GEMV_ARGMAX, m);
        }
    } else {
        rc |= add_int_launch(m->pos, 1, st);
    }
    return rc ? set_error(MXH_ERR_HIP, "step enqueue failed") : MXH_OK;
}

int capture(mxh_model* m, bool with_head, bool wrapped, hipGraphExec_t* out) {
    hipStream_t st = lib_stream();
    hipGraph_t g = nullptr;
    if (int rc = check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture")) return rc;
    const int rc = enqueue_step(m, with_head, wrapped, st);
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (rc) return rc;
    if (int r2 = check_hip(e, "end capture")) return r2;
    const hipError_t ie = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    return check_hip(ie, "graph instantiate");
}

void drop_graph(hipGraphExec_t& g) {
    if (g) (void)hipGraphExecDestroy(g);
    g = nullptr;
}

}  // namespace

namespace {

struct Placement {
    const GgufTensor* t;
    size_t off;
    std::shared_ptr<std::vector<uint8_t>> conv;  // bytes to upload instead of t->data (a promoted copy)
};

// A Q4_K row as Q5_K: each 144-byte block (d, dmin, 12 scale bytes, 128
// nibble bytes) becomes a 176-byte Q5_K block with the same header, a zero
// high-bit plane and the same nibbles.  Both types decode a sub-block as
// d sc q - dmin m with the same 6-bit scale/min unpacking, so every weight
// keeps its value exactly.
std::shared_ptr<std::vector<uint8_t>> q4k_as_q5k(const GgufTensor* t) {
    const int64_t nb = t->rows() * (t->cols() / 256);
    auto out = std::make_shared<std::vector<uint8_t>>((size_t)nb * 176, (uint8_t)0);
    const uint8_t* src = static_cast<const uint8_t*>(t->data);
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* in = src + (size_t)b * 144;
        uint8_t* o = out->data() + (size_t)b * 176;
        std::memcpy(o, in, 16);            // d, dmin, scales
        std::memcpy(o + 48, in + 16, 128);  // qs after the 32 zero qh bytes
    }
    return out;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int free_model(mxh_model* m) {
    if (!m) return MXH_OK;
    (void)hipStreamSynchronize(lib_stream());
    for (hipGraphExec_t* g : {&m->g_prefill, &m->g_decode, &m->g_sample, &m->g_prefill_w, &m->g_decode_w, &m->g_sample_w})
        drop_graph(*g);
    void* bufs[] = {m->blob, m->out_copy, m->kv, m->rope_cs, m->x, m->xn, m->qkv, m->att, m->gu, m->h, m->logits, m->part,
                    m->trace, m->tokens, m->pos, m->red_val, m->red_idx,
                    m->pf_x, m->pf_qkv, m->pf_q, m->pf_att, m->pf_gu, m->pf_a, m->pf_a_lo, m->pf_part,
                    m->pf_h16, m->pf_l16, m->pf_sh, m->pf_sl, m->pf_rscale, m->sprm, m->scand, m->eprm, m->esup,
                    m->ecnt};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    delete m;
    return MXH_OK;
}

template <typename T>
int dalloc(T** p, size_t count) {
    if (hipMalloc((void**)p, sizeof(T) * count + 256) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return set_error(MXH_ERR_OOM, "device allocation of %zu bytes failed", sizeof(T) * count);
    }
    return MXH_OK;
}

bool gemv_type_ok(int t) {
    return t == MXH_Q4_K || t == MXH_Q5_K || t == MXH_Q6_K || t == MXH_Q8_0 || t == MXH_Q5_0 || t == MXH_F16 ||
           t == MXH_F32;
}

}  // namespace

extern "C" {

static int model_open_impl(const char* gguf_path, int n_ctx, int flags, mxh_model** out) {
    if (!gguf_path || !out || n_ctx <= 0) return set_error(MXH_ERR_ARG, "model_open: bad arguments");
    *out = nullptr;
    // the file is checked before any device work
    GgufFile f;
    std::string err;
    if (!f.open(gguf_path, &err)) return set_error(MXH_ERR_ARG, "model_open: %s", err.c_str());
    if (int rc = mxh_init(0)) return rc;
    // Tensors of GGUF type 41 are widened to F32 here, as the reference's
    // loader does (gguf_dequant_q1_0: each byte is the value): `get` returns
    // an F32 copy over the widened values, kept until the upload below.
    std::deque<GgufTensor> widened;
    std::vector<std::vector<uint8_t>> widened_data;
    auto get = [&](const std::string& n) -> const GgufTensor* {
        const GgufTensor* t = f.find(n);
        if (!t || t->type != MXH_Q1_0 || !t->data) return t;
        for (const GgufTensor& w : widened)
            if (w.name == n) return &w;
        std::vector<uint8_t> buf(t->nbytes * sizeof(float));
        float* d = reinterpret_cast<float*>(buf.data());
        for (size_t i = 0; i < t->nbytes; ++i) d[i] = (float)t->data[i];
        GgufTensor w = *t;
        w.type = MXH_F32;
        w.data = buf.data();
        w.nbytes = buf.size();
        widened_data.push_back(std::move(buf));
        widened.push_back(w);
        return &widened.back();
    };

    mxh_model* m = new mxh_model();
    mxh_model_config& c = m->cfg;
    c.n_layer = (int)f.arch_num("block_count", 0);
    c.n_embd = (int)f.arch_num("embedding_length", 0);
    c.n_head = (int)f.arch_num("attention.head_count", 0);
    c.n_head_kv = (int)f.arch_num("attention.head_count_kv", c.n_head);
    c.n_ff = (int)f.arch_num("feed_forward_length", 0);
    c.eps = (float)f.arch_num("attention.layer_norm_rms_epsilon", 1e-6);
    c.rope_theta = (float)f.arch_num("rope.freq_base", 10000.0);
    c.n_ctx = n_ctx;
    // head width from key_length when present (the reference derives it as
    // n_embd / n_head, minxfmr.cpp:1119-1122, which is wrong for Qwen3-0.6B:
    // 16 heads of 128 over a hidden size of 1024)
    c.head_dim = (int)f.arch_num("attention.key_length", c.n_head > 0 ? c.n_embd / c.n_head : 0);
    m->form = (flags & MXH_MODEL_GGML_FORM) ? MXH_FORM_GGML : MXH_FORM_REF;
    m->neox = (flags & MXH_MODEL_ROPE_NEOX) ? 1 : 0;
    auto fail = [&](int code, const std::string& msg) {
        free_model(m);
        return set_error(code, "model_open: %s", msg.c_str());
    };
    if (c.n_layer <= 0 || c.n_embd <= 0 || c.n_head <= 0 || c.n_head_kv <= 0 || c.n_ff <= 0 || c.head_dim <= 0)
        return fail(MXH_ERR_ARG, "missing architecture metadata");
    if (!attention_supported(c.n_head, c.n_head_kv, c.head_dim))
        return fail(MXH_ERR_UNSUPPORTED, "unsupported head layout (head_dim 32/64/128, at most 8 q heads per kv head)");
    const int qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
    // the decode attention addresses the rows of a layer's cache it reads with
    // 32-bit buffer offsets
    if ((int64_t)(n_ctx + 1) * kvd * 2 >= ((int64_t)1 << 31))
        return fail(MXH_ERR_UNSUPPORTED, "context too long: one layer's K cache window must stay below 2 GiB");

    // --- place every tensor in one HBM blob ---
    std::vector<Placement> place;
    size_t off = 0;
    auto put = [&](const GgufTensor* t) -> size_t {
        off = align_up(off, 256);
        const size_t o = off;
        place.push_back({t, o, nullptr});
        off += t->nbytes;
        return o;
    };
    // contiguous run of same-typed matrices sharing cols -> one fused matrix;
    // with `as_q5k`, Q4_K members are promoted to Q5_K (q4k_as_q5k)
    auto put_run = [&](std::vector<const GgufTensor*> ts, bool as_q5k = false) -> size_t {
        off = align_up(off, 256);
        const size_t o = off;
        for (const GgufTensor* t : ts) {
            if (as_q5k && t->type == MXH_Q4_K) {
                auto conv = q4k_as_q5k(t);
                place.push_back({t, off, conv});
                off += conv->size();
            } else {
                place.push_back({t, off, nullptr});
                off += t->nbytes;
            }
        }
        return o;
    };
    // a mix of Q4_K and Q5_K rows fuses as Q5_K
    auto k45 = [](std::initializer_list<const GgufTensor*> ts) {
        bool any5 = false;
        for (const GgufTensor* t : ts) {
            if (t->type != MXH_Q4_K && t->type != MXH_Q5_K) return false;
            any5 |= t->type == MXH_Q5_K;
        }
        return any5;
    };
    auto need = [&](const std::string& n, int64_t rows, int64_t cols) -> const GgufTensor* {
        const GgufTensor* t = get(n);
        if (!t || !t->data || t->rows() != rows || t->cols() != cols) return nullptr;
        return t;
    };
    const GgufTensor* te = get("token_embd.weight");
    if (!te || !te->data || te->cols() != c.n_embd) return fail(MXH_ERR_ARG, "token_embd.weight missing or misshaped");
    const GgufTensor* to = get("output.weight");
    if (to && (!to->data || to->cols() != c.n_embd)) return fail(MXH_ERR_ARG, "output.weight misshaped");
    const GgufTensor* tn = get("output_norm.weight");
    if (!tn || tn->type != MXH_F32 || tn->cols() != c.n_embd) return fail(MXH_ERR_ARG, "output_norm.weight missing");
    c.n_vocab = (int)(to ? to->rows() : te->rows());
    // every id the head can produce must index the embedding table
    if (c.n_vocab > te->rows()) return fail(MXH_ERR_ARG, "output vocabulary larger than the embedding table");
    const size_t o_embd = put(te);
    const size_t o_out = to ? put(to) : o_embd;
    const size_t o_onorm = put(tn);

    struct LOff {
        size_t qkv, q, k, v, o, gu, g, u, down, an, fn, qn, kn, bias;
        const GgufTensor *tq, *tk, *tv, *to, *tg, *tu, *td, *bq, *bk, *bv;
        bool fq, fqk, fgu;
        int tqkv, tgu;  // storage types of the fused runs
        int64_t promoted;  // bytes added by Q4_K -> Q5_K promotion
    };
    std::vector<LOff> lo((size_t)c.n_layer);
    for (int l = 0; l < c.n_layer; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        LOff& L = lo[(size_t)l];
        L.tq = need(p + "attn_q.weight", qd, c.n_embd);
        L.tk = need(p + "attn_k.weight", kvd, c.n_embd);
        L.tv = need(p + "attn_v.weight", kvd, c.n_embd);
        L.to = need(p + "attn_output.weight", c.n_embd, qd);
        L.tg = need(p + "ffn_gate.weight", c.n_ff, c.n_embd);
        L.tu = need(p + "ffn_up.weight", c.n_ff, c.n_embd);
        L.td = need(p + "ffn_down.weight", c.n_embd, c.n_ff);
        if (!L.tq || !L.tk || !L.tv || !L.to || !L.tg || !L.tu || !L.td)
            return fail(MXH_ERR_ARG, "layer " + std::to_string(l) + ": projection weight missing or misshaped");
        for (const GgufTensor* t : {L.tq, L.tk, L.tv, L.to, L.tg, L.tu, L.td})
            if (!gemv_type_ok(t->type)) return fail(MXH_ERR_UNSUPPORTED, t->name + ": unsupported type " + std::to_string(t->type));
        L.promoted = 0;
        const bool qkv45 = k45({L.tq, L.tk, L.tv});
        L.fq = (L.tq->type == L.tk->type && L.tk->type == L.tv->type) || qkv45;
        L.fqk = !L.fq && L.tq->type == L.tk->type;  // q and k rows share one GEMV, v has its own type
        L.tqkv = qkv45 ? MXH_Q5_K : L.tq->type;
        if (L.fq) {
            L.qkv = put_run({L.tq, L.tk, L.tv}, qkv45);
            if (qkv45)
                for (const GgufTensor* t : {L.tq, L.tk, L.tv})
                    if (t->type == MXH_Q4_K) L.promoted += (int64_t)t->nbytes / 144 * 32;
        } else {
            if (L.fqk) {
                L.q = put_run({L.tq, L.tk});
            } else {
                L.q = put(L.tq);
                L.k = put(L.tk);
            }
            L.v = put(L.tv);
        }
        L.o = put(L.to);
        const bool gu45 = k45({L.tg, L.tu});
        L.fgu = L.tg->type == L.tu->type || gu45;
        L.tgu = gu45 ? MXH_Q5_K : L.tg->type;
        if (L.fgu) {
            L.gu = put_run({L.tg, L.tu}, gu45);
            if (gu45)
                for (const GgufTensor* t : {L.tg, L.tu})
                    if (t->type == MXH_Q4_K) L.promoted += (int64_t)t->nbytes / 144 * 32;
        } else {
            L.g = put(L.tg);
            L.u = put(L.tu);
        }
        L.down = put(L.td);
        auto norm = [&](const std::string& n, int64_t len, bool required, size_t* o) -> bool {
            const GgufTensor* t = get(n);
            if (!t) { *o = SIZE_MAX; return !required; }
            if (t->type != MXH_F32 || t->cols() != len) return false;
            *o = put(t);
            return true;
        };
        if (!norm(p + "attn_norm.weight", c.n_embd, true, &L.an) || !norm(p + "ffn_norm.weight", c.n_embd, true, &L.fn))
            return fail(MXH_ERR_ARG, "layer " + std::to_string(l) + ": norm weights missing");
        if (flags & MXH_MODEL_NO_QK_NORM) {
            L.qn = L.kn = SIZE_MAX;
        } else if (!norm(p + "attn_q_norm.weight", c.head_dim, false, &L.qn) ||
                   !norm(p + "attn_k_norm.weight", c.head_dim, false, &L.kn)) {
            return fail(MXH_ERR_ARG, "layer " + std::to_string(l) + ": QK-norm weights misshaped");
        }
        L.bq = get(p + "attn_q.bias");
        L.bk = get(p + "attn_k.bias");
        L.bv = get(p + "attn_v.bias");
        L.bias = SIZE_MAX;
        if (L.bq || L.bk || L.bv) {
            if (!L.bq || !L.bk || !L.bv || L.bq->type != MXH_F32 || L.bk->type != MXH_F32 || L.bv->type != MXH_F32 ||
                L.bq->cols() != qd || L.bk->cols() != kvd || L.bv->cols() != kvd)
                return fail(MXH_ERR_UNSUPPORTED, "layer " + std::to_string(l) + ": partial or misshaped q/k/v bias");
            L.bias = put_run({L.bq, L.bk, L.bv});
        }
    }
    m->blob_bytes = align_up(off, 256);
    c.weight_bytes = (int64_t)m->blob_bytes;
    if (int rc = dalloc(&m->blob, m->blob_bytes)) { free_model(m); return rc; }
    for (const Placement& p : place)
        if (int rc = check_hip(hipMemcpy(m->blob + p.off, p.conv ? p.conv->data() : p.t->data,
                                         p.conv ? p.conv->size() : p.t->nbytes, hipMemcpyHostToDevice),
                               "weight upload")) {
            free_model(m);
            return rc;
        }
    place.clear();  // the promoted host copies
    widened_data.clear();

    auto dw = [&](size_t o, int type, int64_t rows, int64_t cols) { return DevW{m->blob + o, type, rows, cols}; };
    auto fptr = [&](size_t o) -> const float* { return o == SIZE_MAX ? nullptr : (const float*)(m->blob + o); };
    m->embd = dw(o_embd, te->type, te->rows(), te->cols());
    m->out = to ? dw(o_out, to->type, to->rows(), to->cols()) : m->embd;
    if (!gemv_type_ok(m->out.type)) return fail(MXH_ERR_UNSUPPORTED, "output projection type unsupported");
    m->out_norm = fptr(o_onorm);
    int64_t step_bytes = (int64_t)tensor_bytes(m->out.type, m->out.rows, m->out.cols);
    m->layers.resize((size_t)c.n_layer);
    for (int l = 0; l < c.n_layer; ++l) {
        const LOff& L = lo[(size_t)l];
        Layer& D = m->layers[(size_t)l];
        D.qkv_fused = L.fq;
        if (L.fq) D.qkv = dw(L.qkv, L.tqkv, qd + 2 * kvd, c.n_embd);
        else {
            // with q and k fused, D.q covers both row ranges and D.k is empty
            D.q = dw(L.q, L.tq->type, L.fqk ? qd + kvd : qd, c.n_embd);
            if (!L.fqk) D.k = dw(L.k, L.tk->type, kvd, c.n_embd);
            D.v = dw(L.v, L.tv->type, kvd, c.n_embd);
        }
        D.o = dw(L.o, L.to->type, c.n_embd, qd);
        D.gu_fused = L.fgu;
        if (L.fgu) D.gu = dw(L.gu, L.tgu, 2 * (int64_t)c.n_ff, c.n_embd);
        else {
            D.g = dw(L.g, L.tg->type, c.n_ff, c.n_embd);
            D.u = dw(L.u, L.tu->type, c.n_ff, c.n_embd);
        }
        D.down = dw(L.down, L.td->type, c.n_embd, c.n_ff);
        D.attn_norm = fptr(L.an);
        D.ffn_norm = fptr(L.fn);
        D.q_norm = fptr(L.qn);
        D.k_norm = fptr(L.kn);
        D.bias = fptr(L.bias);
        for (const GgufTensor* t : {L.tq, L.tk, L.tv, L.to, L.tg, L.tu, L.td}) step_bytes += (int64_t)t->nbytes;
        step_bytes += L.promoted;
    }
    c.step_read_bytes = step_bytes;
    c.has_qk_norm = m->layers[0].q_norm != nullptr;
    c.has_bias = m->layers[0].bias != nullptr;
    c.type_wq = lo[0].tq->type;
    c.type_wv = lo[0].tv->type;
    c.type_wffn_down = lo[0].td->type;
    c.type_output = m->out.type;
    c.type_embd = m->embd.type;
    if (!(flags & MXH_MODEL_GGUF_LAYOUT)) {
        // regroup the projection weights into the tiled device layout; the
        // embedding table, read one row per token, keeps the GGUF order, and
        // so does an output projection tied to it
        std::vector<DevW*> ws;
        for (Layer& D : m->layers)
            for (DevW* w : {&D.qkv, &D.q, &D.k, &D.v, &D.o, &D.gu, &D.g, &D.u, &D.down}) ws.push_back(w);
        if (to) {
            ws.push_back(&m->out);
        } else if (tiled_type(m->out.type, m->out.cols) != m->out.type) {
            // a tied output projection reads a tiled copy of the table (the
            // lm-head GEMV streams the whole table every token; Qwen3-0.6B:
            // 51 against about 25 us per token)
            const size_t nb = tensor_bytes(m->out.type, m->out.rows, m->out.cols);
            int rc = dalloc(&m->out_copy, nb);
            if (!rc)
                rc = check_hip(hipMemcpy(m->out_copy, m->out.p, nb, hipMemcpyDeviceToDevice), "output table copy");
            if (rc) {
                free_model(m);
                return rc;
            }
            m->out.p = m->out_copy;
            ws.push_back(&m->out);
        }
        for (DevW* w : ws) {
            const int tt = tiled_type(w->type, w->cols);
            if (!w->p || tt == w->type) continue;
            if (int rc = tile_rows_launch(w->type, const_cast<void*>(w->p), w->rows, w->cols, lib_stream())) {
                free_model(m);
                return set_error(rc, "weight tiling failed");
            }
            w->type = tt;
        }
        if (int rc = check_hip(hipStreamSynchronize(lib_stream()), "weight tiling")) {
            free_model(m);
            return rc;
        }
    }

    // --- caches, RoPE table, activations ---
    // the K and V caches: the reference's ring of n_ctx rows as n_ctx + 1
    // slots stored twice (AttnArgs::ring)
    const size_t kv_per_layer = 2 * ((size_t)n_ctx + 1) * kvd;
    int rc = dalloc(&m->kv, 2 * kv_per_layer * (size_t)c.n_layer);
    for (int l = 0; l < c.n_layer && !rc; ++l) {
        m->layers[(size_t)l].kc = m->kv + (size_t)(2 * l) * kv_per_layer;
        m->layers[(size_t)l].vc = m->kv + (size_t)(2 * l + 1) * kv_per_layer;
    }
    const int half = c.head_dim / 2;
    if (!rc) {
        // cos/sin of pos * theta^(-2i/rot) in double, as rope.cpp:26-31 computes them
        // (positions 0 .. n_ctx: past a full ring RoPE stays at n_ctx)
        std::vector<double> cs(((size_t)n_ctx + 1) * half * 2);
        for (int i = 0; i < half; ++i) {
            const double inv_freq = 1.0 / std::pow((double)c.rope_theta, (2.0 * (double)i) / (double)c.head_dim);
            for (int p = 0; p <= n_ctx; ++p) {
                const double ang = (double)p * inv_freq;
                cs[((size_t)p * half + i) * 2] = std::cos(ang);
                cs[((size_t)p * half + i) * 2 + 1] = std::sin(ang);
            }
        }
        rc = dalloc(&m->rope_cs, cs.size());
        if (!rc) rc = check_hip(hipMemcpy(m->rope_cs, cs.data(), cs.size() * sizeof(double), hipMemcpyHostToDevice), "rope table");
    }
    if (!rc) rc = dalloc(&m->x, (size_t)c.n_embd);
    if (!rc) rc = dalloc(&m->xn, (size_t)std::max(c.n_embd, c.n_ff));
    if (!rc) rc = dalloc(&m->qkv, (size_t)(qd + 2 * kvd));
    if (!rc) rc = dalloc(&m->att, (size_t)qd);
    if (!rc) rc = dalloc(&m->gu, 2 * (size_t)c.n_ff);
    if (!rc) rc = dalloc(&m->h, (size_t)c.n_ff);
    if (!rc) rc = dalloc(&m->logits, (size_t)c.n_vocab);
    if (!rc) rc = dalloc(&m->part, attention_scratch_floats(c.n_head, c.n_head_kv, c.head_dim, n_ctx));
    if (!rc)
        rc = check_hip(hipMemset(m->part, 0, sizeof(float) * attention_scratch_floats(c.n_head, c.n_head_kv,
                                                                                       c.head_dim, n_ctx)),
                       "attention partials init");
    if (!rc) rc = dalloc(&m->trace, (size_t)(c.n_layer + 1) * c.n_embd);
    // the id history outlives the ring: up to 2^20 ids (or n_ctx + 1)
    m->token_cap = std::max(n_ctx + 1, 1 << 20);
    if (!rc) rc = dalloc(&m->tokens, (size_t)m->token_cap);
    if (!rc) rc = dalloc(&m->pos, 1);
    // >= workgroups of the head GEMV: at most one per row group (>= 2 rows)
    // and never more than the resident grid
    m->red_cap = c.n_vocab / 2 + 2 < 8192 ? c.n_vocab / 2 + 2 : 8192;
    if (!rc) rc = dalloc(&m->red_val, (size_t)m->red_cap);
    if (!rc) rc = dalloc(&m->red_idx, (size_t)m->red_cap);
    if (!rc) rc = dalloc(&m->sprm, 1);
    if (!rc) rc = dalloc(&m->scand, std::max(sample_scratch_keys(c.n_vocab, 64), (size_t)4096));
    if (!rc) rc = check_hip(hipMemset(m->sprm, 0, sizeof(SampleParams)), "sampler init");
    if (!rc) rc = dalloc(&m->eprm, 1);
    if (!rc) rc = dalloc(&m->esup, (size_t)c.n_vocab);
    if (!rc) rc = dalloc(&m->ecnt, (size_t)c.n_vocab);
    if (!rc) rc = check_hip(hipMemset(m->eprm, 0, sizeof(EditParams)), "edit params init");
    if (!rc) rc = check_hip(hipMemset(m->ecnt, 0, sizeof(int) * (size_t)c.n_vocab), "edit counts init");
    if (!rc) rc = check_hip(hipMemset(m->tokens, 0, sizeof(int) * (size_t)m->token_cap), "token init");
    if (!rc) rc = check_hip(hipMemset(m->pos, 0, sizeof(int)), "position init");
    if (!rc) rc = check_hip(hipDeviceSynchronize(), "model init");
    if (rc) {
        free_model(m);
        return rc;
    }
    m->token_prefill = (flags & MXH_MODEL_TOKEN_PREFILL) != 0;
    m->bf16_prefill = (flags & MXH_MODEL_BF16_PREFILL) != 0;
    if (!(flags & MXH_MODEL_NO_GRAPH)) {
        if ((rc = capture(m, false, false, &m->g_prefill)) || (rc = capture(m, true, false, &m->g_decode))) {
            free_model(m);
            return rc;
        }
    }
    *out = m;
    return MXH_OK;
}

int mxh_model_config_get(const mxh_model* m, mxh_model_config* cfg) {
    if (!m || !cfg) return set_error(MXH_ERR_ARG, "config_get: null argument");
    *cfg = m->cfg;
    return MXH_OK;
}

int mxh_model_reset(mxh_model* m) {
    if (!m) return set_error(MXH_ERR_ARG, "reset: null model");
    m->host_pos = 0;
    const int zero = 0;
    const uint64_t zero64 = 0;
    if (int rc = check_hip(hipMemcpyAsync(m->pos, &zero, sizeof(int), hipMemcpyHostToDevice, lib_stream()), "reset"))
        return rc;
    if (int rc = check_hip(hipMemcpyAsync(&m->sprm->draws, &zero64, sizeof(uint64_t), hipMemcpyHostToDevice,
                                          lib_stream()), "reset"))
        return rc;
    return check_hip(hipStreamSynchronize(lib_stream()), "reset");
}

int mxh_model_position(const mxh_model* m) { return m ? m->host_pos : -1; }

namespace {

// One step at position pos (the device position when it runs)
int run_step(mxh_model* m, bool with_head, int pos) {
    hipStream_t st = lib_stream();
    const bool wrapped = pos >= m->cfg.n_ctx;
    hipGraphExec_t g = with_head ? (m->sampling ? m->g_sample : m->g_decode) : m->g_prefill;
    if (m->trace_on || !g) return enqueue_step(m, with_head, wrapped, st);
    if (wrapped) {
        hipGraphExec_t* w = with_head ? (m->sampling ? &m->g_sample_w : &m->g_decode_w) : &m->g_prefill_w;
        if (!*w) {
            if (int rc = check_hip(hipStreamSynchronize(st), "ring graph")) return rc;
            if (int rc = capture(m, with_head, true, w)) return rc;
        }
        g = *w;
    }
    return check_hip(hipGraphLaunch(g, st), "graph launch");
}

}  // namespace

int mxh_model_step(mxh_model* m, int token, float* logits, float* trace) {
    if (!m) return set_error(MXH_ERR_ARG, "step: null model");
    if (token < 0 || token >= m->embd.rows) return set_error(MXH_ERR_ARG, "step: token %d out of range", token);
    if (m->host_pos + 1 >= m->token_cap)
        return set_error(MXH_ERR_ARG, "step: the id history of %d tokens is full", m->token_cap);
    hipStream_t st = lib_stream();
    if (int rc = check_hip(hipMemcpyAsync(m->tokens + m->host_pos, &token, sizeof(int), hipMemcpyHostToDevice, st), "token"))
        return rc;
    m->trace_on = trace != nullptr;
    int rc = run_step(m, true, m->host_pos);
    m->trace_on = false;
    if (rc) return rc;
    m->host_pos++;
    if (logits && (rc = check_hip(hipMemcpyAsync(logits, m->logits, sizeof(float) * m->cfg.n_vocab, hipMemcpyDeviceToHost, st), "logits")))
        return rc;
    if (trace && (rc = check_hip(hipMemcpyAsync(trace, m->trace, sizeof(float) * (m->cfg.n_layer + 1) * m->cfg.n_embd,
                                                hipMemcpyDeviceToHost, st), "trace")))
        return rc;
    return check_hip(hipStreamSynchronize(st), "step");
}

namespace {

constexpr int kPrefillRows = 512;  // tokens per batched prefill chunk

int ensure_prefill_buffers(mxh_model* m) {
    if (m->pf_rows) return MXH_OK;
    const mxh_model_config& c = m->cfg;
    const int rows = std::min(kPrefillRows, c.n_ctx);
    const size_t qd = (size_t)c.n_head * c.head_dim, kvd = (size_t)c.n_head_kv * c.head_dim;
    const size_t widest = std::max(std::max((size_t)c.n_embd, qd), (size_t)c.n_ff);
    int rc = dalloc(&m->pf_x, (size_t)rows * c.n_embd);
    if (!rc) rc = dalloc(&m->pf_qkv, (size_t)rows * (qd + 2 * kvd));
    if (!rc) rc = dalloc(&m->pf_q, (size_t)rows * qd);
    if (!rc) rc = dalloc(&m->pf_att, (size_t)rows * qd);
    if (!rc) rc = dalloc(&m->pf_gu, (size_t)rows * 2 * c.n_ff);
    if (!rc) rc = dalloc(&m->pf_a, (size_t)rows * widest);
    if (!rc) rc = dalloc(&m->pf_a_lo, (size_t)rows * widest);
    if (!rc) rc = dalloc(&m->pf_h16, (size_t)rows * widest);
    if (!rc) rc = dalloc(&m->pf_l16, (size_t)rows * widest);
    if (!rc) rc = dalloc(&m->pf_sh, (size_t)rows * (widest / 32));
    if (!rc) rc = dalloc(&m->pf_sl, (size_t)rows * (widest / 32));
    if (!rc) rc = dalloc(&m->pf_rscale, (size_t)rows);
    // split-K partials: up to 4 splits of the narrower outputs (x, q|k|v)
    m->pf_part_floats = 4 * (size_t)rows * std::max((size_t)c.n_embd, qd + 2 * kvd);
    if (!rc) rc = dalloc(&m->pf_part, m->pf_part_floats);
    if (!rc) m->pf_rows = rows;
    return rc;
}

// Which input form a prefill GEMM reads: the exact-weight fp16 kernel for
// Q4_K, Q5_K, Q8_0 and Q5_0 rows (pf_h16 / pf_l16 / pf_sh / pf_sl /
// pf_rscale), the split-bf16 kernel otherwise (F32 rows, rows whose length
// is not a multiple of 256, or MXH_MODEL_BF16_PREFILL; pf_a, pf_a_lo).
bool f16_gemm(const mxh_model* m, const DevW& w) {
    return w.p && !m->bf16_prefill && gemm_q_f16_supported(w.type, (int)w.cols);
}

int gemm(mxh_model* m, const DevW& w, int lda, float* out, int ldo, const float* res, int rows, hipStream_t st) {
    if (f16_gemm(m, w))
        return gemm_q_f16_run(w.type, m->pf_h16, m->pf_l16, lda, m->pf_sh, m->pf_sl, lda / 32, m->pf_rscale, w.p,
                                out, ldo, res, rows, (int)w.rows, (int)w.cols, m->form, m->pf_part,
                                m->pf_part_floats, st);
    return gemm_bf16_run(w.type, m->pf_a, m->pf_a_lo, lda, w.p, out, ldo, res, rows, (int)w.rows, (int)w.cols,
                         m->form, m->pf_part, m->pf_part_floats, st);
}

// GEMM inputs from rows of x (normed with nw when given) in the forms the
// consumers `ws` read
int prep_rows(mxh_model* m, std::initializer_list<const DevW*> ws, const float* x, int ldx, const float* nw, float eps,
              int k, int rows, hipStream_t st) {
    bool need16 = false, needbf = false;
    for (const DevW* w : ws)
        if (w->p) (f16_gemm(m, *w) ? need16 : needbf) = true;
    int rc = MXH_OK;
    if (need16)
        rc |= rows_to_f16_launch(x, ldx, nw, eps, k, m->pf_h16, m->pf_l16, k, m->pf_sh, m->pf_sl, k / 32, m->pf_rscale,
                                 rows, st);
    if (needbf) rc |= rows_to_bf16_launch(x, ldx, nw, eps, k, m->pf_a, m->pf_a_lo, k, rows, st);
    return rc;
}

// Prompt tokens tokens[p0 .. p0+rows) through every layer at once, the
// projections on the matrix cores (split-bf16 inputs, fp32 accumulation); the K/V
// rows land in the cache and the position advances by `rows`.  No head: the
// last prompt token runs through the decode step for its logits.
int enqueue_prefill_chunk(mxh_model* m, int p0, int rows, hipStream_t st) {
    const mxh_model_config& c = m->cfg;
    const int d = c.n_embd, hd = c.head_dim, nh = c.n_head, nkv = c.n_head_kv, f = c.n_ff;
    const int qd = nh * hd, kvd = nkv * hd, ldq = qd + 2 * kvd;
    int rc = embed_rows_launch(m->embd.type, m->embd.p, m->tokens, p0, rows, m->pf_x, d, m->form, st);
    for (int l = 0; l < c.n_layer && !rc; ++l) {
        const Layer& L = m->layers[(size_t)l];
        rc |= prep_rows(m, {&L.qkv, &L.q, &L.k, &L.v}, m->pf_x, d, L.attn_norm, c.eps, d, rows, st);
        if (L.qkv_fused) {
            rc |= gemm(m, L.qkv, d, m->pf_qkv, ldq, nullptr, rows, st);
        } else {
            rc |= gemm(m, L.q, d, m->pf_qkv, ldq, nullptr, rows, st);
            if (L.k.p) rc |= gemm(m, L.k, d, m->pf_qkv + qd, ldq, nullptr, rows, st);
            rc |= gemm(m, L.v, d, m->pf_qkv + qd + kvd, ldq, nullptr, rows, st);
        }
        rc |= qkv_prep_rows_launch(m->pf_qkv, ldq, L.bias, L.q_norm, L.k_norm, m->rope_cs, p0, rows, m->pf_q, L.kc,
                                   L.vc, nh, nkv, hd, m->neox, c.eps, st);
        rc |= attention_rows_mfma_launch(m->pf_q, L.kc, L.vc, m->pf_att, p0, rows, nh, nkv, hd, 1.0f / sqrtf((float)hd),
                                          st);
        rc |= prep_rows(m, {&L.o}, m->pf_att, qd, nullptr, 0.f, qd, rows, st);
        rc |= gemm(m, L.o, qd, m->pf_x, d, m->pf_x, rows, st);
        rc |= prep_rows(m, {&L.gu, &L.g, &L.u}, m->pf_x, d, L.ffn_norm, c.eps, d, rows, st);
        if (L.gu_fused) {
            rc |= gemm(m, L.gu, d, m->pf_gu, 2 * f, nullptr, rows, st);
        } else {
            rc |= gemm(m, L.g, d, m->pf_gu, 2 * f, nullptr, rows, st);
            rc |= gemm(m, L.u, d, m->pf_gu + f, 2 * f, nullptr, rows, st);
        }
        if (f16_gemm(m, L.down))
            rc |= silu_mul_f16_launch(m->pf_gu, f, m->pf_h16, m->pf_l16, m->pf_sh, m->pf_sl, m->pf_rscale, rows, st);
        else
            rc |= silu_mul_bf16_launch(m->pf_gu, f, m->pf_a, m->pf_a_lo, rows, st);
        rc |= gemm(m, L.down, f, m->pf_x, d, m->pf_x, rows, st);
    }
    if (!rc) rc = add_int_launch(m->pos, rows, st);
    return rc ? set_error(MXH_ERR_HIP, "prefill enqueue failed") : MXH_OK;
}

bool batched_prefill_supported(const mxh_model* m) {
    const mxh_model_config& c = m->cfg;
    return !m->token_prefill && c.n_embd % 64 == 0 && c.n_ff % 64 == 0 && (c.n_head * c.head_dim) % 64 == 0;
}

// Prompt tokens tokens[p .. p + n) (already on the device) without logits,
// the device position at p: in batched chunks while the cache has room for
// them, token by token past a full cache (every step of the ring is its own:
// RoPE and the rows attended depend on what the step before evicted), and
// token by token throughout with MXH_MODEL_TOKEN_PREFILL.
int run_prefill(mxh_model* m, int p, int n) {
    if (n <= 0) return MXH_OK;
    const int batched = batched_prefill_supported(m) ? std::max(0, std::min(n, m->cfg.n_ctx - p)) : 0;
    if (batched > 0) {
        if (int rc = ensure_prefill_buffers(m)) return rc;
        hipStream_t st = lib_stream();
        for (int done = 0; done < batched;) {
            const int rows = std::min(m->pf_rows, batched - done);
            if (int rc = enqueue_prefill_chunk(m, p + done, rows, st)) return rc;
            done += rows;
        }
    }
    for (int i = batched; i < n; ++i)
        if (int rc = run_step(m, false, p + i)) return rc;
    return MXH_OK;
}

}  // namespace

int mxh_model_set_sampling(mxh_model* m, int top_k, double temperature, double top_p, double min_p, uint64_t seed) {
    if (!m) return set_error(MXH_ERR_ARG, "set_sampling: null model");
    if (temperature > 0.0 && (top_k < 1 || top_k > kSampleTopKMax))
        return set_error(MXH_ERR_ARG, "set_sampling: top_k %d outside 1..%d", top_k, kSampleTopKMax);
    hipStream_t st = lib_stream();
    if (int rc = check_hip(hipStreamSynchronize(st), "set_sampling")) return rc;
    if (!(temperature > 0.0)) {
        m->sampling = false;
        return MXH_OK;
    }
    if (top_k > m->cfg.n_vocab) top_k = m->cfg.n_vocab;  // the reference clamps k to the vocabulary
    SampleParams h{};
    h.top_k = top_k;
    h.temperature = temperature;
    h.top_p = top_p;
    h.min_p = min_p;
    h.seed = seed;
    h.draws = 0;
    if (int rc = check_hip(hipMemcpy(m->sprm, &h, sizeof(h), hipMemcpyHostToDevice), "sampler params")) return rc;
    const bool recapture = m->g_decode && (!m->g_sample || top_k != m->top_k);
    m->top_k = top_k;
    m->sampling = true;
    if (recapture) {
        drop_graph(m->g_sample);
        drop_graph(m->g_sample_w);
        if (int rc = capture(m, true, false, &m->g_sample)) {
            m->sampling = false;
            return rc;
        }
    }
    return MXH_OK;
}

int mxh_model_set_logit_edits(mxh_model* m, const int* suppress, int n_suppress, int repeat_last_n,
                              double repeat_penalty, double frequency_penalty, double presence_penalty) {
    if (!m || n_suppress < 0 || (n_suppress > 0 && !suppress))
        return set_error(MXH_ERR_ARG, "set_logit_edits: bad arguments");
    if (n_suppress > m->cfg.n_vocab) return set_error(MXH_ERR_ARG, "set_logit_edits: %d ids exceed the vocabulary", n_suppress);
    if (!(repeat_penalty > 0.0) || !std::isfinite(repeat_penalty) || !std::isfinite(frequency_penalty) ||
        !std::isfinite(presence_penalty))
        return set_error(MXH_ERR_ARG, "set_logit_edits: penalties must be finite, repeat_penalty > 0");
    hipStream_t st = lib_stream();
    if (int rc = check_hip(hipStreamSynchronize(st), "set_logit_edits")) return rc;
    EditParams h{};
    h.last_n = repeat_last_n;
    h.n_suppress = n_suppress;
    h.repeat_penalty = repeat_penalty;
    h.frequency_penalty = frequency_penalty;
    h.presence_penalty = presence_penalty;
    if (int rc = check_hip(hipMemcpy(m->eprm, &h, sizeof(h), hipMemcpyHostToDevice), "edit params")) return rc;
    if (n_suppress > 0)
        if (int rc = check_hip(hipMemcpy(m->esup, suppress, sizeof(int) * (size_t)n_suppress, hipMemcpyHostToDevice),
                               "suppressed ids"))
            return rc;
    // the reference skips its penalty pass when the window is empty or every
    // penalty is neutral (minxfmr.cpp:2065)
    const bool pen = repeat_last_n != 0 && (repeat_penalty != 1.0 || frequency_penalty != 0.0 || presence_penalty != 0.0);
    const bool want = n_suppress > 0 || pen;
    if (want == m->edits) return MXH_OK;
    m->edits = want;
    // the decode graphs hold the head's form: capture them again (each in
    // its own mode: capture() records the current `sampling` choice)
    const bool sampling = m->sampling;
    int rc = MXH_OK;
    drop_graph(m->g_decode_w);
    drop_graph(m->g_sample_w);
    if (m->g_decode) {
        drop_graph(m->g_decode);
        m->sampling = false;
        rc = capture(m, true, false, &m->g_decode);
    }
    if (!rc && m->g_sample) {
        drop_graph(m->g_sample);
        m->sampling = true;
        rc = capture(m, true, false, &m->g_sample);
    }
    m->sampling = sampling;
    return rc;
}

int mxh_model_prefill(mxh_model* m, const int* tokens, int n) {
    if (!m || (!tokens && n > 0) || n < 0) return set_error(MXH_ERR_ARG, "prefill: bad arguments");
    if ((int64_t)m->host_pos + n >= m->token_cap)
        return set_error(MXH_ERR_ARG, "prefill: position %d + %d exceeds the id history of %d", m->host_pos, n,
                         m->token_cap);
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->embd.rows) return set_error(MXH_ERR_ARG, "prefill: id %d out of range", tokens[i]);
    if (n == 0) return MXH_OK;
    hipStream_t st = lib_stream();
    int rc = check_hip(hipMemcpyAsync(m->tokens + m->host_pos, tokens, sizeof(int) * n, hipMemcpyHostToDevice, st),
                       "prefill ids");
    if (!rc) rc = run_prefill(m, m->host_pos, n);
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "prefill");
    if (!rc) m->host_pos += n;
    return rc;
}

int mxh_model_generate(mxh_model* m, const int* prompt, int n_prompt, int n_gen, int* out, float* prefill_ms,
                       float* decode_ms) {
    if (!m || !prompt || n_prompt <= 0 || n_gen <= 0 || !out) return set_error(MXH_ERR_ARG, "generate: bad arguments");
    if ((int64_t)n_prompt + n_gen >= m->token_cap)
        return set_error(MXH_ERR_ARG, "generate: %d + %d tokens exceed the id history of %d", n_prompt, n_gen,
                         m->token_cap);
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= m->embd.rows) return set_error(MXH_ERR_ARG, "generate: prompt id %d out of range", prompt[i]);
    if (int rc = mxh_model_reset(m)) return rc;
    hipStream_t st = lib_stream();
    hipEvent_t e0, e1, e2;
    if (int rc = check_hip(hipEventCreate(&e0), "event")) return rc;
    (void)hipEventCreate(&e1);
    (void)hipEventCreate(&e2);
    int rc = check_hip(hipMemcpyAsync(m->tokens, prompt, sizeof(int) * n_prompt, hipMemcpyHostToDevice, st), "prompt");
    // the chunk buffers are allocated once per model, before the timed window
    if (!rc && n_prompt > 1 && batched_prefill_supported(m)) rc = ensure_prefill_buffers(m);
    if (!rc) rc = check_hip(hipEventRecord(e0, st), "event");
    // prompt positions 0 .. n_prompt-2 need no logits (batched on the
    // matrix cores, or token by token); the last prompt token runs with the
    // head and yields the first generated id (minxfmr.cpp:1860)
    if (!rc) rc = run_prefill(m, 0, n_prompt - 1);
    if (!rc) rc = check_hip(hipEventRecord(e1, st), "event");
    for (int i = 0; i < n_gen && !rc; ++i) rc = run_step(m, true, n_prompt - 1 + i);
    if (!rc) rc = check_hip(hipEventRecord(e2, st), "event");
    if (!rc) rc = check_hip(hipMemcpyAsync(out, m->tokens + n_prompt, sizeof(int) * n_gen, hipMemcpyDeviceToHost, st), "ids");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "generate");
    if (!rc) {
        m->host_pos = n_prompt + n_gen - 1;
        float ms = 0.f;
        if (prefill_ms) { (void)hipEventElapsedTime(&ms, e0, e1); *prefill_ms = ms; }
        if (decode_ms) { (void)hipEventElapsedTime(&ms, e1, e2); *decode_ms = ms; }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipEventDestroy(e2);
    return rc;
}

int mxh_model_decode(mxh_model* m, int n_gen, int* out, float* decode_ms) {
    if (!m || n_gen <= 0) return set_error(MXH_ERR_ARG, "decode: bad arguments");
    const int p0 = m->host_pos;
    if ((int64_t)p0 + n_gen >= m->token_cap)
        return set_error(MXH_ERR_ARG, "decode: position %d + %d exceeds the id history of %d", p0, n_gen,
                         m->token_cap);
    hipStream_t st = lib_stream();
    hipEvent_t e0, e1;
    if (int rc = check_hip(hipEventCreate(&e0), "event")) return rc;
    (void)hipEventCreate(&e1);
    int rc = check_hip(hipEventRecord(e0, st), "event");
    for (int i = 0; i < n_gen && !rc; ++i) rc = run_step(m, true, p0 + i);
    if (!rc) rc = check_hip(hipEventRecord(e1, st), "event");
    if (!rc && out) rc = check_hip(hipMemcpyAsync(out, m->tokens + p0 + 1, sizeof(int) * n_gen, hipMemcpyDeviceToHost, st), "ids");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "decode");
    if (!rc) {
        m->host_pos = p0 + n_gen;
        if (decode_ms) (void)hipEventElapsedTime(decode_ms, e0, e1);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int mxh_model_set_token(mxh_model* m, int token) {
    if (!m) return set_error(MXH_ERR_ARG, "set_token: null model");
    if (token < 0 || token >= m->embd.rows) return set_error(MXH_ERR_ARG, "set_token: token %d out of range", token);
    // the history holds token_cap ids and every step leaves host_pos below
    // it, so the current position indexes it
    hipStream_t st = lib_stream();
    int rc = check_hip(hipMemcpyAsync(m->tokens + m->host_pos, &token, sizeof(int), hipMemcpyHostToDevice, st), "token");
    if (!rc) rc = check_hip(hipStreamSynchronize(st), "set_token");
    return rc;
}

int mxh_model_bench_gemv(mxh_model* m, int type, int reps, float* ms, int64_t* launches, int64_t* bytes) {
    if (!m || reps <= 0 || !ms) return set_error(MXH_ERR_ARG, "bench_gemv: bad arguments");
    hipStream_t st = lib_stream();
    const mxh_model_config& c = m->cfg;
    const int qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
    // every GEMV of `type` in the form the decode step launches it (fused
    // norms, SwiGLU and residual epilogues), outputs into scratch vectors so
    // the model's state is left as it was; the lm-head in plain mode
    struct Job {
        const DevW* w;
        const float *x, *res, *nw;
        float* y;
        int mode;
    };
    std::vector<Job> jobs;
    auto add = [&](const DevW& w, const float* x, float* y, const float* res, const float* nw, int mode) {
        if (w.p && storage_type(w.type) == type) jobs.push_back(Job{&w, x, res, nw, y, mode});
    };
    for (const Layer& L : m->layers) {
        add(L.qkv, m->x, m->qkv, nullptr, L.attn_norm, GEMV_PLAIN);
        add(L.q, m->x, m->qkv, nullptr, L.attn_norm, GEMV_PLAIN);
        add(L.k, m->x, m->qkv + qd, nullptr, L.attn_norm, GEMV_PLAIN);
        add(L.v, m->x, m->qkv + qd + kvd, nullptr, L.attn_norm, GEMV_PLAIN);
        add(L.o, m->att, m->xn, m->x, nullptr, o_merges(m, L.o) ? GEMV_ATTN : GEMV_PLAIN);
        add(L.gu, m->x, m->h, nullptr, L.ffn_norm, GEMV_SILU);
        add(L.g, m->x, m->gu, nullptr, L.ffn_norm, GEMV_PLAIN);
        add(L.u, m->x, m->gu + c.n_ff, nullptr, L.ffn_norm, GEMV_PLAIN);
        add(L.down, m->h, m->xn, m->x, nullptr, GEMV_PLAIN);
    }
    add(m->out, m->x, m->logits, nullptr, m->out_norm, GEMV_PLAIN);
    if (jobs.empty()) return set_error(MXH_ERR_ARG, "bench_gemv: model has no matrices of type %d", type);
    int64_t b = 0;
    for (const Job& j : jobs) b += (int64_t)row_bytes(j.w->type, j.w->cols) * j.w->rows + 4 * (j.w->rows + j.w->cols);
    hipEvent_t e0, e1;
    if (int rc = check_hip(hipEventCreate(&e0), "event")) return rc;
    (void)hipEventCreate(&e1);
    int rc = check_hip(hipEventRecord(e0, st), "event");
    for (int r = 0; r < reps && !rc; ++r)
        for (const Job& j : jobs) {
            rc = gemv(*j.w, j.x, j.y, j.res, m->form, st, j.nw, c.eps, j.mode, m);
            if (rc) break;
        }
    if (!rc) rc = check_hip(hipEventRecord(e1, st), "event");
    if (!rc) rc = check_hip(hipEventSynchronize(e1), "bench_gemv");
    if (!rc) {
        (void)hipEventElapsedTime(ms, e0, e1);
        if (launches) *launches = (int64_t)jobs.size() * reps;
        if (bytes) *bytes = b * reps;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int mxh_model_bench_attention(mxh_model* m, int reps, float* ms, int64_t* launches, int64_t* bytes) {
    if (!m || reps <= 0 || !ms) return set_error(MXH_ERR_ARG, "bench_attention: bad arguments");
    if (m->host_pos < 1) return set_error(MXH_ERR_ARG, "bench_attention: position %d has no cached rows", m->host_pos);
    hipStream_t st = lib_stream();
    const mxh_model_config& c = m->cfg;
    const int splits = attention_splits(c.n_ctx, c.n_head, c.n_head_kv, c.head_dim);
    const bool merge = splits > kAttnMaxSplits;  // the grouped kernel's partials go through the merge kernel
    hipEvent_t e0, e1;
    if (int rc = check_hip(hipEventCreate(&e0), "event")) return rc;
    (void)hipEventCreate(&e1);
    int rc = check_hip(hipEventRecord(e0, st), "event");
    for (int r = 0; r < reps && !rc; ++r)
        for (const Layer& L : m->layers) {
            rc = attention_run(attn_args(m, L, m->host_pos >= c.n_ctx), c.n_ctx, st);
            if (!rc && merge) rc = attention_merge_launch(m->part, splits, c.n_head, c.head_dim, m->att, st);
            if (rc) break;
        }
    if (!rc) rc = check_hip(hipEventRecord(e1, st), "event");
    if (!rc) rc = check_hip(hipEventSynchronize(e1), "bench_attention");
    if (!rc) rc = check_hip(hipEventElapsedTime(ms, e0, e1), "event");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc) return rc;
    // the K and V rows read: the cached ones (at most the ring's n_ctx; the
    // current row comes from q|k|v)
    const int64_t per = 2 * (int64_t)std::min(m->host_pos, c.n_ctx) * c.n_head_kv * c.head_dim * 2;
    if (launches) *launches = (int64_t)reps * c.n_layer;
    if (bytes) *bytes = per * reps * c.n_layer;
    return MXH_OK;
}

void mxh_model_close(mxh_model* m) { free_model(m); }

// No C++ exception crosses the C ABI: allocation failures and anything else
// a malformed file may raise come back as status codes.
int mxh_model_open(const char* gguf_path, int n_ctx, int flags, mxh_model** out) {
    try {
        return model_open_impl(gguf_path, n_ctx, flags, out);
    } catch (const std::bad_alloc&) {
        return set_error(MXH_ERR_OOM, "model_open: host allocation failed");
    } catch (const std::exception& e) {
        return set_error(MXH_ERR_ARG, "model_open: %s", e.what());
    } catch (...) {
        return set_error(MXH_ERR_ARG, "model_open: unexpected failure");
    }
}

static int write_synthetic_impl(const char* path, const mxh_synth_arch* a, uint64_t seed, int threads);

int mxh_write_synthetic_gguf(const char* path, const mxh_synth_arch* a, uint64_t seed, int threads) {
    try {
        return write_synthetic_impl(path, a, seed, threads);
    } catch (const std::bad_alloc&) {
        return set_error(MXH_ERR_OOM, "write_synthetic_gguf: host allocation failed");
    } catch (const std::exception& e) {
        return set_error(MXH_ERR_ARG, "write_synthetic_gguf: %s", e.what());
    } catch (...) {
        return set_error(MXH_ERR_ARG, "write_synthetic_gguf: unexpected failure");
    }
}

static int write_synthetic_impl(const char* path, const mxh_synth_arch* a, uint64_t seed, int threads) {
    if (!path || !a || !a->arch) return set_error(MXH_ERR_ARG, "write_synthetic_gguf: null argument");
    SynthArch s;
    s.arch = a->arch;
    s.n_layer = a->n_layer; s.n_embd = a->n_embd; s.n_head = a->n_head; s.n_head_kv = a->n_head_kv;
    s.head_dim = a->head_dim; s.n_ff = a->n_ff; s.n_vocab = a->n_vocab; s.ctx = a->ctx;
    s.rope_theta = a->rope_theta; s.eps = a->eps; s.qk_norm = a->qk_norm; s.tied = a->tied;
    s.wtype = a->wtype; s.out_type = a->out_type; s.embd_type = a->embd_type;
    s.attn_v_type = a->attn_v_type; s.ffn_down_type = a->ffn_down_type;
    std::string err;
    if (!write_synthetic_gguf(path, s, seed, threads, &err)) return set_error(MXH_ERR_ARG, "%s", err.c_str());
    return MXH_OK;
}

}  // extern "C"
