// ref_shim.cpp — TEST INFRASTRUCTURE ONLY.
//
// extern "C" entry points over the reference's own CPU sources, compiled in
// place from /root/reference by oracle/Makefile into oracle/_ref/.  Used by
// tests to pin the oracle (mxo.c) against the real reference arithmetic.
// Nothing here is shipped in the product library.
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

#include "backend/backend_runtime.h"
#include "cache/kv_cache.h"
#include "tensor/tensor.h"
#include "transformer/rmsnorm.h"
#include "transformer/rope.h"
#include "transformer/softmax.h"
#include "transformer/transformer.h"
#include "backend/backend_context.h"
#include "../third_party/gguf/gguf_reader.h"

namespace {

// GGUF type id -> reference DataType (tensor.h:5-14); -1 if unsupported.
int to_dtype(int ggml_type, DataType* out) {
    switch (ggml_type) {
    case 0: *out = DataType::F32; return 0;
    case 6: *out = DataType::Q5_0; return 0;
    case 8: *out = DataType::Q8_0; return 0;
    case 12: *out = DataType::Q4_K; return 0;
    }
    return -1;
}

void bind(Tensor& t, int type, const void* data, size_t rows, size_t cols) {
    DataType dt = DataType::F32;
    to_dtype(type, &dt);
    t.data = const_cast<void*>(data);
    t.type = dt;
    t.rows = rows;
    t.cols = cols;
    size_t rb = cols * 4;
    if (dt == DataType::Q4_K) rb = tensor_q4_k_row_bytes(cols);
    if (dt == DataType::Q8_0) rb = tensor_q8_0_row_bytes(cols);
    if (dt == DataType::Q5_0) rb = tensor_q5_0_row_bytes(cols);
    t.bytes = rb * rows;
}

void ensure_cpu() {
    static bool done = false;
    if (!done) {
        backend_set_kind(BackendKind::CPU);
        done = true;
    }
}

}  // namespace

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return tensor_fp16_to_fp32(h); }

int ref_dequant_block(int type, const uint8_t* blk, float* out) {
    switch (type) {
    case 12: tensor_dequant_q4_k_block(blk, out); return 0;
    case 8: tensor_dequant_q8_0_block(blk, out); return 0;
    case 6: tensor_dequant_q5_0_block(blk, out); return 0;
    }
    return -1;
}

int ref_matmul_rhs_t(int type, const float* A, size_t M, size_t K, const void* B, size_t N, float* out) {
    ensure_cpu();
    DataType dt;
    if (to_dtype(type, &dt) != 0) return -1;
    Tensor a, b, o;
    bind(a, 0, A, M, K);
    bind(b, type, B, N, K);
    bind(o, 0, out, M, N);
    return backend_matmul_rhs_transposed(&a, &b, &o) ? 0 : -2;
}

int ref_rmsnorm(const float* x, float* y, size_t rows, size_t n, float eps) {
    Tensor a, b;
    bind(a, 0, x, rows, n);
    bind(b, 0, y, rows, n);
    return rmsnorm_forward(&a, &b, eps) ? 0 : -1;
}

void ref_rope(float* v, size_t rows, size_t n_heads, size_t head_dim, size_t n_rot, size_t start_pos, float theta,
              int neox) {
    backend_context().rope_neox = neox != 0;
    Tensor t;
    bind(t, 0, v, rows, n_heads * head_dim);
    rope_apply(&t, start_pos, n_heads, head_dim, n_rot, theta);
}

void ref_softmax(float* row, size_t len) { softmax_row(row, len); }

void* ref_cache_new(size_t layers, size_t seq_max, size_t dim) { return kvcache_create(layers, seq_max, dim); }
void ref_cache_free(void* c) { kvcache_free(static_cast<KVCache*>(c)); }

// One reference decoder layer (transformer.cpp:330-755) over a [seq x d]
// input.  w_types/w_ptrs/w_rows/w_cols describe, in order, attn_q, attn_k,
// attn_v, attn_output, ffn_gate, ffn_up, ffn_down.  The ggml [out x in]
// layout is selected as the reference does for qwen* architectures
// (minxfmr.cpp:479-481).
int ref_layer_forward(const float* in, float* out, size_t seq, size_t d, void* cache, size_t layer,
                      size_t n_head, size_t n_head_kv, const int* w_types, const void* const* w_ptrs,
                      const size_t* w_rows, const size_t* w_cols, const float* attn_norm,
                      const float* ffn_norm, float theta, float eps, int neox) {
    ensure_cpu();
    backend_context().prefer_ggml_mul_mat_layout = true;
    backend_context().rope_neox = neox != 0;
    Tensor W[7];
    for (int i = 0; i < 7; ++i) bind(W[i], w_types[i], w_ptrs[i], w_rows[i], w_cols[i]);
    Tensor an, fn, x, y;
    bind(an, 0, attn_norm, 1, d);
    bind(fn, 0, ffn_norm, 1, d);
    bind(x, 0, in, seq, d);
    bind(y, 0, out, seq, d);
    std::vector<float> scores(8192, 0.0f);
    const bool ok = transformer_forward_single_layer(&x, &y, static_cast<KVCache*>(cache), layer, n_head, n_head_kv,
                                                     &W[0], &W[1], &W[2], nullptr, nullptr, nullptr, &W[3], &an, &fn,
                                                     &W[4], &W[5], &W[6], scores.data(), scores.size(), theta, 0, eps);
    return ok ? 0 : -1;
}

// The reference's load-time conversion of a GGUF tensor to F32
// (gguf_reader.cpp:759-785 for F32 / F16, :905-1008 for Q6_K, :1010-1098 for
// type 41) over `nbytes`
// of tensor data held in memory; out receives rows x cols floats.  -1 when
// the reference declines the tensor.
int ref_gguf_to_f32(int ggml_type, const void* data, size_t nbytes, uint32_t rows, uint32_t cols, float* out) {
    GGUF_File f;
    f.data.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + nbytes);
    GGUF_TensorInfo info;
    info.offset = 0;
    info.nbytes = nbytes;
    info.rows = rows;
    info.cols = cols;
    info.ggml_type = (uint32_t)ggml_type;
    Tensor* t = nullptr;
    const bool ok = ggml_type == 14   ? gguf_dequant_q6_k(f, info, t)
                    : ggml_type == 41 ? gguf_dequant_q1_0(f, info, t)
                                      : gguf_read_f32_tensor(f, info, t);
    if (!ok || !t) return -1;
    std::memcpy(out, t->data, sizeof(float) * (size_t)rows * cols);
    tensor_free(t);
    return 0;
}

}  // extern "C"
