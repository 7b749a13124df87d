// hip_backend.cpp — the reference's Tensor-based backend calls mapped onto
// the C ABI of libminxfmr_hip.so.  Only tensor/tensor.h and minxfmr_hip.h are
// included, so no HIP header reaches a reference translation unit.
//
// Checks follow the reference: the shape and type tests of
// backend_runtime.cpp:281-285 (rhs_transposed) and cpu_backend.cpp:119-128
// (matmul) are made here, before the library is called; a failure returns
// false and leaves a message, as cuda_backend.cu does through its
// last_error string.
#include "hip_backend.h"

#include <cstdint>
#include <cstdio>
#include <string>

#include "minxfmr_hip.h"

namespace {

std::string g_msg;  // hip_backend_last_error_msg(); one context per process, as in the reference

bool fail(const char* what) {
    g_msg = what;
    return false;
}

// the library's status to the reference's bool, keeping its message
bool lib_ok(int rc) {
    if (rc == MXH_OK) return true;
    g_msg = mxh_last_error();
    return false;
}

// GGUF type ids, the numbering the C ABI uses
int type_id(DataType t) {
    switch (t) {
    case DataType::F32: return MXH_F32;
    case DataType::Q4_K: return MXH_Q4_K;
    case DataType::Q5_0: return MXH_Q5_0;
    case DataType::Q8_0: return MXH_Q8_0;
    }
    return -1;
}

// device 0 is bound once; the outcome is kept, like the CUDA state singleton
// (cuda_backend.cu:34-46)
bool ready() {
    static const int rc = mxh_init(0);
    if (rc == MXH_OK) return true;
    g_msg = mxh_last_error();
    return false;
}

bool f32_matrix(const Tensor* t) { return t && t->data && t->type == DataType::F32; }

}  // namespace

bool hip_backend_is_available() { return ready(); }

void hip_backend_release_resources() { mxh_release_resources(); }

const char* hip_backend_last_error_msg() { return g_msg.c_str(); }

bool hip_backend_preload_tensor(const Tensor* t) {
    if (!t || !t->data || t->bytes == 0) return fail("preload: empty tensor");
    if (!ready()) return false;
    return lib_ok(mxh_preload(t->data, t->bytes));
}

bool hip_backend_matmul(const Tensor* A, const Tensor* B, Tensor* out) {
    if (!f32_matrix(A) || !B || !B->data || !f32_matrix(out)) return fail("matmul: A and out must be F32 tensors");
    if (type_id(B->type) < 0) return fail("matmul: unsupported B type");
    if (A->cols != B->rows) return fail("matmul: inner dimensions differ");
    if (out->rows != A->rows || out->cols != B->cols) return fail("matmul: output shape mismatch");
    if (A->rows == 0 || A->cols == 0 || B->cols == 0) return fail("matmul: empty operand");
    if (!ready()) return false;
    return lib_ok(mxh_host_matmul_q(type_id(B->type), static_cast<const float*>(A->data), (int64_t)A->rows,
                                    (int64_t)A->cols, B->data, B->bytes, (int64_t)B->cols,
                                    static_cast<float*>(out->data), MXH_FORM_REF));
}

bool hip_backend_matmul_rhs_transposed(const Tensor* A, const Tensor* B, Tensor* out) {
    if (!f32_matrix(A) || !B || !B->data || !f32_matrix(out))
        return fail("matmul_rhs_transposed: A and out must be F32 tensors");
    if (type_id(B->type) < 0) return fail("matmul_rhs_transposed: unsupported B type");
    if (A->cols != B->cols) return fail("matmul_rhs_transposed: A and B differ in columns");
    if (out->rows != A->rows || out->cols != B->rows) return fail("matmul_rhs_transposed: output shape mismatch");
    if (A->rows == 0 || A->cols == 0 || B->rows == 0) return fail("matmul_rhs_transposed: empty operand");
    if (!ready()) return false;
    return lib_ok(mxh_host_matmul_rhs_t(type_id(B->type), static_cast<const float*>(A->data), (int64_t)A->rows,
                                        (int64_t)A->cols, B->data, B->bytes, (int64_t)B->rows,
                                        static_cast<float*>(out->data), MXH_FORM_REF));
}

bool hip_backend_matvec_strided(const float* vec, const float* mat, float* out, size_t K, size_t N,
                                size_t mat_row_stride) {
    if (!ready()) return false;
    return lib_ok(mxh_host_matvec_strided(vec, mat, out, K, N, mat_row_stride));
}

bool hip_backend_vec_dot_rows(const float* vec, const float* mat_rows, float* out, size_t K, size_t Nrows,
                              size_t row_stride) {
    if (!ready()) return false;
    return lib_ok(mxh_host_vec_dot_rows(vec, mat_rows, out, K, Nrows, row_stride));
}

bool hip_backend_vec_dot_rows_ring(const float* vec, const float* ring, size_t head, size_t seq_max, size_t len,
                                   size_t K, size_t row_stride, float* out) {
    if (!ready()) return false;
    return lib_ok(mxh_host_vec_dot_rows_ring(vec, ring, head, seq_max, len, K, row_stride, out));
}

bool hip_backend_vec_mul_rows_cols(const float* vec, const float* mat_rows, float* out, size_t Nrows, size_t Ncols,
                                   size_t row_stride) {
    if (!ready()) return false;
    return lib_ok(mxh_host_vec_mul_rows_cols(vec, mat_rows, out, Nrows, Ncols, row_stride));
}
