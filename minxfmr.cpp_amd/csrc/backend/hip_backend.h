// hip_backend.h — the reference's backend operator interface, served by the
// gfx950 library (libminxfmr_hip.so, include/minxfmr_hip.h).
//
// Each function has the name, signature, argument meaning and error
// behaviour of its CUDA counterpart in the reference
// (src/backend/cuda/cuda_backend.h:5-29): `false` on a type or shape
// mismatch or a device failure, with a backend-owned message from
// hip_backend_last_error_msg().  Pointers are host pointers, `out` is
// allocated by the caller, and every call returns with its result in host
// memory.  The file is meant to sit at src/backend/hip/ in the reference
// tree, whose targets compile with src/ on the include path (as
// tensor/tensor.cpp itself includes "tensor/tensor.h").
#pragma once

#include <cstddef>

#include "tensor/tensor.h"

// cuda_backend.h:5 — binds device 0 on first use; false when no gfx950 device
// is visible.
bool hip_backend_is_available();
// cuda_backend.h:6 — frees the device weight cache and staging buffers.
void hip_backend_release_resources();
// cuda_backend.h:7 — uploads a weight once, keyed by (t->data, t->bytes).
bool hip_backend_preload_tensor(const Tensor* t);
// cuda_backend.h:22 — message of the last failure; empty when none.
const char* hip_backend_last_error_msg();

// cuda_backend.h:24 — out[m x n] = A[m x k] . B[k x n]; A, out F32; B F32,
// Q4_K, Q5_0 or Q8_0 (quantized along its rows, cpu_backend.cpp:119-200).
bool hip_backend_matmul(const Tensor* A, const Tensor* B, Tensor* out);
// cuda_backend.h:25 — out[m x n] = A[m x k] . B[n x k]^T, B F32 or quantized
// (backend_runtime.cpp:266-376).
bool hip_backend_matmul_rhs_transposed(const Tensor* A, const Tensor* B, Tensor* out);
// cuda_backend.h:26 — out[n] = sum_k vec[k] mat[k * stride + n].
bool hip_backend_matvec_strided(const float* vec, const float* mat, float* out, size_t K, size_t N,
                                size_t mat_row_stride);
// cuda_backend.h:27 — out[j] = dot(vec, mat_rows[j * stride .. + K]).
bool hip_backend_vec_dot_rows(const float* vec, const float* mat_rows, float* out, size_t K, size_t Nrows,
                              size_t row_stride);
// cuda_backend.h:28 — out[j] = dot(vec, ring[(head + j) % seq_max]), j < len.
bool hip_backend_vec_dot_rows_ring(const float* vec, const float* ring, size_t head, size_t seq_max, size_t len,
                                   size_t K, size_t row_stride, float* out);
// cuda_backend.h:29 — out[c] = sum_r vec[r] mat_rows[r * stride + c].
bool hip_backend_vec_mul_rows_cols(const float* vec, const float* mat_rows, float* out, size_t Nrows, size_t Ncols,
                                   size_t row_stride);
