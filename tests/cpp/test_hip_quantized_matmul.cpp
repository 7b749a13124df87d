// The checks of the reference's tests/test_cuda_quantized_matmul.cpp, run
// through the HIP backend's reference interface (hip_backend.h):
//   1. the Q4_K scale-form regression — the crafted block of
//      test_cuda_quantized_matmul.cpp:18-42 decodes to -1 at element 128 in
//      the reference CPU form — decoded on the device, bit for bit against
//      the reference's own tensor_dequant_q4_k_block;
//   2. the F32 product [[1,2,3],[4,5,6]] . [[7,8],[9,10],[11,12]]
//      (test_cuda_quantized_matmul.cpp:57-90) against cpu_matmul and the
//      known answer [[58,64],[139,154]].
// The expected side is the reference's CPU code (oracle/_ref/libmxref.so).
// Without a device the GPU checks are skipped (exit 0) as the reference's
// test does, unless --require-device is given.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <string>
#include <vector>

#include "backend/cpu/cpu_backend.h"
#include "hip_backend.h"
#include "tensor/tensor.h"

namespace {

// elementwise |got - want| <= atol or <= rtol |want| (the reference test's allclose bar)
bool allclose(const float* got, const float* want, size_t n, float rtol, float atol) {
    for (size_t i = 0; i < n; ++i) {
        const float d = std::fabs(got[i] - want[i]);
        if (d > atol && d > rtol * std::fabs(want[i])) {
            std::cerr << "    [" << i << "] got " << got[i] << ", want " << want[i] << "\n";
            return false;
        }
    }
    return true;
}

// d = dmin = 1.0; scale bytes 4 and 8 make sub-block 4 (elements 128..159)
// scale 16, min 17 in the reference form; qs byte 64 puts q = 1 at element
// 128, so y[128] = 16 * 1 - 17 = -1
std::vector<uint8_t> regression_block() {
    std::vector<uint8_t> b(TENSOR_Q4_K_BLOCK_SIZE, 0);
    const uint16_t one = 0x3c00;
    std::memcpy(b.data(), &one, 2);
    std::memcpy(b.data() + 2, &one, 2);
    b[4 + 4] = 0x40;
    b[4 + 8] = 0x10;
    b[16 + 64] = 0x01;
    return b;
}

bool q4k_regression() {
    const std::vector<uint8_t> blk = regression_block();
    std::vector<float> host(TENSOR_Q4_K_QK_K);
    tensor_dequant_q4_k_block(blk.data(), host.data());
    if (host[128] != -1.0f) {
        std::cout << "  x reference CPU decode gives " << host[128] << " at 128\n";
        return false;
    }
    Tensor* B = tensor_create_q4_k_from_bytes(1, TENSOR_Q4_K_QK_K, blk.data(), blk.size());
    Tensor* one = tensor_create_f32(1, 1);
    Tensor* row = tensor_create_f32(1, TENSOR_Q4_K_QK_K);
    Tensor* e128 = tensor_create_f32(1, TENSOR_Q4_K_QK_K);
    Tensor* y = tensor_create_f32(1, 1);
    if (!B || !one || !row || !e128 || !y) return false;
    static_cast<float*>(one->data)[0] = 1.0f;
    static_cast<float*>(e128->data)[128] = 1.0f;

    bool ok = true;
    // [1] . B[1 x 256]: the device decode of the whole block, times one
    if (!hip_backend_matmul(one, B, row)) {
        std::cout << "  x hip_backend_matmul failed: " << hip_backend_last_error_msg() << "\n";
        ok = false;
    } else if (std::memcmp(row->data, host.data(), sizeof(float) * TENSOR_Q4_K_QK_K) != 0) {
        std::cout << "  x device decode differs from tensor_dequant_q4_k_block\n";
        ok = false;
    }
    // e_128 . B^T through the quantized GEMV kernel
    if (!hip_backend_matmul_rhs_transposed(e128, B, y)) {
        std::cout << "  x hip_backend_matmul_rhs_transposed failed: " << hip_backend_last_error_msg() << "\n";
        ok = false;
    } else if (std::fabs(static_cast<float*>(y->data)[0] + 1.0f) >= 1e-5f) {
        std::cout << "  x GEMV gives " << static_cast<float*>(y->data)[0] << " for element 128\n";
        ok = false;
    }
    std::cout << (ok ? "  ✓ Q4_K dequant regression passed on the device" : "  ✗ Q4_K dequant regression failed")
              << std::endl;
    tensor_free(B);
    tensor_free(one);
    tensor_free(row);
    tensor_free(e128);
    tensor_free(y);
    return ok;
}

bool f32_matmul() {
    Tensor* A = tensor_create_f32(2, 3);
    Tensor* B = tensor_create_f32(3, 2);
    Tensor* C_cpu = tensor_create_f32(2, 2);
    Tensor* C_hip = tensor_create_f32(2, 2);
    if (!A || !B || !C_cpu || !C_hip) return false;
    const float a[6] = {1, 2, 3, 4, 5, 6}, b[6] = {7, 8, 9, 10, 11, 12}, known[4] = {58, 64, 139, 154};
    std::memcpy(A->data, a, sizeof a);
    std::memcpy(B->data, b, sizeof b);
    bool ok = cpu_matmul(A, B, C_cpu) && allclose(static_cast<float*>(C_cpu->data), known, 4, 0.f, 0.f);
    if (!ok) std::cout << "  x cpu_matmul does not give the known answer\n";
    if (!hip_backend_matmul(A, B, C_hip)) {
        std::cout << "  x hip_backend_matmul failed: " << hip_backend_last_error_msg() << "\n";
        ok = false;
    } else {
        const bool same = allclose(static_cast<float*>(C_hip->data), static_cast<float*>(C_cpu->data), 4, 1e-3f, 1e-4f) &&
                          allclose(static_cast<float*>(C_hip->data), known, 4, 0.f, 0.f);
        std::cout << (same ? "  ✓ CPU and HIP outputs match" : "  ✗ CPU and HIP outputs differ") << std::endl;
        ok = ok && same;
    }
    tensor_free(A);
    tensor_free(B);
    tensor_free(C_cpu);
    tensor_free(C_hip);
    return ok;
}

// shape and type errors return false with a message and launch nothing
bool argument_errors() {
    Tensor* A = tensor_create_f32(1, 3);
    Tensor* B = tensor_create_f32(2, 2);
    Tensor* C = tensor_create_f32(1, 2);
    const bool ok = A && B && C && !hip_backend_matmul(A, B, C) && std::strlen(hip_backend_last_error_msg()) > 0 &&
                    !hip_backend_matmul_rhs_transposed(A, B, C) && !hip_backend_matmul(nullptr, B, C);
    std::cout << (ok ? "  ✓ shape mismatches rejected" : "  ✗ a shape mismatch was accepted") << std::endl;
    tensor_free(A);
    tensor_free(B);
    tensor_free(C);
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    const bool require = argc > 1 && std::string(argv[1]) == "--require-device";
    std::cout << "[TEST] HIP quantized matmul (reference interface)" << std::endl;
    if (!hip_backend_is_available()) {
        std::cout << "HIP not available (" << hip_backend_last_error_msg() << "); skipping GPU parity check"
                  << std::endl;
        return require ? 7 : 0;
    }
    bool ok = q4k_regression();
    ok = f32_matmul() && ok;
    ok = argument_errors() && ok;
    hip_backend_release_resources();
    std::cout << "Test finished" << std::endl;
    return ok ? 0 : 1;
}
